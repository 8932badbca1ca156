// libpjrt_amd.so -- the PJRT plugin: GetPjrtApi over the megakernel VM runtime.
//
// jaxlib loads this library by path (pjrt_amd.initialize registers it as
// platform "mi355x") and calls GetPjrtApi once (reference plugin.cc:1083-1087).
// The table carries PJRT 0.112 (plugin.cc:997-999).  What this plugin does:
//   * one client, one device (HIP device 0), one memory of kind "device";
//   * buffers are pool-owned HIP device memory (vmrt_alloc), filled and read
//     back synchronously;
//   * Execute is asynchronous: the program is launched on the runtime's stream
//     with a status of its own (vmrt_submit), which is the Execute's
//     completion event and its outputs' ready event; its error is that
//     launch's VM status (a barrier time-out, say), never another launch's.
//     Everything runs on the one stream, so later launches and copies are
//     ordered after it and pool memory may be reused at once.  OnReady
//     callbacks of pending events run on one waiter thread per client.  (The
//     reference's events are born complete, plugin.cc:175-184.);
//   * the runtime is shared by the client, its executables and its buffers,
//     and closed when the last of them goes, so an executable or buffer that
//     outlives its client is still destroyed safely;
//   * Compile hands the StableHLO program to the Python lowering service and
//     loads the VMProgram v3 bytes it returns (plugin.cc:748-819); the service
//     runs as one child process per client, started at Client_Create, with
//     one framed request per compile (pjrt_amd/lower_service.py, --serve);
//   * Execute binds the argument buffers as the program's zero-copy inputs,
//     allocates fresh output buffers (or hands an output a donated argument's
//     memory, when the lowering found that safe) and runs the VM
//     (plugin.cc:941-988).
// Every slot jaxlib may call is populated; the ones this plugin does not
// provide return UNIMPLEMENTED naming the call (plugin.cc:95-102).  The four
// that jaxlib cannot tolerate as stubs are implemented: Error_ForEachPayload,
// Device_GetAttributes, LoadedExecutable_AddressableDeviceLogicalIds and
// LoadedExecutable_GetDeviceAssignment.
#include <fcntl.h>
#include <poll.h>
#include <signal.h>
#include <spawn.h>
#include <sys/stat.h>
#include <sys/wait.h>
#include <time.h>
#include <unistd.h>

#include <cerrno>
#include <condition_variable>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/vmrt.h"
#include "pjrt_abi.h"

extern char** environ;

// ---- objects --------------------------------------------------------------------------------
struct PJRT_Error {
  PJRT_Error_Code code;
  std::string message;
};

namespace {
struct ExecState;
class Waiter;

// The runtime, shared by the client, its executables and its buffers, and
// destroyed with the last of them (a program or buffer freed after its client
// still needs the runtime that owns its memory).
struct RtOwner {
  vmrt_runtime* rt = nullptr;
  ~RtOwner() {
    if (rt) vmrt_destroy(rt);
  }
};
}  // namespace

struct PJRT_DeviceDescription {
  int id = 0;
  std::string kind, debug, text;
  std::vector<PJRT_NamedValue> attrs;
  std::vector<std::string> attr_names;
  std::vector<int64_t> attr_ints;
};

struct PJRT_Memory {
  PJRT_Client* client = nullptr;
  PJRT_Device* device = nullptr;
};

struct PJRT_Device {
  PJRT_Client* client = nullptr;
  PJRT_DeviceDescription desc;
  PJRT_Memory* memory = nullptr;
};

namespace {

// The lowering service, one child process per client (pjrt_amd/lower_service.py --serve).
class LowerService {
 public:
  std::string python, script;
  double timeout_s = 60.0;

  ~LowerService() { stop(); }

  bool start(std::string* err) {
    if (pid_ > 0) return true;
    if (python.empty() || script.empty()) {
      *err = "no lowering service configured (create the client with the python_exe and lower_service options, "
             "or set PJRT_AMD_PYTHON and PJRT_AMD_LOWER_SERVICE)";
      return false;
    }
    int in[2], out[2];
    if (pipe2(in, O_CLOEXEC) != 0) return fail(err, "pipe");
    if (pipe2(out, O_CLOEXEC) != 0) {
      close(in[0]);
      close(in[1]);
      return fail(err, "pipe");
    }
    posix_spawn_file_actions_t fa;
    posix_spawn_file_actions_init(&fa);
    posix_spawn_file_actions_adddup2(&fa, in[0], 0);
    posix_spawn_file_actions_adddup2(&fa, out[1], 1);
    std::vector<char*> argv = {const_cast<char*>(python.c_str()), const_cast<char*>(script.c_str()),
                               const_cast<char*>("--serve"), nullptr};
    pid_t pid = -1;
    const int rc = posix_spawn(&pid, python.c_str(), &fa, nullptr, argv.data(), environ);
    posix_spawn_file_actions_destroy(&fa);
    close(in[0]);
    close(out[1]);
    if (rc != 0) {
      close(in[1]);
      close(out[0]);
      *err = "cannot start the lowering service " + python + " " + script + ": " + std::strerror(rc);
      return false;
    }
    pid_ = pid;
    to_ = in[1];
    from_ = out[0];
    return true;
  }

  void stop() {
    if (pid_ <= 0) return;
    const uint32_t end[6] = {0, 0, 0, 0, 0xFFFFFFFFu, 0xFFFFFFFFu};
    (void)!write(to_, end, sizeof end);
    close(to_);
    close(from_);
    int status = 0;
    for (int k = 0; k < 50 && waitpid(pid_, &status, WNOHANG) == 0; ++k) usleep(2000);
    if (waitpid(pid_, &status, WNOHANG) == 0) {
      kill(pid_, SIGKILL);
      waitpid(pid_, &status, 0);
    }
    pid_ = -1;
  }

  // status: the one-shot exit code (0 ok, 2 unsupported, 3 internal); payload:
  // v3 bytes or the JSON error.  false = the service itself failed.
  bool compile(const char* code, size_t n, const vmrt_device_info& dev, const std::string& costs, uint32_t* status,
               std::string* payload, std::vector<std::pair<uint32_t, uint32_t>>* aliases, std::string* err) {
    if (!start(err)) return false;
    uint32_t head[4] = {dev.n_lanes, dev.ew_ts, dev.mma_t, uint32_t(costs.size())};
    uint64_t len = n;
    std::string req(reinterpret_cast<const char*>(head), sizeof head);
    req.append(reinterpret_cast<const char*>(&len), 8);
    req.append(costs);
    req.append(code, n);
    std::string resp_head;
    if (!transfer(req, &resp_head, 16, err)) return restart_fail(err);
    uint32_t st, n_alias;
    uint64_t plen;
    std::memcpy(&st, resp_head.data(), 4);
    std::memcpy(&n_alias, resp_head.data() + 4, 4);
    std::memcpy(&plen, resp_head.data() + 8, 8);
    if (!transfer(std::string(), payload, plen, err)) return restart_fail(err);
    aliases->clear();
    if (n_alias) {
      std::string raw;
      if (n_alias > 65536 || !transfer(std::string(), &raw, uint64_t(n_alias) * 8, err)) return restart_fail(err);
      for (uint32_t k = 0; k < n_alias; ++k) {
        uint32_t io[2];
        std::memcpy(io, raw.data() + 8 * k, 8);
        aliases->emplace_back(io[0], io[1]);
      }
    }
    *status = st;
    return true;
  }

 private:
  pid_t pid_ = -1;
  int to_ = -1, from_ = -1;

  static bool fail(std::string* err, const char* what) {
    *err = std::string(what) + ": " + std::strerror(errno);
    return false;
  }

  bool restart_fail(std::string* err) {
    stop();   // a service that timed out or died is restarted on the next compile
    return false;
  }

  // SIGPIPE held back on this thread while writing to a service that may have
  // died (the write then fails with EPIPE instead of ending the process)
  struct NoSigpipe {
    sigset_t set, old;
    NoSigpipe() {
      sigemptyset(&set);
      sigaddset(&set, SIGPIPE);
      pthread_sigmask(SIG_BLOCK, &set, &old);
    }
    ~NoSigpipe() {
      timespec zero{0, 0};
      while (sigtimedwait(&set, nullptr, &zero) > 0) {
      }
      pthread_sigmask(SIG_SETMASK, &old, nullptr);
    }
  };

  // write `out` while reading `want` bytes into `in`, within the time-out
  bool transfer(const std::string& out, std::string* in, uint64_t want, std::string* err) {
    NoSigpipe guard;
    size_t sent = 0;
    in->clear();
    timespec t0;
    clock_gettime(CLOCK_MONOTONIC, &t0);
    char buf[1 << 16];
    while (sent < out.size() || in->size() < want) {
      timespec now;
      clock_gettime(CLOCK_MONOTONIC, &now);
      const double left = timeout_s - ((now.tv_sec - t0.tv_sec) + 1e-9 * (now.tv_nsec - t0.tv_nsec));
      if (left <= 0) {
        *err = "lowering service timed out";
        return false;
      }
      pollfd fds[2];
      int nf = 0;
      if (sent < out.size()) fds[nf++] = {to_, POLLOUT, 0};
      if (in->size() < want) fds[nf++] = {from_, POLLIN, 0};
      const int r = poll(fds, nf, int(left * 1000) + 1);
      if (r < 0 && errno == EINTR) continue;
      if (r < 0) return fail(err, "poll");
      for (int k = 0; k < nf; ++k) {
        if (fds[k].fd == to_ && (fds[k].revents & (POLLOUT | POLLERR | POLLHUP))) {
          const ssize_t w = write(to_, out.data() + sent, out.size() - sent);
          if (w < 0 && errno != EAGAIN && errno != EINTR) return fail(err, "write to the lowering service");
          if (w > 0) sent += size_t(w);
        }
        if (fds[k].fd == from_ && (fds[k].revents & (POLLIN | POLLERR | POLLHUP))) {
          const ssize_t r2 = read(from_, buf, std::min<uint64_t>(sizeof buf, want - in->size()));
          if (r2 == 0) {
            *err = "lowering service exited";
            return false;
          }
          if (r2 < 0 && errno != EAGAIN && errno != EINTR) return fail(err, "read from the lowering service");
          if (r2 > 0) in->append(buf, size_t(r2));
        }
      }
    }
    return true;
  }
};

PJRT_Error* make_error(PJRT_Error_Code code, std::string msg) { return new PJRT_Error{code, std::move(msg)}; }

PJRT_Error* from_vmrt(int rc, const char* err, const char* what) {
  return make_error(static_cast<PJRT_Error_Code>(rc), std::string(what) + ": " + err);
}

// VMProgram dtype enum -> PJRT element type, and element sizes
PJRT_Buffer_Type pjrt_type(uint32_t dt) {
  switch (dt) {
    case 0: return PJRT_Buffer_Type_F32;
    case 1: return PJRT_Buffer_Type_S32;
    case 2: return PJRT_Buffer_Type_U32;
    case 3: return PJRT_Buffer_Type_PRED;
    case 4: return PJRT_Buffer_Type_S64;
    case 5: return PJRT_Buffer_Type_F64;
    case 6: return PJRT_Buffer_Type_F16;
    case 7: return PJRT_Buffer_Type_BF16;
    default: return PJRT_Buffer_Type_INVALID;
  }
}

size_t type_size(PJRT_Buffer_Type t) {
  switch (t) {
    case PJRT_Buffer_Type_PRED: case PJRT_Buffer_Type_S8: case PJRT_Buffer_Type_U8: return 1;
    case PJRT_Buffer_Type_S16: case PJRT_Buffer_Type_U16: case PJRT_Buffer_Type_F16: case PJRT_Buffer_Type_BF16: return 2;
    case PJRT_Buffer_Type_S32: case PJRT_Buffer_Type_U32: case PJRT_Buffer_Type_F32: return 4;
    case PJRT_Buffer_Type_S64: case PJRT_Buffer_Type_U64: case PJRT_Buffer_Type_F64: return 8;
    default: return 0;
  }
}

}  // namespace

struct PJRT_Client {
  std::shared_ptr<RtOwner> owner;   // holds the runtime; rt is owner->rt
  vmrt_runtime* rt = nullptr;
  vmrt_device_info info{};
  PJRT_Device device;
  PJRT_Memory memory;
  PJRT_Device* device_list[1] = {&device};
  PJRT_Memory* memory_list[1] = {&memory};
  LowerService lower;
  std::string version;
  std::string costs;     // the cost table handed to the lowering (JSON), or empty
  std::mutex compile_mu;
  std::shared_ptr<Waiter> waiter;      // runs OnReady callbacks of pending events
  ~PJRT_Client();
};

struct PJRT_Buffer {
  PJRT_Client* client = nullptr;
  std::shared_ptr<RtOwner> owner;      // the runtime whose pool holds ptr
  void* ptr = nullptr;
  size_t bytes = 0;
  PJRT_Buffer_Type type = PJRT_Buffer_Type_INVALID;
  std::vector<int64_t> dims;
  bool deleted = false;
  std::shared_ptr<ExecState> ready;    // the Execute that produced it (null: ready)
  void release() {
    if (ptr && owner && owner->rt) vmrt_free(owner->rt, ptr);
    ptr = nullptr;
  }
};

namespace {
// The compiled program and its signature; shared by the loaded executable and
// the PJRT_Executable views handed out for metadata.
struct Program {
  std::shared_ptr<RtOwner> owner;      // released after the program is unloaded
  vmrt_program* prog = nullptr;
  std::string name, fingerprint;
  int64_t code_bytes = 0;
  std::vector<uint32_t> in_dt, out_dt;
  std::vector<uint64_t> in_bytes, out_bytes;
  std::vector<std::vector<int64_t>> in_dims, out_dims;
  std::vector<PJRT_Buffer_Type> out_types;
  std::vector<int64_t> out_dims_flat;
  std::vector<size_t> out_rank;
  std::vector<const char*> out_kinds;
  std::vector<size_t> out_kind_sizes;
  // donations the program can take: (input, output) pairs whose memory an
  // Execute may share when the input is donated (lowering.donation_aliases)
  std::vector<std::pair<uint32_t, uint32_t>> aliases;
  ~Program() {
    if (prog) vmrt_unload(prog);
  }
};
}  // namespace

namespace {
// Completion of one Execute: its launch (vmrt_submit), whose own status is read
// once it has completed.  Shared by the Execute's completion event and the
// ready events of its outputs.  Querying takes no runtime lock and never waits.
struct ExecState {
  vmrt_launch* launch = nullptr;
  std::shared_ptr<Program> prog;       // keeps the program (and the runtime) alive
  std::weak_ptr<Waiter> waiter;
  std::mutex mu;
  bool done = false;
  PJRT_Error_Code code = PJRT_Error_Code_OK;
  std::string message;
  ~ExecState() {
    if (launch) vmrt_launch_release(launch);
  }
  bool ready() {
    {
      std::lock_guard<std::mutex> g(mu);
      if (done) return true;
    }
    if (launch && vmrt_launch_query(launch) == VMRT_UNAVAILABLE) return false;
    wait();                         // complete: reads the launch's status without waiting
    return true;
  }
  void wait() {
    {
      std::lock_guard<std::mutex> g(mu);
      if (done) return;
    }
    char e[1024] = "";
    const int rc = launch ? vmrt_launch_wait(launch, e, sizeof e) : VMRT_OK;
    std::lock_guard<std::mutex> g(mu);
    if (done) return;
    done = true;
    if (rc != VMRT_OK) {
      code = static_cast<PJRT_Error_Code>(rc);
      message = std::string("execute: ") + e;
    }
  }
  // a new error object for the outcome (null: success); call once done
  PJRT_Error* error() {
    std::lock_guard<std::mutex> g(mu);
    return code == PJRT_Error_Code_OK ? nullptr : new PJRT_Error{code, message};
  }
};

// One thread per client that waits for pending events and runs their OnReady
// callbacks in the order they were registered; it drains its queue before the
// client goes.
class Waiter {
 public:
  Waiter() : th_([this] { run(); }) {}
  ~Waiter() {
    {
      std::lock_guard<std::mutex> g(mu_);
      stop_ = true;
    }
    cv_.notify_all();
    th_.join();
  }
  void post(std::shared_ptr<ExecState> s, PJRT_Event_OnReadyCallback cb, void* arg) {
    {
      std::lock_guard<std::mutex> g(mu_);
      q_.push_back(Item{std::move(s), cb, arg});
    }
    cv_.notify_one();
  }

 private:
  struct Item {
    std::shared_ptr<ExecState> s;
    PJRT_Event_OnReadyCallback cb;
    void* arg;
  };
  void run() {
    for (;;) {
      Item it;
      {
        std::unique_lock<std::mutex> lk(mu_);
        cv_.wait(lk, [&] { return stop_ || !q_.empty(); });
        if (q_.empty()) return;
        it = std::move(q_.front());
        q_.pop_front();
      }
      it.s->wait();
      it.cb(it.s->error(), it.arg);
    }
  }
  std::mutex mu_;
  std::condition_variable cv_;
  std::deque<Item> q_;
  bool stop_ = false;
  std::thread th_;
};
}  // namespace

PJRT_Client::~PJRT_Client() {
  waiter.reset();             // pending callbacks run first
  lower.stop();
  owner.reset();              // the runtime goes with the last executable or buffer
}

struct PJRT_Event {
  std::shared_ptr<ExecState> s;   // null: complete, no error
};

struct PJRT_Executable {
  std::shared_ptr<Program> p;
};

struct PJRT_LoadedExecutable {
  PJRT_Client* client = nullptr;
  std::shared_ptr<Program> p;
  bool deleted = false;
};

// ---- implementations ------------------------------------------------------------------------
namespace {

void Error_Destroy(PJRT_Error_Destroy_Args* a) { delete a->error; }
void Error_Message(PJRT_Error_Message_Args* a) {
  a->message = a->error->message.c_str();
  a->message_size = a->error->message.size();
}
PJRT_Error* Error_GetCode(PJRT_Error_GetCode_Args* a) {
  a->code = a->error->code;
  return nullptr;
}
PJRT_Error* Error_ForEachPayload(PJRT_Error_ForEachPayload_Args*) { return nullptr; }   // no payloads

PJRT_Error* Plugin_Initialize(PJRT_Plugin_Initialize_Args*) { return nullptr; }
PJRT_Error* Plugin_Attributes(PJRT_Plugin_Attributes_Args* a) {
  // jaxlib serializes programs at the StableHLO version a plugin advertises
  // (plugin.cc:295-305)
  static const int64_t kVersion[3] = {1, 17, 0};
  static PJRT_NamedValue attr = [] {
    PJRT_NamedValue v{};
    v.struct_size = sizeof(PJRT_NamedValue);
    v.name = "stablehlo_current_version";
    v.name_size = std::strlen(v.name);
    v.type = PJRT_NamedValue_kInt64List;
    v.int64_array_value = kVersion;
    v.value_size = 3;
    return v;
  }();
  a->attributes = &attr;
  a->num_attributes = 1;
  return nullptr;
}

PJRT_Error* Event_Destroy(PJRT_Event_Destroy_Args* a) {
  delete a->event;
  return nullptr;
}
PJRT_Error* Event_IsReady(PJRT_Event_IsReady_Args* a) {
  a->is_ready = !a->event->s || a->event->s->ready();
  return nullptr;
}
PJRT_Error* Event_Error(PJRT_Event_Error_Args* a) {
  if (!a->event->s) return nullptr;
  a->event->s->wait();            // the API expects a ready event; waiting keeps a premature call correct
  return a->event->s->error();
}
PJRT_Error* Event_Await(PJRT_Event_Await_Args* a) {
  if (!a->event->s) return nullptr;
  a->event->s->wait();
  return a->event->s->error();
}
PJRT_Error* Event_OnReady(PJRT_Event_OnReady_Args* a) {
  const std::shared_ptr<ExecState>& s = a->event->s;
  std::shared_ptr<Waiter> w = s ? s->waiter.lock() : nullptr;
  if (!s || s->ready() || !w) {
    if (s) s->wait();
    a->callback(s ? s->error() : nullptr, a->user_arg);
  } else {
    w->post(s, a->callback, a->user_arg);
  }
  return nullptr;
}

std::string option_string(const PJRT_Client_Create_Args* a, const char* key) {
  for (size_t i = 0; i < a->num_options; ++i) {
    const PJRT_NamedValue& o = a->create_options[i];
    if (o.type == PJRT_NamedValue_kString && std::string(o.name, o.name_size) == key)
      return std::string(o.string_value, o.value_size);
  }
  return {};
}

std::string fingerprint(const std::string& bytes) {
  uint64_t h = 1469598103934665603ull;   // FNV-1a, 64 bit
  for (unsigned char ch : bytes) h = (h ^ ch) * 1099511628211ull;
  char buf[17];
  std::snprintf(buf, sizeof buf, "%016llx", static_cast<unsigned long long>(h));
  return buf;
}

std::string read_file(const std::string& path) {
  std::string out;
  if (std::FILE* f = std::fopen(path.c_str(), "rb")) {
    char buf[4096];
    size_t n;
    while ((n = std::fread(buf, 1, sizeof buf, f)) > 0) out.append(buf, n);
    std::fclose(f);
  }
  return out;
}

// The cost table for the lowering (runtime.cc:2433-2517): PJRT_OCL_COST_TABLE
// (a path) when set; else measured by vmrt_calibrate once per device and
// library version and cached as
// ${PJRT_OCL_CACHE_DIR:-${XDG_CACHE_HOME:-$HOME/.cache}/pjrt_amd}/costs-<key>.json;
// PJRT_OCL_CALIBRATE=0 turns measuring off (the model's built-in constants
// then), =1 re-measures.
std::string cost_table(vmrt_runtime* rt, const vmrt_device_info& info) {
  if (const char* p = std::getenv("PJRT_OCL_COST_TABLE"); p && *p) return read_file(p);
  const char* cal = std::getenv("PJRT_OCL_CALIBRATE");
  if (cal && !std::strcmp(cal, "0")) return {};
  std::string dir;
  if (const char* d = std::getenv("PJRT_OCL_CACHE_DIR"); d && *d) dir = d;
  else if (const char* x = std::getenv("XDG_CACHE_HOME"); x && *x) dir = std::string(x) + "/pjrt_amd";
  else if (const char* h = std::getenv("HOME"); h && *h) dir = std::string(h) + "/.cache/pjrt_amd";
  const std::string key = fingerprint(std::string(info.name) + "|" + info.arch + "|" + vmrt_version() + "|" +
                                      std::to_string(info.n_lanes) + "|" + std::to_string(info.ew_ts) + "|" +
                                      std::to_string(info.mma_t));
  const std::string path = dir.empty() ? std::string() : dir + "/costs-" + key + ".json";
  if (!path.empty() && !(cal && !std::strcmp(cal, "1"))) {
    std::string cached = read_file(path);
    if (!cached.empty()) return cached;
  }
  char json[4096], e[1024];
  if (vmrt_calibrate(rt, json, sizeof json, e, sizeof e) != VMRT_OK) return {};
  if (!path.empty()) {
    for (size_t k = 1; k <= dir.size(); ++k)   // mkdir -p, one component at a time
      if (k == dir.size() || dir[k] == '/') mkdir(dir.substr(0, k).c_str(), 0755);
    if (std::FILE* f = std::fopen(path.c_str(), "wb")) {
      std::fputs(json, f);
      std::fclose(f);
    }
  }
  return json;
}

PJRT_Error* Client_Create(PJRT_Client_Create_Args* a) {
  auto c = std::make_unique<PJRT_Client>();
  c->lower.python = option_string(a, "python_exe");
  c->lower.script = option_string(a, "lower_service");
  // environment overrides, under this build's names and the reference's (plugin.cc:319-322)
  for (const char* k : {"PJRT_OCL_PYTHON", "PJRT_AMD_PYTHON"})
    if (const char* v = std::getenv(k); v && *v) c->lower.python = v;
  for (const char* k : {"PJRT_OCL_LOWER_SERVICE", "PJRT_AMD_LOWER_SERVICE"})
    if (const char* v = std::getenv(k); v && *v) c->lower.script = v;
  if (const char* v = std::getenv("PJRT_AMD_LOWER_TIMEOUT_S"); v && std::atof(v) > 0) c->lower.timeout_s = std::atof(v);
  // the service starts before the device is opened, so the child is not forked
  // from a process with an initialised GPU (when this is the first HIP user)
  std::string err;
  if (!c->lower.python.empty() && !c->lower.script.empty() && !c->lower.start(&err))
    return make_error(PJRT_Error_Code_FAILED_PRECONDITION, err);
  vmrt_options o;
  vmrt_default_options(&o);
  char e[1024];
  if (int rc = vmrt_create(&o, &c->rt, e, sizeof e)) return from_vmrt(rc, e, "device");
  c->owner = std::make_shared<RtOwner>();
  c->owner->rt = c->rt;
  vmrt_device_info_get(c->rt, &c->info);
  c->waiter = std::make_shared<Waiter>();
  c->version = vmrt_version();
  c->costs = cost_table(c->rt, c->info);
  PJRT_Device& d = c->device;
  d.client = c.get();
  d.memory = &c->memory;
  d.desc.kind = "MI355X";
  d.desc.text = "MI355X(id=0)";
  d.desc.debug = std::string("MI355X(id=0, arch=") + c->info.arch + ", compute units=" +
                 std::to_string(c->info.compute_units) + ", lanes=" + std::to_string(c->info.n_lanes) + ")";
  d.desc.attr_names = {"compute_units", "vm_lanes"};
  d.desc.attr_ints = {int64_t(c->info.compute_units), int64_t(c->info.n_lanes)};
  for (size_t i = 0; i < d.desc.attr_names.size(); ++i) {
    PJRT_NamedValue v{};
    v.struct_size = sizeof v;
    v.name = d.desc.attr_names[i].c_str();
    v.name_size = d.desc.attr_names[i].size();
    v.type = PJRT_NamedValue_kInt64;
    v.int64_value = d.desc.attr_ints[i];
    v.value_size = 1;
    d.desc.attrs.push_back(v);
  }
  c->memory.client = c.get();
  c->memory.device = &c->device;
  a->client = c.release();
  return nullptr;
}

PJRT_Error* Client_Destroy(PJRT_Client_Destroy_Args* a) {
  delete a->client;
  return nullptr;
}
PJRT_Error* Client_PlatformName(PJRT_Client_PlatformName_Args* a) {
  static const char kName[] = "mi355x";
  a->platform_name = kName;
  a->platform_name_size = sizeof kName - 1;
  return nullptr;
}
PJRT_Error* Client_ProcessIndex(PJRT_Client_ProcessIndex_Args* a) {
  a->process_index = 0;
  return nullptr;
}
PJRT_Error* Client_PlatformVersion(PJRT_Client_PlatformVersion_Args* a) {
  a->platform_version = a->client->version.c_str();
  a->platform_version_size = a->client->version.size();
  return nullptr;
}
PJRT_Error* Client_Devices(PJRT_Client_Devices_Args* a) {
  a->devices = a->client->device_list;
  a->num_devices = 1;
  return nullptr;
}
PJRT_Error* Client_AddressableDevices(PJRT_Client_AddressableDevices_Args* a) {
  a->addressable_devices = a->client->device_list;
  a->num_addressable_devices = 1;
  return nullptr;
}
PJRT_Error* Client_LookupDevice(PJRT_Client_LookupDevice_Args* a) {
  if (a->id != 0) return make_error(PJRT_Error_Code_NOT_FOUND, "no device with id " + std::to_string(a->id));
  a->device = &a->client->device;
  return nullptr;
}
PJRT_Error* Client_LookupAddressableDevice(PJRT_Client_LookupAddressableDevice_Args* a) {
  if (a->local_hardware_id != 0)
    return make_error(PJRT_Error_Code_NOT_FOUND, "no device with local id " + std::to_string(a->local_hardware_id));
  a->addressable_device = &a->client->device;
  return nullptr;
}
PJRT_Error* Client_AddressableMemories(PJRT_Client_AddressableMemories_Args* a) {
  a->addressable_memories = a->client->memory_list;
  a->num_addressable_memories = 1;
  return nullptr;
}
PJRT_Error* Client_DefaultDeviceAssignment(PJRT_Client_DefaultDeviceAssignment_Args* a) {
  if (a->num_replicas * a->num_partitions != 1)
    return make_error(PJRT_Error_Code_UNIMPLEMENTED, "one replica and one partition on one device only");
  if (a->default_assignment_size >= 1) a->default_assignment[0] = 0;
  return nullptr;
}


PJRT_Error* Client_Compile(PJRT_Client_Compile_Args* a) {
  PJRT_Client* c = a->client;
  const PJRT_Program* prog = a->program;
  const std::string format(prog->format, prog->format_size);
  if (format != "mlir")
    return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "program format '" + format + "' (expected 'mlir')");
  uint32_t status = 0;
  std::string payload, err;
  std::vector<std::pair<uint32_t, uint32_t>> aliases;
  {
    std::lock_guard<std::mutex> g(c->compile_mu);
    if (!c->lower.compile(prog->code, prog->code_size, c->info, c->costs, &status, &payload, &aliases, &err))
      return make_error(PJRT_Error_Code_INTERNAL, "lowering service: " + err);
  }
  if (status == 2) return make_error(PJRT_Error_Code_UNIMPLEMENTED, "unsupported program: " + payload);
  if (status != 0) return make_error(PJRT_Error_Code_INTERNAL, "lowering failed: " + payload);
  auto p = std::make_shared<Program>();
  p->owner = c->owner;
  char e[1024];
  if (int rc = vmrt_load(c->rt, payload.data(), payload.size(), c->info.ew_ts, c->info.mma_t, &p->prog, e, sizeof e))
    return from_vmrt(rc, e, "load");
  p->name = "jit_main";
  p->fingerprint = fingerprint(payload);
  p->code_bytes = int64_t(payload.size());
  uint32_t n_in = 0, n_out = 0, lanes = 0;
  vmrt_program_counts(p->prog, &n_in, &n_out, &lanes);
  for (int is_out = 0; is_out < 2; ++is_out) {
    for (uint32_t i = 0; i < (is_out ? n_out : n_in); ++i) {
      uint32_t dt = 0, rank = 0;
      uint64_t bytes = 0, dims[16];
      vmrt_program_io(p->prog, is_out, i, &dt, &bytes, &rank, dims);
      std::vector<int64_t> d(dims, dims + rank);
      (is_out ? p->out_dt : p->in_dt).push_back(dt);
      (is_out ? p->out_bytes : p->in_bytes).push_back(bytes);
      (is_out ? p->out_dims : p->in_dims).push_back(d);
    }
  }
  static const char kKind[] = "device";
  for (size_t i = 0; i < p->out_dt.size(); ++i) {
    p->out_types.push_back(pjrt_type(p->out_dt[i]));
    p->out_rank.push_back(p->out_dims[i].size());
    p->out_dims_flat.insert(p->out_dims_flat.end(), p->out_dims[i].begin(), p->out_dims[i].end());
    p->out_kinds.push_back(kKind);
    p->out_kind_sizes.push_back(sizeof kKind - 1);
  }
  for (const auto& io : aliases)
    if (io.first < p->in_dt.size() && io.second < p->out_dt.size() && p->in_bytes[io.first] == p->out_bytes[io.second] &&
        p->in_dt[io.first] == p->out_dt[io.second])
      p->aliases.push_back(io);
  auto* ex = new PJRT_LoadedExecutable;
  ex->client = c;
  ex->p = std::move(p);
  a->executable = ex;
  return nullptr;
}

PJRT_Error* Client_BufferFromHostBuffer(PJRT_Client_BufferFromHostBuffer_Args* a) {
  const size_t es = type_size(a->type);
  if (!es) return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "element type " + std::to_string(a->type) + " unsupported");
  size_t n = 1;
  for (size_t i = 0; i < a->num_dims; ++i) n *= size_t(a->dims[i]);
  if (a->byte_strides && a->num_byte_strides) {   // only the dense row-major layout
    int64_t want = int64_t(es);
    for (size_t i = a->num_dims; i-- > 0;) {
      if (a->dims[i] > 1 && a->byte_strides[i] != want)
        return make_error(PJRT_Error_Code_UNIMPLEMENTED, "host buffers must be dense and row-major");
      want *= a->dims[i];
    }
  }
  auto b = std::make_unique<PJRT_Buffer>();
  b->client = a->client;
  b->owner = a->client->owner;
  b->bytes = n * es;
  b->type = a->type;
  b->dims.assign(a->dims, a->dims + a->num_dims);
  char e[1024];
  if (int rc = vmrt_alloc(a->client->rt, b->bytes, &b->ptr, e, sizeof e)) return from_vmrt(rc, e, "device buffer");
  if (b->bytes)
    if (int rc = vmrt_h2d(a->client->rt, b->ptr, a->data, b->bytes, e, sizeof e)) {
      b->release();
      return from_vmrt(rc, e, "host to device");
    }
  a->done_with_host_buffer = new PJRT_Event{};   // the copy above is complete
  a->buffer = b.release();
  return nullptr;
}

// device descriptions, devices, memories
PJRT_Error* DD_Id(PJRT_DeviceDescription_Id_Args* a) {
  a->id = a->device_description->id;
  return nullptr;
}
PJRT_Error* DD_ProcessIndex(PJRT_DeviceDescription_ProcessIndex_Args* a) {
  a->process_index = 0;
  return nullptr;
}
PJRT_Error* DD_Attributes(PJRT_DeviceDescription_Attributes_Args* a) {
  a->attributes = a->device_description->attrs.data();
  a->num_attributes = a->device_description->attrs.size();
  return nullptr;
}
PJRT_Error* DD_Kind(PJRT_DeviceDescription_String_Args* a) {
  a->text = a->device_description->kind.c_str();
  a->text_size = a->device_description->kind.size();
  return nullptr;
}
PJRT_Error* DD_DebugString(PJRT_DeviceDescription_String_Args* a) {
  a->text = a->device_description->debug.c_str();
  a->text_size = a->device_description->debug.size();
  return nullptr;
}
PJRT_Error* DD_ToString(PJRT_DeviceDescription_String_Args* a) {
  a->text = a->device_description->text.c_str();
  a->text_size = a->device_description->text.size();
  return nullptr;
}
PJRT_Error* Device_GetDescription(PJRT_Device_GetDescription_Args* a) {
  a->device_description = &a->device->desc;
  return nullptr;
}
PJRT_Error* Device_IsAddressable(PJRT_Device_IsAddressable_Args* a) {
  a->is_addressable = true;
  return nullptr;
}
PJRT_Error* Device_LocalHardwareId(PJRT_Device_LocalHardwareId_Args* a) {
  a->local_hardware_id = 0;
  return nullptr;
}
PJRT_Error* Device_AddressableMemories(PJRT_Device_AddressableMemories_Args* a) {
  a->memories = a->device->client->memory_list;
  a->num_memories = 1;
  return nullptr;
}
PJRT_Error* Device_DefaultMemory(PJRT_Device_DefaultMemory_Args* a) {
  a->memory = a->device->memory;
  return nullptr;
}
PJRT_Error* Device_GetAttributes(PJRT_Device_GetAttributes_Args* a) {
  a->attributes = a->device->desc.attrs.data();
  a->num_attributes = a->device->desc.attrs.size();
  a->device_attributes = nullptr;
  a->attributes_deleter = [](PJRT_Device_Attributes*) {};
  return nullptr;
}
PJRT_Error* Memory_Id(PJRT_Memory_Id_Args* a) {
  a->id = 0;
  return nullptr;
}
PJRT_Error* Memory_Kind(PJRT_Memory_String_Args* a) {
  static const char k[] = "device";
  a->text = k;
  a->text_size = sizeof k - 1;
  return nullptr;
}
PJRT_Error* Memory_DebugString(PJRT_Memory_String_Args* a) {
  static const char k[] = "MI355X HBM (id=0, kind=device)";
  a->text = k;
  a->text_size = sizeof k - 1;
  return nullptr;
}
PJRT_Error* Memory_ToString(PJRT_Memory_String_Args* a) {
  static const char k[] = "MI355X HBM(id=0)";
  a->text = k;
  a->text_size = sizeof k - 1;
  return nullptr;
}
PJRT_Error* Memory_AddressableByDevices(PJRT_Memory_AddressableByDevices_Args* a) {
  a->devices = a->memory->client->device_list;
  a->num_devices = 1;
  return nullptr;
}
PJRT_Error* Memory_Kind_Id(PJRT_Memory_Kind_Id_Args* a) {
  a->kind_id = 0;
  return nullptr;
}

// executables
PJRT_Error* Exe_Destroy(PJRT_Executable_Destroy_Args* a) {
  delete a->executable;
  return nullptr;
}
PJRT_Error* Exe_Name(PJRT_Executable_Name_Args* a) {
  a->executable_name = a->executable->p->name.c_str();
  a->executable_name_size = a->executable->p->name.size();
  return nullptr;
}
PJRT_Error* Exe_One(PJRT_Executable_Count_Args* a) {
  a->count = 1;
  return nullptr;
}
PJRT_Error* Exe_NumOutputs(PJRT_Executable_Count_Args* a) {
  a->count = a->executable->p->out_dt.size();
  return nullptr;
}
PJRT_Error* Exe_CodeSize(PJRT_Executable_SizeOfGeneratedCodeInBytes_Args* a) {
  a->size_in_bytes = a->executable->p->code_bytes;
  return nullptr;
}
PJRT_Error* Exe_OutputElementTypes(PJRT_Executable_OutputElementTypes_Args* a) {
  a->output_types = a->executable->p->out_types.data();
  a->num_output_types = a->executable->p->out_types.size();
  return nullptr;
}
PJRT_Error* Exe_OutputDimensions(PJRT_Executable_OutputDimensions_Args* a) {
  a->num_outputs = a->executable->p->out_rank.size();
  a->dims = a->executable->p->out_dims_flat.data();
  a->dim_sizes = a->executable->p->out_rank.data();
  return nullptr;
}
PJRT_Error* Exe_OutputMemoryKinds(PJRT_Executable_OutputMemoryKinds_Args* a) {
  a->num_outputs = a->executable->p->out_kinds.size();
  a->memory_kinds = a->executable->p->out_kinds.data();
  a->memory_kind_sizes = a->executable->p->out_kind_sizes.data();
  return nullptr;
}
PJRT_Error* Exe_Fingerprint(PJRT_Executable_Fingerprint_Args* a) {
  a->executable_fingerprint = a->executable->p->fingerprint.c_str();
  a->executable_fingerprint_size = a->executable->p->fingerprint.size();
  return nullptr;
}

PJRT_Error* LE_Destroy(PJRT_LoadedExecutable_Destroy_Args* a) {
  delete a->executable;
  return nullptr;
}
PJRT_Error* LE_GetExecutable(PJRT_LoadedExecutable_GetExecutable_Args* a) {
  a->executable = new PJRT_Executable{a->loaded_executable->p};
  return nullptr;
}
PJRT_Error* LE_AddressableDevices(PJRT_LoadedExecutable_AddressableDevices_Args* a) {
  a->addressable_devices = a->executable->client->device_list;
  a->num_addressable_devices = 1;
  return nullptr;
}
PJRT_Error* LE_Delete(PJRT_LoadedExecutable_Delete_Args* a) {
  a->executable->deleted = true;
  return nullptr;
}
PJRT_Error* LE_IsDeleted(PJRT_LoadedExecutable_IsDeleted_Args* a) {
  a->is_deleted = a->executable->deleted;
  return nullptr;
}
PJRT_Error* LE_AddressableDeviceLogicalIds(PJRT_LoadedExecutable_AddressableDeviceLogicalIds_Args* a) {
  static PJRT_LogicalDeviceIds ids[1] = {{0, 0}};
  a->addressable_device_logical_ids = ids;
  a->num_addressable_device_logical_ids = 1;
  return nullptr;
}
PJRT_Error* LE_GetDeviceAssignment(PJRT_LoadedExecutable_GetDeviceAssignment_Args* a) {
  // xla.DeviceAssignmentProto {replica_count: 1, computation_count: 1,
  // computation_devices {replica_device_ids: [0]}} in protobuf wire format:
  // field 1 varint 1, field 2 varint 1, field 3 (3 bytes) = field 1 packed [0]
  static const char kProto[] = {0x08, 0x01, 0x10, 0x01, 0x1a, 0x03, 0x0a, 0x01, 0x00};
  a->serialized_bytes = kProto;
  a->serialized_bytes_size = sizeof kProto;
  a->serialized_device_assignment = nullptr;
  a->serialized_device_assignment_deleter = [](PJRT_DeviceAssignmentSerialized*) {};
  return nullptr;
}
PJRT_Error* LE_Fingerprint(PJRT_LoadedExecutable_Fingerprint_Args* a) {
  a->executable_fingerprint = a->executable->p->fingerprint.c_str();
  a->executable_fingerprint_size = a->executable->p->fingerprint.size();
  return nullptr;
}

PJRT_Error* LE_Execute(PJRT_LoadedExecutable_Execute_Args* a) {
  PJRT_LoadedExecutable* ex = a->executable;
  if (ex->deleted) return make_error(PJRT_Error_Code_FAILED_PRECONDITION, "executable was deleted");
  if (a->num_devices != 1)
    return make_error(PJRT_Error_Code_UNIMPLEMENTED, "execution on " + std::to_string(a->num_devices) +
                                                         " devices (this plugin drives one)");
  const Program& p = *ex->p;
  if (a->num_args != p.in_dt.size())
    return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "expected " + std::to_string(p.in_dt.size()) +
                                                            " arguments, got " + std::to_string(a->num_args));
  std::vector<const void*> ins(a->num_args);
  for (size_t i = 0; i < a->num_args; ++i) {
    const PJRT_Buffer* b = a->argument_lists[0][i];
    if (!b || b->deleted) return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "argument " + std::to_string(i) + " is deleted");
    if (b->type != pjrt_type(p.in_dt[i]) || b->bytes != p.in_bytes[i])
      return make_error(PJRT_Error_Code_INVALID_ARGUMENT,
                        "argument " + std::to_string(i) + ": type or size differs from the compiled signature");
    ins[i] = b->ptr;
  }
  PJRT_Client* c = ex->client;
  // donation (docs/memory.md:26-27): an output the program may alias with a
  // donated input takes that input's memory, and the input buffer is deleted.
  // Arguments are donated unless listed in non_donatable_input_indices (with no
  // options nothing is donated); a buffer passed twice is never donated.
  std::vector<int> donor(p.out_dt.size(), -1);
  if (a->options && !p.aliases.empty()) {
    const PJRT_ExecuteOptions* o = a->options;
    auto donatable = [&](uint32_t i) {
      for (size_t k = 0; k < o->num_non_donatable_input_indices; ++k)
        if (o->non_donatable_input_indices[k] == int64_t(i)) return false;
      for (size_t j = 0; j < a->num_args; ++j)
        if (j != i && a->argument_lists[0][j] == a->argument_lists[0][i]) return false;
      return true;
    };
    std::vector<bool> used(a->num_args, false);
    for (const auto& io : p.aliases)
      if (!used[io.first] && donor[io.second] < 0 && donatable(io.first)) {
        donor[io.second] = int(io.first);
        used[io.first] = true;
      }
  }
  std::vector<std::unique_ptr<PJRT_Buffer>> outs;
  std::vector<void*> optr;
  char e[1024];
  for (size_t i = 0; i < p.out_dt.size(); ++i) {
    auto b = std::make_unique<PJRT_Buffer>();
    b->client = c;
    b->owner = c->owner;
    b->bytes = p.out_bytes[i];
    b->type = p.out_types[i];
    b->dims = p.out_dims[i];
    if (donor[i] >= 0) {
      b->ptr = const_cast<void*>(ins[size_t(donor[i])]);   // taken over below, once the launch is queued
    } else if (int rc = vmrt_alloc(c->rt, b->bytes, &b->ptr, e, sizeof e)) {
      for (size_t k = 0; k < outs.size(); ++k)
        if (donor[k] < 0) outs[k]->release();
      return from_vmrt(rc, e, "output buffer");
    }
    optr.push_back(b->ptr);
    outs.push_back(std::move(b));
  }
  auto drop_outputs = [&] {
    for (size_t k = 0; k < outs.size(); ++k)
      if (donor[k] < 0) outs[k]->release();
  };
  auto st = std::make_shared<ExecState>();
  st->prog = ex->p;
  st->waiter = c->waiter;
  if (int rc = vmrt_submit(p.prog, ins.data(), ins.size(), optr.data(), optr.size(), &st->launch, e, sizeof e)) {
    drop_outputs();
    return from_vmrt(rc, e, "execute");
  }
  for (size_t k = 0; k < outs.size(); ++k)
    if (donor[k] >= 0) {                       // the donated input's memory now belongs to output k
      PJRT_Buffer* in = a->argument_lists[0][size_t(donor[k])];
      in->ptr = nullptr;
      in->deleted = true;
    }
  for (size_t i = 0; i < outs.size(); ++i) {
    outs[i]->ready = st;
    a->output_lists[0][i] = outs[i].release();
  }
  if (a->device_complete_events) a->device_complete_events[0] = new PJRT_Event{st};
  return nullptr;
}

// buffers
PJRT_Error* Buf_Destroy(PJRT_Buffer_Destroy_Args* a) {
  if (a->buffer) a->buffer->release();
  delete a->buffer;
  return nullptr;
}
PJRT_Error* Buf_ElementType(PJRT_Buffer_ElementType_Args* a) {
  a->type = a->buffer->type;
  return nullptr;
}
PJRT_Error* Buf_Dimensions(PJRT_Buffer_Dimensions_Args* a) {
  a->dims = a->buffer->dims.data();
  a->num_dims = a->buffer->dims.size();
  return nullptr;
}
PJRT_Error* Buf_DynamicDimensionIndices(PJRT_Buffer_DynamicDimensionIndices_Args* a) {
  a->dynamic_dim_indices = nullptr;
  a->num_dynamic_dims = 0;
  return nullptr;
}
PJRT_Error* Buf_OnDeviceSize(PJRT_Buffer_OnDeviceSizeInBytes_Args* a) {
  a->on_device_size_in_bytes = a->buffer->bytes;
  return nullptr;
}
PJRT_Error* Buf_Device(PJRT_Buffer_Device_Args* a) {
  a->device = &a->buffer->client->device;
  return nullptr;
}
PJRT_Error* Buf_Memory(PJRT_Buffer_Memory_Args* a) {
  a->memory = &a->buffer->client->memory;
  return nullptr;
}
PJRT_Error* Buf_Delete(PJRT_Buffer_Delete_Args* a) {
  a->buffer->release();
  a->buffer->deleted = true;
  return nullptr;
}
PJRT_Error* Buf_IsDeleted(PJRT_Buffer_IsDeleted_Args* a) {
  a->is_deleted = a->buffer->deleted;
  return nullptr;
}
PJRT_Error* Buf_ToHostBuffer(PJRT_Buffer_ToHostBuffer_Args* a) {
  PJRT_Buffer* b = a->src;
  if (b->deleted) return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "buffer is deleted");
  if (!a->dst) {                 // a size query
    a->dst_size = b->bytes;
    return nullptr;
  }
  if (a->dst_size < b->bytes)
    return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "destination of " + std::to_string(a->dst_size) +
                                                            " bytes for a " + std::to_string(b->bytes) + "-byte buffer");
  if (b->ready) {                // the producing Execute's outcome comes first
    b->ready->wait();
    if (PJRT_Error* err = b->ready->error()) return err;
  }
  char e[1024];
  if (b->bytes)
    if (int rc = vmrt_d2h(b->owner->rt, a->dst, b->ptr, b->bytes, e, sizeof e)) return from_vmrt(rc, e, "device to host");
  a->event = new PJRT_Event{};
  return nullptr;
}
PJRT_Error* Buf_IsOnCpu(PJRT_Buffer_IsOnCpu_Args* a) {
  a->is_on_cpu = false;
  return nullptr;
}
PJRT_Error* Buf_ReadyEvent(PJRT_Buffer_ReadyEvent_Args* a) {
  a->event = new PJRT_Event{a->buffer->ready};
  return nullptr;
}
PJRT_Error* Buf_UnsafePointer(PJRT_Buffer_UnsafePointer_Args* a) {
  a->buffer_pointer = reinterpret_cast<uintptr_t>(a->buffer->ptr);
  return nullptr;
}
PJRT_Error* Buf_OpaquePointer(PJRT_Buffer_OpaqueDeviceMemoryDataPointer_Args* a) {
  a->device_memory_ptr = a->buffer->ptr;
  return nullptr;
}

// the slots this plugin does not provide: UNIMPLEMENTED with the call's name
#define PJRT_AMD_STUB(name) \
  PJRT_Error* Stub_##name(void*) { return make_error(PJRT_Error_Code_UNIMPLEMENTED, #name " is not implemented by pjrt_amd"); }
PJRT_AMD_API_SLOTS(PJRT_AMD_STUB)
#undef PJRT_AMD_STUB

template <typename F>
PjrtSlot slot(F f) {
  return reinterpret_cast<PjrtSlot>(f);
}

PJRT_Api make_api() {
  PJRT_Api api{};
  api.struct_size = sizeof(PJRT_Api);
  api.pjrt_api_version = {sizeof(PJRT_Api_Version), nullptr, kPjrtApiMajor, kPjrtApiMinor};
#define PJRT_AMD_FILL(name) api.slots[kSlot_##name] = slot(&Stub_##name);
  PJRT_AMD_API_SLOTS(PJRT_AMD_FILL)
#undef PJRT_AMD_FILL
  PjrtSlot* s = api.slots;
  s[kSlot_PJRT_Error_Destroy] = slot(&Error_Destroy);
  s[kSlot_PJRT_Error_Message] = slot(&Error_Message);
  s[kSlot_PJRT_Error_GetCode] = slot(&Error_GetCode);
  s[kSlot_PJRT_Error_ForEachPayload] = slot(&Error_ForEachPayload);
  s[kSlot_PJRT_Plugin_Initialize] = slot(&Plugin_Initialize);
  s[kSlot_PJRT_Plugin_Attributes] = slot(&Plugin_Attributes);
  s[kSlot_PJRT_Event_Destroy] = slot(&Event_Destroy);
  s[kSlot_PJRT_Event_IsReady] = slot(&Event_IsReady);
  s[kSlot_PJRT_Event_Error] = slot(&Event_Error);
  s[kSlot_PJRT_Event_Await] = slot(&Event_Await);
  s[kSlot_PJRT_Event_OnReady] = slot(&Event_OnReady);
  s[kSlot_PJRT_Client_Create] = slot(&Client_Create);
  s[kSlot_PJRT_Client_Destroy] = slot(&Client_Destroy);
  s[kSlot_PJRT_Client_PlatformName] = slot(&Client_PlatformName);
  s[kSlot_PJRT_Client_ProcessIndex] = slot(&Client_ProcessIndex);
  s[kSlot_PJRT_Client_PlatformVersion] = slot(&Client_PlatformVersion);
  s[kSlot_PJRT_Client_Devices] = slot(&Client_Devices);
  s[kSlot_PJRT_Client_AddressableDevices] = slot(&Client_AddressableDevices);
  s[kSlot_PJRT_Client_LookupDevice] = slot(&Client_LookupDevice);
  s[kSlot_PJRT_Client_LookupAddressableDevice] = slot(&Client_LookupAddressableDevice);
  s[kSlot_PJRT_Client_AddressableMemories] = slot(&Client_AddressableMemories);
  s[kSlot_PJRT_Client_Compile] = slot(&Client_Compile);
  s[kSlot_PJRT_Client_DefaultDeviceAssignment] = slot(&Client_DefaultDeviceAssignment);
  s[kSlot_PJRT_Client_BufferFromHostBuffer] = slot(&Client_BufferFromHostBuffer);
  s[kSlot_PJRT_DeviceDescription_Id] = slot(&DD_Id);
  s[kSlot_PJRT_DeviceDescription_ProcessIndex] = slot(&DD_ProcessIndex);
  s[kSlot_PJRT_DeviceDescription_Attributes] = slot(&DD_Attributes);
  s[kSlot_PJRT_DeviceDescription_Kind] = slot(&DD_Kind);
  s[kSlot_PJRT_DeviceDescription_DebugString] = slot(&DD_DebugString);
  s[kSlot_PJRT_DeviceDescription_ToString] = slot(&DD_ToString);
  s[kSlot_PJRT_Device_GetDescription] = slot(&Device_GetDescription);
  s[kSlot_PJRT_Device_IsAddressable] = slot(&Device_IsAddressable);
  s[kSlot_PJRT_Device_LocalHardwareId] = slot(&Device_LocalHardwareId);
  s[kSlot_PJRT_Device_AddressableMemories] = slot(&Device_AddressableMemories);
  s[kSlot_PJRT_Device_DefaultMemory] = slot(&Device_DefaultMemory);
  s[kSlot_PJRT_Device_GetAttributes] = slot(&Device_GetAttributes);
  s[kSlot_PJRT_Memory_Id] = slot(&Memory_Id);
  s[kSlot_PJRT_Memory_Kind] = slot(&Memory_Kind);
  s[kSlot_PJRT_Memory_DebugString] = slot(&Memory_DebugString);
  s[kSlot_PJRT_Memory_ToString] = slot(&Memory_ToString);
  s[kSlot_PJRT_Memory_AddressableByDevices] = slot(&Memory_AddressableByDevices);
  s[kSlot_PJRT_Memory_Kind_Id] = slot(&Memory_Kind_Id);
  s[kSlot_PJRT_Executable_Destroy] = slot(&Exe_Destroy);
  s[kSlot_PJRT_Executable_Name] = slot(&Exe_Name);
  s[kSlot_PJRT_Executable_NumReplicas] = slot(&Exe_One);
  s[kSlot_PJRT_Executable_NumPartitions] = slot(&Exe_One);
  s[kSlot_PJRT_Executable_NumOutputs] = slot(&Exe_NumOutputs);
  s[kSlot_PJRT_Executable_SizeOfGeneratedCodeInBytes] = slot(&Exe_CodeSize);
  s[kSlot_PJRT_Executable_OutputElementTypes] = slot(&Exe_OutputElementTypes);
  s[kSlot_PJRT_Executable_OutputDimensions] = slot(&Exe_OutputDimensions);
  s[kSlot_PJRT_Executable_OutputMemoryKinds] = slot(&Exe_OutputMemoryKinds);
  s[kSlot_PJRT_Executable_Fingerprint] = slot(&Exe_Fingerprint);
  s[kSlot_PJRT_LoadedExecutable_Destroy] = slot(&LE_Destroy);
  s[kSlot_PJRT_LoadedExecutable_GetExecutable] = slot(&LE_GetExecutable);
  s[kSlot_PJRT_LoadedExecutable_AddressableDevices] = slot(&LE_AddressableDevices);
  s[kSlot_PJRT_LoadedExecutable_Delete] = slot(&LE_Delete);
  s[kSlot_PJRT_LoadedExecutable_IsDeleted] = slot(&LE_IsDeleted);
  s[kSlot_PJRT_LoadedExecutable_Execute] = slot(&LE_Execute);
  s[kSlot_PJRT_LoadedExecutable_AddressableDeviceLogicalIds] = slot(&LE_AddressableDeviceLogicalIds);
  s[kSlot_PJRT_LoadedExecutable_GetDeviceAssignment] = slot(&LE_GetDeviceAssignment);
  s[kSlot_PJRT_LoadedExecutable_Fingerprint] = slot(&LE_Fingerprint);
  s[kSlot_PJRT_Buffer_Destroy] = slot(&Buf_Destroy);
  s[kSlot_PJRT_Buffer_ElementType] = slot(&Buf_ElementType);
  s[kSlot_PJRT_Buffer_Dimensions] = slot(&Buf_Dimensions);
  s[kSlot_PJRT_Buffer_UnpaddedDimensions] = slot(&Buf_Dimensions);
  s[kSlot_PJRT_Buffer_DynamicDimensionIndices] = slot(&Buf_DynamicDimensionIndices);
  s[kSlot_PJRT_Buffer_OnDeviceSizeInBytes] = slot(&Buf_OnDeviceSize);
  s[kSlot_PJRT_Buffer_Device] = slot(&Buf_Device);
  s[kSlot_PJRT_Buffer_Memory] = slot(&Buf_Memory);
  s[kSlot_PJRT_Buffer_Delete] = slot(&Buf_Delete);
  s[kSlot_PJRT_Buffer_IsDeleted] = slot(&Buf_IsDeleted);
  s[kSlot_PJRT_Buffer_ToHostBuffer] = slot(&Buf_ToHostBuffer);
  s[kSlot_PJRT_Buffer_IsOnCpu] = slot(&Buf_IsOnCpu);
  s[kSlot_PJRT_Buffer_ReadyEvent] = slot(&Buf_ReadyEvent);
  s[kSlot_PJRT_Buffer_UnsafePointer] = slot(&Buf_UnsafePointer);
  s[kSlot_PJRT_Buffer_OpaqueDeviceMemoryDataPointer] = slot(&Buf_OpaquePointer);
  return api;
}

}  // namespace

extern "C" __attribute__((visibility("default"))) const PJRT_Api* GetPjrtApi(void) {
  static const PJRT_Api api = make_api();
  return &api;
}
