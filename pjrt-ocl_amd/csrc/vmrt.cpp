// libvmrt: host runtime of the MI355X megakernel VM.
//
// Parse -> validate -> load (arena, constants, tasks, entries, lane table, aux;
// buffer ids patched to handles) -> execute (bind caller buffers as ports, launch
// the persistent kernel, check its status word).  Mirrors the reference runtime
// (pjrt_plugin/src/runtime.{h,cc}) on HIP: OclRuntime -> vmrt_runtime,
// LoadedProgram -> vmrt_program.
//
// Every task's memory footprint is checked against the buffer table on the host
// before a program can launch, so a malformed program is an error here and never
// an out-of-bounds access on the device.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <set>
#include <string>
#include <vector>

#include "../../include/vmrt.h"
#include "launch_slots.h"
#include "vm_abi.h"

extern "C" int vm_kernel_smem_bytes();
extern "C" hipError_t vm_kernel_prepare();
extern "C" hipError_t vm_kernel_occupancy(int* blocks_per_cu);
extern "C" hipError_t vm_kernel_launch(const vm::VmArgs* args, hipStream_t stream, int cooperative);
extern "C" hipError_t vm_status_epilogue_launch(uint32_t* ctl, uint32_t* slot, uint8_t* scratch, uint64_t scratch_bytes,
                                                hipStream_t stream);

namespace {

using namespace vm;

struct Error {
  int code = VMRT_OK;
  std::string msg;
};

int set_err(char* err, size_t errlen, int code, const std::string& msg) {
  if (err && errlen) {
    std::snprintf(err, errlen, "%s", msg.c_str());
  }
  return code;
}

std::string fmt(const char* f, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, f);
  std::vsnprintf(buf, sizeof buf, f, ap);
  va_end(ap);
  return buf;
}

std::string hip_msg(hipError_t e) { return std::string(hipGetErrorName(e)) + ": " + hipGetErrorString(e); }

uint32_t dt_size(uint32_t dt) {
  switch (dt) {
    case DT_I64: case DT_F64: return 8;
    case DT_BOOL: return 1;
    case DT_F16: case DT_BF16: return 2;
    default: return 4;
  }
}

// ---- VMProgram v3 (docs/vmprogram.md; runtime.cc:90-251) --------------------------------
struct Buffer {
  uint64_t off, size;
  uint32_t dtype;
};
struct Program {
  uint64_t arena_bytes = 0;
  std::vector<Buffer> buffers;
  std::vector<uint32_t> inputs, outputs;
  std::vector<std::vector<uint64_t>> in_shapes, out_shapes;
  std::vector<int32_t> aux;
  std::vector<std::pair<uint32_t, std::vector<uint8_t>>> consts;
  uint32_t n_instrs = 0, main_len = 0;
  std::vector<Task> tasks;
  std::vector<Entry> entries;
  std::vector<LaneSpan> lanes;
  uint32_t n_flags = 0;
};

struct Reader {
  const uint8_t* p;
  size_t n, pos = 0;
  bool need(size_t k) const { return pos + k <= n; }
  template <typename T>
  T get() {
    T v;
    std::memcpy(&v, p + pos, sizeof(T));
    pos += sizeof(T);
    return v;
  }
  void align8() { pos += (8 - pos % 8) % 8; }
};

constexpr uint32_t kMagic = 0x314D5056u;

bool parse_program(const uint8_t* data, size_t len, Program* P, std::string* err) {
  Reader r{data, len};
  auto fail = [&](const std::string& m) {
    *err = "VmProgram::Parse: " + m;
    return false;
  };
  if (!r.need(48)) return fail("truncated header");
  const uint32_t magic = r.get<uint32_t>(), version = r.get<uint32_t>();
  const uint32_t n_buffers = r.get<uint32_t>(), n_instrs = r.get<uint32_t>(), n_consts = r.get<uint32_t>();
  const uint32_t main_len = r.get<uint32_t>(), n_inputs = r.get<uint32_t>(), n_outputs = r.get<uint32_t>();
  const uint32_t n_aux = r.get<uint32_t>(), hpad = r.get<uint32_t>();
  const uint64_t arena = r.get<uint64_t>();
  if (magic != kMagic) return fail(fmt("bad magic 0x%08x", magic));
  if (version != 3) return fail(fmt("unsupported version %u", version));
  if (hpad != 0) return fail("header pad nonzero");
  if (main_len > n_instrs) return fail("main_len > n_instrs");
  if (arena > (uint64_t(1) << 31)) return fail("arena exceeds the 31-bit handle space");
  P->arena_bytes = arena;
  P->n_instrs = n_instrs;
  P->main_len = main_len;
  if (!r.need(uint64_t(n_buffers) * 24)) return fail("truncated buffer table");
  for (uint32_t i = 0; i < n_buffers; ++i) {
    Buffer b;
    b.off = r.get<uint64_t>();
    b.size = r.get<uint64_t>();
    b.dtype = r.get<uint32_t>();
    const uint32_t pad = r.get<uint32_t>();
    if (b.off % 64 || b.off + b.size > arena || b.size > arena) return fail(fmt("buffer %u outside arena", i));
    if (b.dtype >= DT_COUNT) return fail(fmt("buffer %u dtype %u", i, b.dtype));
    if (pad) return fail(fmt("buffer %u pad nonzero", i));
    P->buffers.push_back(b);
  }
  auto ids = [&](uint32_t count, std::vector<uint32_t>* out, const char* what) {
    if (!r.need(uint64_t(count) * 4)) return fail(std::string("truncated ") + what + " map");
    for (uint32_t i = 0; i < count; ++i) {
      const uint32_t v = r.get<uint32_t>();
      if (v >= n_buffers) return fail(std::string("bad ") + what + " map");
      out->push_back(v);
    }
    r.align8();
    return true;
  };
  if (!ids(n_inputs, &P->inputs, "input") || !ids(n_outputs, &P->outputs, "output")) return false;
  auto shape = [&](std::vector<uint64_t>* dims) {
    if (!r.need(8)) return fail("truncated io shape");
    const uint32_t rank = r.get<uint32_t>(), pad = r.get<uint32_t>();
    if (rank > 16 || pad) return fail("bad io shape entry");
    if (!r.need(uint64_t(rank) * 8)) return fail("truncated io shape dims");
    for (uint32_t k = 0; k < rank; ++k) dims->push_back(r.get<uint64_t>());
    return true;
  };
  P->in_shapes.resize(n_inputs);
  P->out_shapes.resize(n_outputs);
  for (auto& s : P->in_shapes)
    if (!shape(&s)) return false;
  for (auto& s : P->out_shapes)
    if (!shape(&s)) return false;
  if (!r.need(uint64_t(n_aux) * 4)) return fail("truncated aux pool");
  P->aux.resize(n_aux);
  for (uint32_t i = 0; i < n_aux; ++i) P->aux[i] = r.get<int32_t>();
  r.align8();
  for (uint32_t c = 0; c < n_consts; ++c) {
    if (!r.need(8)) return fail("truncated const entry");
    const uint32_t bid = r.get<uint32_t>(), blen = r.get<uint32_t>();
    if (bid >= n_buffers || blen > P->buffers[bid].size) return fail("bad const entry");
    if (!r.need(blen)) return fail("truncated const data");
    P->consts.emplace_back(bid, std::vector<uint8_t>(data + r.pos, data + r.pos + blen));
    r.pos += blen;
    r.align8();
  }
  // Tensor instructions are the lowering's record; the device runs the schedule.
  if (!r.need(uint64_t(n_instrs) * 32)) return fail("truncated instructions");
  r.pos += uint64_t(n_instrs) * 32;
  if (r.pos == len) return fail("program has no schedule sections");
  if (!r.need(16)) return fail("truncated schedule header");
  const uint32_t n_tasks = r.get<uint32_t>(), n_entries = r.get<uint32_t>();
  P->n_flags = r.get<uint32_t>();
  const uint32_t n_lanes = r.get<uint32_t>();
  if (n_lanes < 1 || n_lanes > 4096) return fail(fmt("bad n_lanes %u", n_lanes));
  const uint64_t rest = uint64_t(n_tasks) * 48 + uint64_t(n_lanes) * 16 + uint64_t(n_entries) * 32;
  if (r.pos + rest != len) return fail("schedule section size mismatch (truncated or trailing bytes)");
  P->tasks.resize(n_tasks);
  std::memcpy(P->tasks.data(), data + r.pos, size_t(n_tasks) * 48);
  r.pos += size_t(n_tasks) * 48;
  P->lanes.resize(n_lanes);
  std::memcpy(P->lanes.data(), data + r.pos, size_t(n_lanes) * 16);
  r.pos += size_t(n_lanes) * 16;
  P->entries.resize(n_entries);
  std::memcpy(P->entries.data(), data + r.pos, size_t(n_entries) * 32);
  for (uint32_t i = 0; i < n_tasks; ++i) {
    const Task& t = P->tasks[i];
    if ((t.tile_op & 0xFF) >= TOP_COUNT) return fail(fmt("task %u: unknown tile_op %u", i, t.tile_op & 0xFF));
    if (((t.tile_op >> 8) & 0xFF) >= DT_COUNT || ((t.tile_op >> 16) & 0xFF) >= DT_COUNT)
      return fail(fmt("task %u: unknown dtype", i));
    if (t.dst >= n_buffers || t.a >= n_buffers || t.b >= n_buffers)
      return fail(fmt("task %u: buffer id out of range", i));
  }
  for (uint32_t l = 0; l < n_lanes; ++l) {
    const LaneSpan& s = P->lanes[l];
    if (uint64_t(s.off) + s.count > n_entries || s.root_len > s.count) return fail(fmt("lane %u: bad stream range", l));
  }
  return true;
}

// ---- schedule validation ----------------------------------------------------------------
// Control must be uniform across lanes (every lane reaches the same barriers and
// control entries in the same order), sub-ranges must lie inside the lane's own
// stream, nesting must fit the kernel's 8-frame stack.
struct CtlSig {
  std::vector<uint64_t> toks;
  // tile entries in walk order: (entry index in the lane's stream, segment),
  // the segment being the control-token count before the entry -- equal in
  // two lanes exactly when the entries sit between the same pair of grid
  // barriers (control is uniform)
  std::vector<std::pair<uint32_t, uint64_t>> tiles;
};

bool control_sig(const Program& P, uint32_t lane, uint32_t start, uint32_t len, int depth, CtlSig* sig,
                 std::string* err) {
  const LaneSpan& s = P.lanes[lane];
  if (depth >= 8) {
    *err = fmt("lane %u: control nesting exceeds 8 frames", lane);
    return false;
  }
  if (uint64_t(start) + len > s.count) {
    *err = fmt("lane %u: control sub-range outside the lane stream", lane);
    return false;
  }
  for (uint32_t i = start; i < start + len; ++i) {
    const Entry& e = P.entries[s.off + i];
    switch (e.task) {
      case ENT_NOP: break;
      case ENT_BARRIER: sig->toks.push_back(1); break;
      case ENT_WHILE:
        sig->toks.push_back(2);
        if (e.signal_flag >= P.buffers.size()) { *err = "while: cond buffer out of range"; return false; }
        sig->toks.push_back(e.signal_flag);
        if (!control_sig(P, lane, e.tile_lo, e.tile_hi, depth + 1, sig, err)) return false;
        sig->toks.push_back(3);
        if (!control_sig(P, lane, e.wait_flag, e.wait_count, depth + 1, sig, err)) return false;
        sig->toks.push_back(4);
        break;
      case ENT_FOR:
        sig->toks.push_back(5);
        sig->toks.push_back(e.wait_flag);
        if (e.wait_flag && !control_sig(P, lane, e.tile_lo, e.tile_hi, depth + 1, sig, err)) return false;
        sig->toks.push_back(6);
        break;
      case ENT_IF:
        sig->toks.push_back(7);
        if (e.signal_flag >= P.buffers.size()) { *err = "if: cond buffer out of range"; return false; }
        sig->toks.push_back(e.signal_flag);
        if (!control_sig(P, lane, e.tile_lo, e.tile_hi, depth + 1, sig, err)) return false;
        sig->toks.push_back(8);
        if (!control_sig(P, lane, e.wait_flag, e.wait_count, depth + 1, sig, err)) return false;
        sig->toks.push_back(9);
        break;
      default:
        if (e.task >= P.tasks.size()) {
          *err = fmt("lane %u entry %u: task index out of range", lane, i);
          return false;
        }
        sig->tiles.emplace_back(i, sig->toks.size());
        break;
    }
  }
  return true;
}

// ---- completion flags (extension of the reserved WAIT / SIGNAL entry fields) --------------
// A program declaring n_flags > 0 may let tile entries signal one flag and wait
// for a range of flags.  Checked so that every wait ends: each flag is signaled
// by exactly one tile entry; every waited flag is signaled in the same barrier
// segment; no entry both waits and signals; and in each lane's segment no entry
// signals after one that waits (signals never block, so all happen).  With
// n_flags == 0 the fields of tile entries carry no meaning (the reference leaves
// them FLAG_NONE) and the loader clears them.
constexpr uint32_t kMaxFlags = 1u << 20;

bool check_flags(const Program& P, const std::vector<CtlSig>& sigs, std::string* err) {
  if (!P.n_flags) return true;
  if (P.n_flags > kMaxFlags) {
    *err = fmt("%u completion flags (at most %u)", P.n_flags, kMaxFlags);
    return false;
  }
  std::vector<int64_t> sig_seg(P.n_flags, -1);
  for (uint32_t l = 0; l < sigs.size(); ++l)
    for (const auto& t : sigs[l].tiles) {
      const Entry& e = P.entries[P.lanes[l].off + t.first];
      if (e.signal_flag == FLAG_NONE) continue;
      if (e.signal_flag >= P.n_flags) {
        *err = fmt("lane %u entry %u: signals flag %u of %u", l, t.first, e.signal_flag, P.n_flags);
        return false;
      }
      if (sig_seg[e.signal_flag] >= 0) {
        *err = fmt("completion flag %u is signaled by more than one entry", e.signal_flag);
        return false;
      }
      sig_seg[e.signal_flag] = int64_t(t.second);
    }
  for (uint32_t l = 0; l < sigs.size(); ++l) {
    int64_t wait_seg = -1;     // segment of the last waiting entry seen in walk order
    for (const auto& t : sigs[l].tiles) {
      const Entry& e = P.entries[P.lanes[l].off + t.first];
      const bool waits = e.wait_count != 0;
      if (waits) {
        if (e.signal_flag != FLAG_NONE) {
          *err = fmt("lane %u entry %u: both waits for and signals completion flags", l, t.first);
          return false;
        }
        if (e.wait_flag == FLAG_NONE || uint64_t(e.wait_flag) + e.wait_count > P.n_flags) {
          *err = fmt("lane %u entry %u: waits for flags outside [0, %u)", l, t.first, P.n_flags);
          return false;
        }
        for (uint32_t f = e.wait_flag; f < e.wait_flag + e.wait_count; ++f)
          if (sig_seg[f] != int64_t(t.second)) {
            *err = fmt("lane %u entry %u: waits for flag %u, which no entry of the same phase signals", l, t.first,
                       f);
            return false;
          }
        wait_seg = int64_t(t.second);
      } else if (e.signal_flag != FLAG_NONE && wait_seg == int64_t(t.second)) {
        *err = fmt("lane %u entry %u: signals a completion flag after an entry of the same phase waits", l, t.first);
        return false;
      }
    }
  }
  return true;
}

// ---- per-task footprint checks -------------------------------------------------------------
struct Checker {
  const Program& P;
  uint32_t ew_ts, mma_t;
  std::string* err;
  uint32_t lds_bytes;

  bool fail(uint32_t ti, const std::string& m) {
    *err = fmt("task %u: ", ti) + m;
    return false;
  }
  uint64_t elems(uint32_t id, uint32_t dt) const { return P.buffers[id].size / dt_size(dt); }
  bool aux_ok(int64_t off, int64_t n) const { return off >= 0 && n >= 0 && uint64_t(off + n) <= P.aux.size(); }
  // affine map {rank, dims, strides, off} at aux[x]: element count and [min, max] offset
  bool affine_range(uint32_t x, uint64_t* count, int64_t* mn, int64_t* mx) const {
    if (!aux_ok(x, 1)) return false;
    const int32_t rank = P.aux[x];
    if (rank < 0 || rank > 16 || !aux_ok(x, 2 + 2 * int64_t(rank))) return false;
    uint64_t c = 1;
    int64_t lo = P.aux[x + 1 + 2 * rank], hi = lo;
    for (int e = 0; e < rank; ++e) {
      const int64_t d = P.aux[x + 1 + e], st = P.aux[x + 1 + rank + e];
      if (d < 0) return false;
      c *= uint64_t(d);
      if (d == 0) continue;
      const int64_t span = (d - 1) * st;
      if (span < 0) lo += span; else hi += span;
    }
    *count = c;
    *mn = lo;
    *mx = hi;
    return true;
  }
  // a view (aux offset + 1) read as `count` elements from a buffer of `n` elements
  bool view_ok(uint32_t view1, uint64_t count, uint64_t n) const {
    uint64_t c;
    int64_t lo, hi;
    if (!affine_range(view1 - 1, &c, &lo, &hi)) return false;
    return c == count && (count == 0 || (lo >= 0 && uint64_t(hi) < n));
  }
  uint64_t n_tiles(const Task& t) const {
    const uint32_t top = t.tile_op & 0xFF;
    auto cdiv = [](uint64_t a, uint64_t b) { return (a + b - 1) / b; };
    switch (top) {
      case TOP_EW: case TOP_GATHER: case TOP_IOTA_DIM: case TOP_SCATTER: case TOP_DYN_GATHER:
      case TOP_DYN_SCATTER: case TOP_MAP_REGION: case TOP_GATHER_INDEX:
        return std::max<uint64_t>(1, cdiv(t.p[1], ew_ts));
      case TOP_RED_STRIDED: return std::max<uint64_t>(1, cdiv(t.p[0], ew_ts));
      case TOP_MMA: {
        const uint32_t code = (t.p[3] >> 24) & 0xF;
        const uint64_t T = code == 1 ? 64 : code == 2 ? 128 : code == 3 ? 256 : mma_t;
        return cdiv(t.p[0], T) * cdiv(t.p[1], T) * std::max<uint64_t>(1, t.p[3] & 0xFFFFFF) << (t.p[3] >> 28);
      }
      case TOP_RED_PART: return t.p[1] ? std::max<uint64_t>(1, cdiv(t.p[0], t.p[1])) : 1;
      case TOP_RED_COMB: return 1;
      case TOP_RED_SEG: case TOP_SOFTMAX_SEG: case TOP_LAYERNORM_SEG:
        return std::max<uint64_t>(1, t.p[0]);
      case TOP_ARGMAX_SEG: return std::max<uint64_t>(1, uint64_t(t.p[0]) * std::max<uint32_t>(1, t.p[3]));
      case TOP_FLASH_ATTN: return std::max<uint64_t>(1, uint64_t(t.p[1]) * (cdiv(t.p[2], 256) * 256));   // rows padded to 256-row blocks
      case TOP_GEMV: return t.p[4] ? std::max<uint64_t>(1, t.p[3]) * cdiv(t.p[1], t.p[4]) : 0;
      case TOP_DECODE_ATTN: return std::max<uint64_t>(1, uint64_t(t.p[4] & 0xFFFF) * std::max<uint32_t>(1, t.p[4] >> 16));
      default: return 0;
    }
  }

  bool check(uint32_t ti) {
    const Task& t = P.tasks[ti];
    const uint32_t top = t.tile_op & 0xFF, dt = (t.tile_op >> 8) & 0xFF, adt = (t.tile_op >> 16) & 0xFF;
    const uint32_t nb = uint32_t(P.buffers.size());
    auto has = [&](uint32_t id, uint64_t n, uint32_t d) { return id < nb && elems(id, d) >= n; };
    switch (top) {
      case TOP_EW: {
        const uint32_t sub = t.p[0];
        const uint64_t n = t.p[1];
        if (sub >= SUB_COUNT) return fail(ti, fmt("unknown EW subop %u", sub));
        if (sub == SUB_LTS) return (has(t.dst, 1, dt) && has(t.a, 1, adt) && has(t.b, 1, adt)) || fail(ti, "LTS operands");
        const bool cmp = sub == SUB_CMP, isf = sub == SUB_ISFINITE;
        if (!has(t.dst, n, (cmp || isf) ? DT_BOOL : dt)) return fail(ti, "EW destination smaller than n");
        if (sub == SUB_FILL || sub == SUB_IOTA_FLAT) return true;
        if (sub == SUB_SELECT)
          return (has(t.p[3], n, DT_BOOL) && has(t.a, n, dt) && has(t.b, n, dt)) || fail(ti, "select operands");
        if (cmp) return (has(t.a, n, adt) && has(t.b, n, adt)) || fail(ti, "compare operands");
        if (sub == SUB_CONVERT || isf) return has(t.a, n, adt) || fail(ti, "operand smaller than n");
        if (sub == SUB_BITCAST) return has(t.a, n, dt) || fail(ti, "bitcast operand");
        const bool fl = dt == DT_F32 || dt == DT_F16 || dt == DT_BF16;
        const bool vw = fl && (sub <= SUB_POW || (sub >= SUB_ATAN2 && sub <= SUB_REMAINDER) ||
                               (sub >= SUB_COPY && sub <= SUB_SIGN) || (sub >= SUB_LOG1P && sub <= SUB_ROUND) ||
                               sub == SUB_GELU);
        const bool bin = sub <= SUB_POW || sub == SUB_ATAN2 || sub == SUB_REMAINDER || sub == SUB_AND ||
                         sub == SUB_OR || sub == SUB_XOR || sub == SUB_SHL || sub == SUB_SHR_L || sub == SUB_SHR_A;
        const uint32_t av = vw ? t.p[2] : 0, bv = vw ? t.p[3] : 0;
        if (av ? !view_ok(av, n, elems(t.a, dt)) : !has(t.a, n, dt)) return fail(ti, "EW operand a");
        if (bin && (bv ? !view_ok(bv, n, elems(t.b, dt)) : !has(t.b, n, dt))) return fail(ti, "EW operand b");
        return true;
      }
      case TOP_GATHER: case TOP_SCATTER: {
        uint64_t c;
        int64_t lo, hi;
        if (!affine_range(t.p[0], &c, &lo, &hi) || c != t.p[1]) return fail(ti, "gather/scatter map");
        const uint32_t src = top == TOP_GATHER ? t.a : t.dst, seq = top == TOP_GATHER ? t.dst : t.a;
        if (c && (lo < 0 || uint64_t(hi) >= elems(src, dt))) return fail(ti, "gather/scatter map out of range");
        return has(seq, c, dt) || fail(ti, "gather/scatter sequential side");
      }
      case TOP_IOTA_DIM: {
        const uint32_t x = t.p[0];
        if (!aux_ok(x, 1) || P.aux[x] < 1 || !aux_ok(x, 2 + P.aux[x])) return fail(ti, "iota descriptor");
        const int32_t rank = P.aux[x], dim = P.aux[x + 1 + rank];
        uint64_t c = 1;
        for (int e = 0; e < rank; ++e) {
          if (P.aux[x + 1 + e] <= 0) return fail(ti, "iota dims");
          c *= uint64_t(P.aux[x + 1 + e]);
        }
        if (dim < 0 || dim >= rank || c != t.p[1]) return fail(ti, "iota shape");
        return has(t.dst, c, dt) || fail(ti, "iota destination");
      }
      case TOP_DYN_GATHER: case TOP_DYN_SCATTER: {
        const uint32_t x = t.p[0];
        if (!aux_ok(x, 1)) return fail(ti, "dyn descriptor");
        const int32_t rank = P.aux[x];
        if (rank < 0 || rank > 16 || !aux_ok(x, 2 + 5 * int64_t(rank))) return fail(ti, "dyn descriptor");
        const bool is64 = P.aux[x + 1 + 5 * rank] != 0;
        uint64_t c = 1;
        int64_t mx = 0;
        for (int e = 0; e < rank; ++e) {
          const int64_t d = P.aux[x + 1 + e], st = P.aux[x + 1 + rank + e], cm = P.aux[x + 1 + 2 * rank + e];
          const uint32_t sid = uint32_t(P.aux[x + 1 + 4 * rank + e]);
          if (d < 0 || st < 0 || cm < 0 || sid >= nb || P.buffers[sid].size < (is64 ? 8u : 4u))
            return fail(ti, "dyn descriptor fields");
          c *= uint64_t(d);
          if (d) mx += (d - 1 + cm) * st;
        }
        if (c != t.p[1]) return fail(ti, "dyn slice size");
        const uint32_t big = top == TOP_DYN_GATHER ? t.a : t.dst, seq = top == TOP_DYN_GATHER ? t.dst : t.a;
        if (c && uint64_t(mx) >= elems(big, dt)) return fail(ti, "dyn slice out of range");
        return has(seq, c, dt) || fail(ti, "dyn slice sequential side");
      }
      case TOP_GATHER_INDEX: {
        const uint32_t x = t.p[0];
        if (!aux_ok(x, 6)) return fail(ti, "gather descriptor");
        const int32_t orank = P.aux[x], nidx = P.aux[x + 1], vstride = P.aux[x + 2];
        const bool is64 = P.aux[x + 3] != 0;
        const uint32_t ib = uint32_t(P.aux[x + 5]);
        if (orank < 0 || orank > 16 || nidx < 0 || nidx > 16 || ib >= nb ||
            !aux_ok(x, 6 + 3 * int64_t(orank) + 2 * int64_t(nidx)))
          return fail(ti, "gather descriptor");
        const int32_t* od = &P.aux[x + 6];
        uint64_t c = 1;
        int64_t omax = 0, smax = 0;
        for (int e = 0; e < orank; ++e) {
          const int64_t d = od[e], os = od[orank + e], ss = od[2 * orank + e];
          if (d < 0 || os < 0 || ss < 0) return fail(ti, "gather strides");
          c *= uint64_t(d);
          if (d) { omax += (d - 1) * os; smax += (d - 1) * ss; }
        }
        for (int k = 0; k < nidx; ++k) {
          const int64_t ios = od[3 * orank + k], cm = od[3 * orank + nidx + k];
          if (ios < 0 || cm < 0) return fail(ti, "gather index strides");
          omax += cm * ios;
        }
        if (nidx) smax += int64_t(nidx - 1) * vstride;
        if (vstride < 0 || c != t.p[1]) return fail(ti, "gather size");
        if (c && (uint64_t(omax) >= elems(t.a, dt) || uint64_t(smax) >= elems(ib, is64 ? DT_I64 : DT_I32)))
          return fail(ti, "gather out of range");
        return has(t.dst, c, dt) || fail(ti, "gather destination");
      }
      case TOP_RED_PART: {
        const uint64_t n = t.p[0], chunk = t.p[1];
        if (!chunk || t.p[2] > 6) return fail(ti, "reduce chunk/kind");
        return (has(t.a, n, dt) && has(t.dst, (n + chunk - 1) / chunk, dt)) || fail(ti, "reduce partial operands");
      }
      case TOP_RED_COMB:
        return (t.p[1] <= 6 && has(t.a, t.p[0], dt) && has(t.dst, 1, dt)) || fail(ti, "reduce combine operands");
      case TOP_RED_SEG: {
        const uint64_t n_out = t.p[0], seg = t.p[1];
        const uint32_t src_dt = (dt == DT_I32 || dt == DT_U32 || dt == DT_I64 || dt == DT_BOOL) && !t.p[3] ? dt : adt;
        if (t.p[2] > 6) return fail(ti, "reduce kind");
        if (!has(t.a, n_out * seg, src_dt) || !has(t.dst, n_out, dt)) return fail(ti, "segmented reduce operands");
        return !t.p[3] || has(t.b, seg, adt) || fail(ti, "GEMV vector");
      }
      case TOP_RED_STRIDED: {
        const uint64_t n_out = t.p[0], red = t.p[1], inner = t.p[2];
        if (!inner || n_out % inner || t.p[3] > 6) return fail(ti, "strided reduce shape");
        const uint32_t src_dt = (dt == DT_I32 || dt == DT_U32 || dt == DT_I64 || dt == DT_BOOL) ? dt : adt;
        return (has(t.a, n_out / inner * red * inner, src_dt) && has(t.dst, n_out, dt)) ||
               fail(ti, "strided reduce operands");
      }
      case TOP_SOFTMAX_SEG: case TOP_LAYERNORM_SEG: {
        const uint64_t n = uint64_t(t.p[0]) * t.p[1];
        if (!has(t.a, n, adt) || !has(t.dst, n, dt)) return fail(ti, "row op operands");
        if (top == TOP_LAYERNORM_SEG && (t.p[3] & LN_AFFINE) &&
            !(has(t.b, t.p[1], DT_F32) && has(t.p[4], t.p[1], DT_F32)))
          return fail(ti, "layernorm gamma/beta");
        if (top == TOP_LAYERNORM_SEG && t.p[5] && t.p[0] % t.p[5])
          return fail(ti, "layernorm row interleave must divide the row count");
        return true;
      }
      case TOP_ARGMAX_SEG: {
        const uint64_t n_out = t.p[0], seg = t.p[1];
        if (dt != DT_I32 && dt != DT_U32 && dt != DT_I64) return fail(ti, "argmax index dtype");
        if (t.p[3] > kArgmaxMaxSplits) return fail(ti, "argmax splits");
        return (has(t.a, n_out * seg, adt) && has(t.dst, n_out, dt) && has(t.b, n_out, adt)) ||
               fail(ti, "argmax operands");
      }
      case TOP_MAP_REGION: {
        const uint32_t x = t.p[0];
        const uint64_t n = t.p[1];
        if (!aux_ok(x, 3)) return fail(ti, "region descriptor");
        const int32_t n_in = P.aux[x], n_micro = P.aux[x + 2];
        if (n_in < 1 || n_in > 8 || n_micro < 0 || !aux_ok(x, 3 + n_in + 6 * int64_t(n_micro)))
          return fail(ti, "region descriptor");
        const uint32_t hs[8] = {t.a, t.b, t.p[2], t.p[3], t.p[4], t.p[5], t.p[6], t.p[7]};
        for (int k = 0; k < n_in; ++k)
          if (!has(hs[k], n, dt)) return fail(ti, "region input");
        return has(t.dst, n, dt) || fail(ti, "region destination");
      }
      case TOP_FLASH_ATTN: {
        const uint32_t x = t.p[3];
        if (!aux_ok(x, 9)) return fail(ti, "attention descriptor");
        const int64_t H = P.aux[x], T = P.aux[x + 1], C = P.aux[x + 2], hd = P.aux[x + 3];
        const uint32_t qv = P.aux[x + 6], kv = P.aux[x + 7], vv = P.aux[x + 8];
        if (H <= 0 || T <= 0 || C <= 0 || hd <= 0 || hd > 256 || uint64_t(H) != t.p[1] || uint64_t(T) != t.p[2])
          return fail(ti, "attention shape");
        if (t.p[0] >= nb) return fail(ti, "attention V buffer");
        const uint64_t nq = uint64_t(H) * T * hd, nk = uint64_t(H) * C * hd;
        if (qv ? !view_ok(qv, nq, elems(t.a, adt)) : !has(t.a, nq, adt)) return fail(ti, "attention Q");
        if (kv ? !view_ok(kv, nk, elems(t.b, adt)) : !has(t.b, nk, adt)) return fail(ti, "attention K");
        if (vv ? !view_ok(vv, nk, elems(t.p[0], adt)) : !has(t.p[0], nk, adt)) return fail(ti, "attention V");
        return has(t.dst, nq, dt) || fail(ti, "attention output");
      }
      case TOP_MMA: {
        const uint64_t M = t.p[0], N = t.p[1], K = t.p[2], G = std::max<uint32_t>(1, t.p[3] & 0xFFFFFF);
        if (adt != DT_F32 && adt != DT_BF16 && adt != DT_F16) return fail(ti, "matmul operand dtype");
        if ((t.p[3] >> 28) > kMmaMaxSplitLog2) return fail(ti, "matmul K split");
        if (dt != DT_F32 && dt != DT_BF16 && dt != DT_F16) return fail(ti, "matmul result dtype");
        if (t.p[4] ? !view_ok(t.p[4], G * M * K, elems(t.a, adt)) : !has(t.a, G * M * K, adt))
          return fail(ti, "matmul A");
        if (t.p[5] ? !view_ok(t.p[5], G * K * N, elems(t.b, adt)) : !has(t.b, G * K * N, adt))
          return fail(ti, "matmul B");
        if (!has(t.dst, G * M * N, dt)) return fail(ti, "matmul C");
        if (t.p[6]) {
          const uint32_t e = t.p[6] - 1;
          if (!aux_ok(e, 1) || P.aux[e] < 0 || !aux_ok(e, 1 + 4 * int64_t(P.aux[e]))) return fail(ti, "epilogue");
          for (int k = 0; k < P.aux[e]; ++k) {
            const int32_t kind = P.aux[e + 1 + 4 * k], src = P.aux[e + 2 + 4 * k];
            // float micro-ops of the store epilogue (mma.cl:67-96): binary, unary,
            // affine and GELU; operand 0 self, 1 residual, 2 column, 3 constant s
            const bool kind_ok = (kind >= SUB_ADD && kind <= SUB_SIGN) || (kind >= SUB_ATAN2 && kind <= SUB_ROUND) ||
                                 kind == SUB_AFFINE || kind == SUB_GELU;
            if (!kind_ok) return fail(ti, "matmul epilogue kind");
            if (src < 0 || src > 3) return fail(ti, "matmul epilogue operand source");
            if (src == 1 && !has(t.p[7], G * M * N, DT_F32)) return fail(ti, "epilogue residual");
            if (src == 2 && !has(t.p[7], N, DT_F32)) return fail(ti, "epilogue bias");
          }
        }
        return true;
      }
      case TOP_GEMV: {
        const uint64_t M = t.p[0], N = t.p[1], K = t.p[2], G = std::max<uint32_t>(1, t.p[3]), CW = t.p[4];
        if (adt != DT_F32 && adt != DT_BF16 && adt != DT_F16) return fail(ti, "gemv operand dtype");
        if (dt != DT_F32 && dt != DT_BF16 && dt != DT_F16) return fail(ti, "gemv result dtype");
        if (M < 1 || M > kGemvMaxM || N < 8 || N % 8 || K < 1 || CW < 8 || CW > 256 || (CW & (CW - 1)))
          return fail(ti, "gemv shape / strip width");
        if ((((M * K + 3) & ~uint64_t(3)) + 4096 * M) * 4 > uint64_t(lds_bytes))
          return fail(ti, "gemv x row does not fit the LDS");
        if (!has(t.a, G * M * K, adt) || !has(t.b, G * K * N, adt)) return fail(ti, "gemv operands");
        if (!has(t.dst, G * M * N, dt)) return fail(ti, "gemv result");
        if (t.p[5]) {
          const uint32_t li = t.p[5] - 1;
          if (li >= P.tasks.size()) return fail(ti, "gemv layernorm prologue task");
          const Task& L = P.tasks[li];
          if ((L.tile_op & 0xFF) != TOP_LAYERNORM_SEG || L.p[0] != M || L.p[1] != K || G != 1 ||
              ((L.tile_op >> 8) & 0xFF) != adt)
            return fail(ti, "gemv layernorm prologue shape");
        }
        if (t.p[6]) {
          const uint32_t e = t.p[6] - 1;
          if (!aux_ok(e, 1) || P.aux[e] < 0 || !aux_ok(e, 1 + 4 * int64_t(P.aux[e]))) return fail(ti, "epilogue");
          for (int k = 0; k < P.aux[e]; ++k) {
            const int32_t kind = P.aux[e + 1 + 4 * k], src = P.aux[e + 2 + 4 * k];
            if (!(kind == SUB_AFFINE || kind == SUB_GELU || kind == SUB_COPY || (kind >= 0 && kind <= SUB_DIV) ||
                  kind == SUB_MAX || kind == SUB_MIN))
              return fail(ti, "gemv epilogue kind");
            if (src < 0 || src > 3) return fail(ti, "gemv epilogue operand source");
            if (src == 1 && !has(t.p[7], G * M * N, DT_F32)) return fail(ti, "epilogue residual");
            if (src == 2 && !has(t.p[7], N, DT_F32)) return fail(ti, "epilogue bias");
          }
        }
        return true;
      }
      case TOP_DECODE_ATTN: {
        const uint64_t H = t.p[4] & 0xFFFF, S = t.p[4] >> 16, hd = t.p[5] & 0xFFFF, C = t.p[6];
        if (dt != adt || (adt != DT_F32 && adt != DT_BF16 && adt != DT_F16)) return fail(ti, "decode attention dtype");
        if (H < 1 || hd < 8 || hd > 256 || hd % 8 || C < 8 || C % 8 || S > kDecMaxSplits)
          return fail(ti, "decode attention shape");
        if ((t.p[5] >> 18) != 0) return fail(ti, "decode attention flags");
        if (((C + std::max<uint64_t>(S, 1) - 1) / std::max<uint64_t>(S, 1) + 7) / 8 * 8 > kDecSplitKeys)
          return fail(ti, "decode attention: more than 64 cache keys per split");
        if (!has(t.a, H * hd, adt) || !has(t.p[1], H * hd, adt) || !has(t.p[2], H * hd, adt))
          return fail(ti, "decode attention q / k / v");
        if (!has(t.b, H * hd * C, adt) || !has(t.p[0], H * C * hd, adt)) return fail(ti, "decode attention caches");
        if (t.p[3] >= nb || P.buffers[t.p[3]].dtype != DT_I32 || !has(t.p[3], 1, DT_I32))
          return fail(ti, "decode attention position (i32 scalar)");
        return has(t.dst, H * hd, dt) || fail(ti, "decode attention output");
      }
      default:
        return fail(ti, fmt("tile op %u is not supported by this runtime", top));
    }
  }
};

// ---- pool ------------------------------------------------------------------------------
struct Pool {
  std::mutex mu;
  std::multimap<size_t, void*> free_;
  std::map<void*, size_t> live_;
  static constexpr int kKeepPerSize = 4;

  hipError_t alloc(size_t bytes, void** p) {
    bytes = std::max<size_t>(bytes, 256);
    {
      std::lock_guard<std::mutex> g(mu);
      auto it = free_.find(bytes);
      if (it != free_.end()) {
        *p = it->second;
        free_.erase(it);
        live_[*p] = bytes;
        return hipSuccess;
      }
    }
    hipError_t e = hipMalloc(p, bytes);
    if (e == hipSuccess) {
      std::lock_guard<std::mutex> g(mu);
      live_[*p] = bytes;
    }
    return e;
  }
  bool release(void* p) {
    std::lock_guard<std::mutex> g(mu);
    auto it = live_.find(p);
    if (it == live_.end()) return false;
    const size_t bytes = it->second;
    live_.erase(it);
    if (free_.count(bytes) < size_t(kKeepPerSize)) free_.emplace(bytes, p);
    else hipFree(p);
    return true;
  }
  ~Pool() {
    for (auto& kv : free_) hipFree(kv.second);
    for (auto& kv : live_) hipFree(kv.first);
  }
};

}  // namespace

// ---- device memory of the allocation-free entry point (vmrt_run_noalloc) ----
// One array per GPU, reserved when the library's code object loads and held
// until the process ends.  Host code never uses the name `scratch` as an
// address: hipGetSymbolAddress gives each device's own copy, kept in
// g_scratch_dev at vmrt_create.
constexpr size_t kNoAllocBytes = size_t(64) << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocBytes];
constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static uint8_t* g_scratch_dev[kMaxDevices];

// Pinned host memory for the launches' status slots (the device writes them).
static void* slot_alloc(size_t bytes) {
  void* p = nullptr;
  return hipHostMalloc(&p, bytes, hipHostMallocCoherent | hipHostMallocMapped) == hipSuccess ? p : nullptr;
}
static void slot_free(void* p) { (void)hipHostFree(p); }

struct vmrt_runtime {
  int device = 0;
  hipStream_t stream = nullptr;
  vmrt_device_info info{};
  uint32_t timeout_ticks = 0;
  std::mutex mu;     // serialises execute / transfers (runtime.h:233, 301)
  Pool pool;
  std::set<vmrt_program*> programs;   // loaded and not yet unloaded (guarded by mu)
  vmrt_host::SlotPool slots{slot_alloc, slot_free};   // per-launch status (vmrt_submit)
};

// A launch submitted with vmrt_submit: the event recorded after its status
// epilogue, and the slot that epilogue writes.
struct vmrt_launch {
  vmrt_runtime* rt = nullptr;
  hipEvent_t ev = nullptr;
  uint32_t* slot = nullptr;
};

struct vmrt_program {
  vmrt_runtime* rt = nullptr;
  Program prog;
  uint32_t ew_ts = 0, mma_t = 0;
  uint8_t* arena = nullptr;
  int32_t* aux = nullptr;
  Task* tasks = nullptr;
  Entry* entries = nullptr;
  LaneSpan* lanes = nullptr;
  uint32_t* ctl = nullptr;
  uint64_t* stats = nullptr;                  // profiling counters (PJRT_AMD_PROFILE=1)
  size_t stats_words = 0;
  uint8_t* scratch = nullptr;                 // split partials + arrival counters, zeroed at load
  uint64_t scratch_bytes = 0;
  uint64_t flag_off = 0;                      // byte offset of the completion flags in the scratch
  uint32_t launch_seq = 0;                    // launches so far (completion flag values)
  uint32_t* task_scratch = nullptr;           // per task: byte offset of its scratch region
  std::vector<int> input_port, output_port;   // -1 = arena copy
  std::vector<uint32_t> in_bytes, out_bytes;
  hipStream_t last_stream = nullptr;          // the stream of the latest launch (null: none yet)
  bool launched = false;
  VmArgs args{};
};

extern "C" {

const char* vmrt_version(void) { return "vmrt 0.1 (gfx950 persistent VM, VMProgram v3)"; }

void vmrt_default_options(vmrt_options* o) {
  std::memset(o, 0, sizeof *o);
  o->cooperative = 0xFFFFFFFFu;
}

int vmrt_create(const vmrt_options* opts, vmrt_runtime** out, char* err, size_t errlen) {
  vmrt_options o;
  if (opts) o = *opts;
  else vmrt_default_options(&o);
  int ndev = 0;
  hipError_t e = hipGetDeviceCount(&ndev);
  if (e != hipSuccess || ndev == 0) return set_err(err, errlen, VMRT_NOT_FOUND, "no HIP device: " + hip_msg(e));
  if (o.device < 0 || o.device >= ndev) return set_err(err, errlen, VMRT_NOT_FOUND, fmt("device %d not present", o.device));
  if ((e = hipSetDevice(o.device)) != hipSuccess) return set_err(err, errlen, VMRT_INTERNAL, hip_msg(e));
  if (o.device < kMaxDevices) {
    std::lock_guard<std::mutex> g(g_scratch_mu);
    if (!g_scratch_dev[o.device]) {
      void* ptr = nullptr;
      if ((e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch))) != hipSuccess || !ptr)
        return set_err(err, errlen, VMRT_INTERNAL, "device address of the static scratch array: " + hip_msg(e));
      g_scratch_dev[o.device] = static_cast<uint8_t*>(ptr);
    }
  }
  hipDeviceProp_t prop;
  if ((e = hipGetDeviceProperties(&prop, o.device)) != hipSuccess) return set_err(err, errlen, VMRT_INTERNAL, hip_msg(e));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return set_err(err, errlen, VMRT_FAILED_PRECONDITION,
                   std::string("libvmrt is built for gfx950; device is ") + prop.gcnArchName);
  if ((e = vm_kernel_prepare()) != hipSuccess) return set_err(err, errlen, VMRT_INTERNAL, "kernel setup: " + hip_msg(e));
  int per_cu = 0;
  if ((e = vm_kernel_occupancy(&per_cu)) != hipSuccess || per_cu < 1)
    return set_err(err, errlen, VMRT_INTERNAL, "occupancy query: " + hip_msg(e));
  auto rt = std::make_unique<vmrt_runtime>();
  rt->device = o.device;
  if ((e = hipStreamCreateWithFlags(&rt->stream, hipStreamNonBlocking)) != hipSuccess)
    return set_err(err, errlen, VMRT_INTERNAL, "stream: " + hip_msg(e));
  vmrt_device_info& I = rt->info;
  I.compute_units = uint32_t(prop.multiProcessorCount);
  I.lanes_per_cu = uint32_t(per_cu);
  I.max_lanes = I.compute_units * I.lanes_per_cu;
  // One lane per CU by default: every tile op is written for a whole CU.
  I.max_lanes = std::min(I.max_lanes, kMaxLanes);
  I.n_lanes = o.n_lanes ? std::min(o.n_lanes, I.max_lanes) : I.compute_units;
  if (const char* s = std::getenv("PJRT_OCL_VM_LANES")) {
    const long v = std::strtol(s, nullptr, 10);
    if (v > 0) I.n_lanes = std::min<uint32_t>(uint32_t(v), I.max_lanes);
  }
  I.ew_ts = o.ew_ts ? o.ew_ts : 4096;
  I.mma_t = o.mma_t ? o.mma_t : 128;
  if (I.ew_ts % 64 || (I.mma_t != 64 && I.mma_t != 128 && I.mma_t != 256))
    return set_err(err, errlen, VMRT_INVALID_ARGUMENT, "ew_ts must be a multiple of 64, mma_t one of 64/128/256");
  // Plain launch by default: hipLaunchCooperativeKernel costs ~20 us of launch gap
  // per call on ROCm 7, while co-residency of all lanes already holds because
  // n_lanes <= CUs x resident workgroups per CU; a lane that never became resident
  // would surface as a grid-barrier timeout error, never as a hang.
  I.cooperative = o.cooperative == 0xFFFFFFFFu ? 0u : (o.cooperative ? 1u : 0u);
  if (const char* s = std::getenv("PJRT_AMD_COOPERATIVE")) I.cooperative = std::atoi(s) != 0;
  I.lds_bytes = uint32_t(vm_kernel_smem_bytes());
  std::snprintf(I.arch, sizeof I.arch, "%s", prop.gcnArchName);
  std::snprintf(I.name, sizeof I.name, "%s", prop.name);
  uint32_t tmo = o.barrier_timeout_ms ? o.barrier_timeout_ms : 2000;
  if (const char* s = std::getenv("PJRT_AMD_BARRIER_TIMEOUT_MS")) {
    const long v = std::strtol(s, nullptr, 10);
    if (v > 0) tmo = uint32_t(v);
  }
  // s_memrealtime runs at 100 MHz
  rt->timeout_ticks = uint32_t(std::min<uint64_t>(uint64_t(tmo) * 100000ull, 0xFFFFFFFFull));
  *out = rt.release();
  return VMRT_OK;
}

static void free_program_memory(vmrt_program* p);

void vmrt_destroy(vmrt_runtime* rt) {
  if (!rt) return;
  hipSetDevice(rt->device);
  // the runtime's stream, and each program's latest launch on a caller's stream
  // (which must still exist); other work on the device is not waited for
  hipStreamSynchronize(rt->stream);
  {
    // programs still loaded are unloaded with their runtime: they borrow its
    // device, stream and mutex (runtime.h:365), so none may outlive it
    std::lock_guard<std::mutex> g(rt->mu);
    for (vmrt_program* p : rt->programs)
      if (p->launched && p->last_stream != rt->stream) hipStreamSynchronize(p->last_stream);
    for (vmrt_program* p : rt->programs) {
      free_program_memory(p);
      delete p;
    }
    rt->programs.clear();
  }
  hipStreamDestroy(rt->stream);
  delete rt;
}

int vmrt_device_info_get(vmrt_runtime* rt, vmrt_device_info* out) {
  if (!rt || !out) return VMRT_INVALID_ARGUMENT;
  *out = rt->info;
  return VMRT_OK;
}

static void free_program_memory(vmrt_program* p) {
  for (void* q : {static_cast<void*>(p->arena), static_cast<void*>(p->aux), static_cast<void*>(p->tasks),
                  static_cast<void*>(p->entries), static_cast<void*>(p->lanes), static_cast<void*>(p->ctl),
                  static_cast<void*>(p->stats), static_cast<void*>(p->scratch), static_cast<void*>(p->task_scratch)})
    if (q) hipFree(q);
  p->stats = nullptr;
  p->scratch = nullptr;
  p->task_scratch = nullptr;
  p->arena = nullptr;
  p->aux = nullptr;
  p->tasks = nullptr;
  p->entries = nullptr;
  p->lanes = nullptr;
  p->ctl = nullptr;
}

void vmrt_unload(vmrt_program* p) {
  if (!p) return;
  vmrt_runtime* rt = p->rt;
  std::lock_guard<std::mutex> g(rt->mu);
  if (!rt->programs.erase(p)) return;   // not a live program of this runtime
  hipSetDevice(rt->device);
  // its latest launch, on the runtime's stream or the caller's stream it was
  // enqueued on (which must still exist), finishes before its memory goes
  if (p->launched) hipStreamSynchronize(p->last_stream);
  free_program_memory(p);
  delete p;
}

// Scratch bytes a task needs (0: none): a split decode attention keeps one
// partial (running max, sum, hd channels) per split and head, and one arrival
// counter per head; a K-split matmul one f32 partial tile per split and output
// tile, and one arrival counter per output tile.
static uint64_t task_scratch_bytes(const Task& t, uint32_t mma_t) {
  if ((t.tile_op & 0xFF) == TOP_MMA && (t.p[3] >> 28)) {
    const uint32_t code = (t.p[3] >> 24) & 0xF;
    const uint64_t T = code == 1 ? 64 : code == 2 ? 128 : code == 3 ? 256 : mma_t;
    const uint64_t tiles = ((t.p[0] + T - 1) / T) * ((t.p[1] + T - 1) / T) * std::max<uint64_t>(1, t.p[3] & 0xFFFFFF);
    return (tiles * (uint64_t(1) << (t.p[3] >> 28)) * T * T + tiles) * 4;
  }
  if ((t.tile_op & 0xFF) == TOP_ARGMAX_SEG && t.p[3] > 1) return (2ull * t.p[0] * t.p[3] + t.p[0]) * 4;
  if ((t.tile_op & 0xFF) == TOP_DECODE_ATTN && (t.p[4] >> 16) > 1) {
    const uint64_t H = t.p[4] & 0xFFFF, S = t.p[4] >> 16, hd = t.p[5] & 0xFFFF;
    return (H * S * (hd + 2) + H) * 4;
  }
  return 0;
}

// The device copy of the lane table carries, in each span's pad word, the
// task of the lane's first entry (0xFFFFFFFF when it is a control entry or the
// lane has none): the kernel then requests that entry and its task record
// together at launch instead of one after the other.
static std::vector<LaneSpan> device_lanes(const std::vector<LaneSpan>& lanes, const std::vector<Entry>& entries) {
  std::vector<LaneSpan> out = lanes;
  for (LaneSpan& s : out) {
    s.pad = 0xFFFFFFFFu;
    if (s.root_len && s.off < entries.size() && entries[s.off].task < ENT_FOR) s.pad = entries[s.off].task;
  }
  return out;
}

// Host half of a load: parse, validate, choose ports, patch buffer ids to handles
// and lay out the task scratch.  Fills lp (program, tile sizes, ports, I/O sizes,
// scratch size) and the patched tables in `pr`; touches no device memory.
struct Prepared {
  std::vector<Task> tasks;
  std::vector<int32_t> aux;
  std::vector<Entry> entries;
  std::vector<uint32_t> task_scratch;
};

static int prepare_program(vmrt_runtime* rt, vmrt_program* lp, const void* bytes, size_t len, uint32_t ew_ts,
                           uint32_t mma_t, Prepared* pr, char* err, size_t errlen) {
  lp->rt = rt;
  std::string msg;
  if (!parse_program(static_cast<const uint8_t*>(bytes), len, &lp->prog, &msg))
    return set_err(err, errlen, VMRT_INVALID_ARGUMENT, msg);
  Program& P = lp->prog;
  lp->ew_ts = ew_ts ? ew_ts : rt->info.ew_ts;
  lp->mma_t = mma_t ? mma_t : rt->info.mma_t;
  if (lp->ew_ts % 64 || (lp->mma_t != 64 && lp->mma_t != 128 && lp->mma_t != 256))
    return set_err(err, errlen, VMRT_INVALID_ARGUMENT, "ew_ts must be a multiple of 64, mma_t one of 64/128/256");
  const uint32_t n_lanes = uint32_t(P.lanes.size());
  if (n_lanes > rt->info.max_lanes)
    return set_err(err, errlen, VMRT_INVALID_ARGUMENT,
                   fmt("program scheduled for %u lanes; this device holds %u co-resident lanes", n_lanes,
                       rt->info.max_lanes));

  // control uniformity across lanes, then the completion flags
  {
    std::vector<CtlSig> sigs(n_lanes);
    for (uint32_t l = 0; l < n_lanes; ++l) {
      CtlSig& s = sigs[l];
      if (!control_sig(P, l, 0, P.lanes[l].root_len, 0, &s, &msg))
        return set_err(err, errlen, VMRT_INVALID_ARGUMENT, "LoadedProgram: " + msg);
      if (l > 0 && s.toks != sigs[0].toks)
        return set_err(err, errlen, VMRT_INVALID_ARGUMENT,
                       fmt("LoadedProgram: lane %u control flow differs from lane 0 (non-uniform barriers)", l));
    }
    if (!check_flags(P, sigs, &msg)) return set_err(err, errlen, VMRT_INVALID_ARGUMENT, "LoadedProgram: " + msg);
  }
  // task footprints and entry tile ranges
  Checker chk{P, lp->ew_ts, lp->mma_t, &msg, uint32_t(vm_kernel_smem_bytes())};
  for (uint32_t i = 0; i < P.tasks.size(); ++i)
    if (!chk.check(i)) {
      const uint32_t top = P.tasks[i].tile_op & 0xFF;
      const int code = (top == TOP_CONV || top == TOP_SCATTER_INDEX || top == TOP_RED_WINDOW) ? VMRT_UNIMPLEMENTED
                                                                                                : VMRT_INVALID_ARGUMENT;
      return set_err(err, errlen, code, "LoadedProgram: " + msg);
    }
  for (uint32_t l = 0; l < n_lanes; ++l) {
    const LaneSpan& s = P.lanes[l];
    for (uint32_t k = 0; k < s.count; ++k) {
      const Entry& e = P.entries[s.off + k];
      if (e.task >= ENT_FOR) continue;
      if (e.task >= P.tasks.size())
        return set_err(err, errlen, VMRT_INVALID_ARGUMENT, fmt("LoadedProgram: lane %u entry %u task index", l, k));
      if (e.tile_lo > e.tile_hi || e.tile_hi > chk.n_tiles(P.tasks[e.task]))
        return set_err(err, errlen, VMRT_INVALID_ARGUMENT,
                       fmt("LoadedProgram: lane %u entry %u tiles [%u,%u) outside task %u's %llu tiles", l, k,
                           e.tile_lo, e.tile_hi, e.task, (unsigned long long)chk.n_tiles(P.tasks[e.task])));
    }
  }

  // ---- ports: a buffer that is only an input or only an output, first kMaxPorts ----
  std::set<uint32_t> in_ids(P.inputs.begin(), P.inputs.end()), out_ids(P.outputs.begin(), P.outputs.end());
  std::map<uint32_t, int> port_of;
  int next_port = 0;
  auto assign = [&](uint32_t id) -> int {
    if (in_ids.count(id) && out_ids.count(id)) return -1;
    auto it = port_of.find(id);
    if (it != port_of.end()) return it->second;
    if (next_port >= kMaxPorts) return -1;
    return port_of[id] = next_port++;
  };
  for (uint32_t id : P.inputs) lp->input_port.push_back(assign(id));
  for (uint32_t id : P.outputs) lp->output_port.push_back(assign(id));
  // a constant buffer is arena-resident; a port never aliases one
  for (auto& c : P.consts)
    if (port_of.count(c.first))
      return set_err(err, errlen, VMRT_INVALID_ARGUMENT, "LoadedProgram: constant buffer is also program I/O");
  auto handle = [&](uint32_t id) -> uint32_t {
    auto it = port_of.find(id);
    if (it != port_of.end()) return PORT_BIT | uint32_t(it->second);
    return uint32_t(P.buffers[id].off);
  };

  // ---- patch tasks (runtime.cc:826-875) ----
  std::vector<Task>& tasks = pr->tasks;
  tasks = P.tasks;
  for (Task& t : tasks) {
    const uint32_t top = t.tile_op & 0xFF;
    const Task orig = t;
    t.dst = handle(orig.dst);
    t.a = handle(orig.a);
    t.b = handle(orig.b);
    if (top == TOP_EW && orig.p[0] == SUB_SELECT) t.p[3] = handle(orig.p[3]);
    if (top == TOP_FLASH_ATTN) t.p[0] = handle(orig.p[0]);
    if (top == TOP_MMA && orig.p[6]) t.p[7] = handle(orig.p[7]);
    if (top == TOP_MAP_REGION) {
      const int32_t n_in = P.aux[orig.p[0]];
      for (int k = 2; k < 8; ++k) t.p[k] = handle(k < n_in ? orig.p[k] : orig.a);
    }
    if (top == TOP_LAYERNORM_SEG && (orig.p[3] & LN_AFFINE)) t.p[4] = handle(orig.p[4]);
    if (top == TOP_GEMV && orig.p[6]) t.p[7] = handle(orig.p[7]);
    if (top == TOP_DECODE_ATTN)
      for (int k = 0; k < 4; ++k) t.p[k] = handle(orig.p[k]);
  }
  // ---- patch aux: runtime start-scalar / index-buffer locations (runtime.cc:883-924) ----
  std::vector<int32_t>& aux = pr->aux;
  aux = P.aux;
  for (const Task& t : P.tasks) {
    const uint32_t top = t.tile_op & 0xFF;
    const uint32_t x = t.p[0];
    if (top == TOP_GATHER_INDEX) {
      aux[x + 4] = int32_t(handle(uint32_t(P.aux[x + 5])));
    } else if (top == TOP_DYN_GATHER || top == TOP_DYN_SCATTER) {
      const int32_t rank = P.aux[x];
      for (int d = 0; d < rank; ++d) aux[x + 1 + 3 * rank + d] = int32_t(handle(uint32_t(P.aux[x + 1 + 4 * rank + d])));
    }
  }
  // ---- patch control entries: cond buffer -> handle, pad -> cond format ----
  std::vector<Entry>& entries = pr->entries;
  entries = P.entries;
  for (Entry& e : entries) {
    if (e.task < ENT_FOR) {        // a tile entry: no flags unless the program declares them
      if (!P.n_flags || !e.wait_count) {
        e.wait_flag = FLAG_NONE;
        e.wait_count = 0;
      }
      if (!P.n_flags) e.signal_flag = FLAG_NONE;
      continue;
    }
    if (e.task == ENT_WHILE || e.task == ENT_IF) {
      const Buffer& b = P.buffers[e.signal_flag];
      const uint32_t w = dt_size(b.dtype);
      const bool fl = b.dtype == DT_F32 || b.dtype == DT_F64 || b.dtype == DT_F16 || b.dtype == DT_BF16;
      if (b.size < w) return set_err(err, errlen, VMRT_INVALID_ARGUMENT, "LoadedProgram: empty cond buffer");
      e.signal_flag = handle(e.signal_flag);
      e.pad = w | (fl ? 0x100u : 0u);
    }
  }
  // each task that needs scratch gets its own region (tasks of one phase run at once)
  std::vector<uint32_t>& task_scratch = pr->task_scratch;
  task_scratch.assign(tasks.size(), 0);
  for (size_t i = 0; i < tasks.size(); ++i) {
    const uint64_t nb = task_scratch_bytes(tasks[i], lp->mma_t);
    if (!nb) continue;
    task_scratch[i] = uint32_t(lp->scratch_bytes);
    lp->scratch_bytes += (nb + 255) & ~uint64_t(255);
    if (lp->scratch_bytes > 0xFFFFFFFFull)
      return set_err(err, errlen, VMRT_RESOURCE_EXHAUSTED, "LoadedProgram: task scratch exceeds 4 GiB");
  }
  // completion flags: 64-bit words after the task scratch (zeroed with it)
  lp->flag_off = lp->scratch_bytes;
  lp->scratch_bytes += (uint64_t(P.n_flags) * 8 + 255) & ~uint64_t(255);
  if (lp->scratch_bytes > 0xFFFFFFFFull)
    return set_err(err, errlen, VMRT_RESOURCE_EXHAUSTED, "LoadedProgram: task scratch exceeds 4 GiB");
  for (size_t i = 0; i < P.inputs.size(); ++i) lp->in_bytes.push_back(uint32_t(P.buffers[P.inputs[i]].size));
  for (size_t i = 0; i < P.outputs.size(); ++i) lp->out_bytes.push_back(uint32_t(P.buffers[P.outputs[i]].size));

  return VMRT_OK;
}

int vmrt_load(vmrt_runtime* rt, const void* bytes, size_t len, uint32_t ew_ts, uint32_t mma_t, vmrt_program** out,
              char* err, size_t errlen) {
  if (!rt || !bytes || !out) return set_err(err, errlen, VMRT_INVALID_ARGUMENT, "null argument");
  auto lp = std::make_unique<vmrt_program>();
  Prepared pr;
  if (int rc = prepare_program(rt, lp.get(), bytes, len, ew_ts, mma_t, &pr, err, errlen)) return rc;
  const Program& P = lp->prog;
  const uint32_t n_lanes = uint32_t(P.lanes.size());
  const std::vector<Task>& tasks = pr.tasks;
  const std::vector<int32_t>& aux = pr.aux;
  const std::vector<Entry>& entries = pr.entries;
  const std::vector<uint32_t>& task_scratch = pr.task_scratch;

  // ---- device memory ----
  std::lock_guard<std::mutex> g(rt->mu);
  hipSetDevice(rt->device);
  auto up = [&](void** dst, const void* src, size_t n) -> hipError_t {
    hipError_t e = hipMalloc(dst, std::max<size_t>(n, 64));
    if (e != hipSuccess) return e;
    if (n) e = hipMemcpy(*dst, src, n, hipMemcpyHostToDevice);
    return e;
  };
  hipError_t e;
  if ((e = hipMalloc(reinterpret_cast<void**>(&lp->arena), std::max<uint64_t>(P.arena_bytes, 64) + 64)) != hipSuccess) {
    free_program_memory(lp.get());
    return set_err(err, errlen, VMRT_RESOURCE_EXHAUSTED, "arena alloc: " + hip_msg(e));
  }
  e = hipMemset(lp->arena, 0, std::max<uint64_t>(P.arena_bytes, 64) + 64);
  if (e == hipSuccess) e = up(reinterpret_cast<void**>(&lp->aux), aux.data(), aux.size() * 4);
  if (e == hipSuccess) e = up(reinterpret_cast<void**>(&lp->tasks), tasks.data(), tasks.size() * sizeof(Task));
  if (e == hipSuccess) e = up(reinterpret_cast<void**>(&lp->entries), entries.data(), entries.size() * sizeof(Entry));
  const std::vector<LaneSpan> dlanes = device_lanes(P.lanes, entries);
  if (e == hipSuccess) e = up(reinterpret_cast<void**>(&lp->lanes), dlanes.data(), dlanes.size() * sizeof(LaneSpan));
  if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&lp->ctl), BAR_WORDS * 4);
  if (e == hipSuccess) e = hipMemset(lp->ctl, 0, BAR_WORDS * 4);
  if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&lp->scratch), std::max<uint64_t>(lp->scratch_bytes, 256));
  if (e == hipSuccess) e = hipMemset(lp->scratch, 0, std::max<uint64_t>(lp->scratch_bytes, 256));
  if (e == hipSuccess)
    e = up(reinterpret_cast<void**>(&lp->task_scratch), task_scratch.data(), task_scratch.size() * 4);
  if (const char* prof = std::getenv("PJRT_AMD_PROFILE"); e == hipSuccess && prof && std::atoi(prof) != 0) {
    lp->stats_words = kStatTask + 4 * tasks.size();
    e = hipMalloc(reinterpret_cast<void**>(&lp->stats), lp->stats_words * 8);
    if (e == hipSuccess) e = hipMemset(lp->stats, 0, lp->stats_words * 8);
  }
  for (auto& c : P.consts) {
    if (e != hipSuccess) break;
    if (!c.second.empty()) e = hipMemcpy(lp->arena + P.buffers[c.first].off, c.second.data(), c.second.size(), hipMemcpyHostToDevice);
  }
  if (e != hipSuccess) {
    free_program_memory(lp.get());
    return set_err(err, errlen, VMRT_RESOURCE_EXHAUSTED, "program upload: " + hip_msg(e));
  }
  VmArgs& a = lp->args;
  a.arena = lp->arena;
  a.aux = lp->aux;
  a.tasks = lp->tasks;
  a.entries = lp->entries;
  a.lanes = lp->lanes;
  a.ctl = lp->ctl;
  a.n_lanes = n_lanes;
  a.ew_ts = lp->ew_ts;
  a.mma_t = lp->mma_t;
  a.timeout_ticks = rt->timeout_ticks;
  a.stats = lp->stats;
  a.scratch = lp->scratch;
  a.task_scratch = lp->task_scratch;
  a.flags = P.n_flags ? reinterpret_cast<uint64_t*>(lp->scratch + lp->flag_off) : nullptr;
  for (int k = 0; k < kMaxPorts; ++k) a.ports[k] = lp->arena;   // unbound ports point at the arena
  rt->programs.insert(lp.get());
  *out = lp.release();
  return VMRT_OK;
}

int vmrt_program_counts(vmrt_program* p, uint32_t* n_in, uint32_t* n_out, uint32_t* n_lanes) {
  if (!p) return VMRT_INVALID_ARGUMENT;
  if (n_in) *n_in = uint32_t(p->prog.inputs.size());
  if (n_out) *n_out = uint32_t(p->prog.outputs.size());
  if (n_lanes) *n_lanes = uint32_t(p->prog.lanes.size());
  return VMRT_OK;
}

int vmrt_program_io(vmrt_program* p, int is_output, uint32_t index, uint32_t* dtype, uint64_t* bytes, uint32_t* rank,
                    uint64_t* dims16) {
  if (!p) return VMRT_INVALID_ARGUMENT;
  const auto& ids = is_output ? p->prog.outputs : p->prog.inputs;
  const auto& shapes = is_output ? p->prog.out_shapes : p->prog.in_shapes;
  if (index >= ids.size()) return VMRT_INVALID_ARGUMENT;
  const Buffer& b = p->prog.buffers[ids[index]];
  if (dtype) *dtype = b.dtype;
  if (bytes) *bytes = b.size;
  if (rank) *rank = uint32_t(shapes[index].size());
  if (dims16)
    for (size_t k = 0; k < shapes[index].size(); ++k) dims16[k] = shapes[index][k];
  return VMRT_OK;
}

static int enqueue_locked(vmrt_program* p, const void* const* inputs, size_t n_in, void* const* outputs, size_t n_out,
                          hipStream_t s, char* err, size_t errlen) {
  const Program& P = p->prog;
  if (n_in != P.inputs.size() || n_out != P.outputs.size())
    return set_err(err, errlen, VMRT_INVALID_ARGUMENT,
                   fmt("expected %zu inputs and %zu outputs, got %zu and %zu", P.inputs.size(), P.outputs.size(), n_in,
                       n_out));
  VmArgs a = p->args;
  a.seq = ++p->launch_seq;     // a new identity for this launch's completion flag values
  hipError_t e = hipSuccess;
  for (size_t i = 0; i < n_in; ++i) {
    if (!inputs[i] && p->in_bytes[i]) return set_err(err, errlen, VMRT_INVALID_ARGUMENT, fmt("input %zu is null", i));
    if (p->input_port[i] >= 0) a.ports[p->input_port[i]] = static_cast<uint8_t*>(const_cast<void*>(inputs[i]));
    else if (p->in_bytes[i])
      e = hipMemcpyAsync(p->arena + P.buffers[P.inputs[i]].off, inputs[i], p->in_bytes[i], hipMemcpyDeviceToDevice, s);
    if (e != hipSuccess) return set_err(err, errlen, VMRT_INTERNAL, "input copy: " + hip_msg(e));
  }
  for (size_t o = 0; o < n_out; ++o) {
    if (!outputs[o] && p->out_bytes[o]) return set_err(err, errlen, VMRT_INVALID_ARGUMENT, fmt("output %zu is null", o));
    if (p->output_port[o] >= 0) a.ports[p->output_port[o]] = static_cast<uint8_t*>(outputs[o]);
  }
  e = vm_kernel_launch(&a, s, int(p->rt->info.cooperative));
  if (e != hipSuccess) return set_err(err, errlen, VMRT_INTERNAL, "VM launch: " + hip_msg(e));
  for (size_t o = 0; o < n_out; ++o) {
    if (p->output_port[o] < 0 && p->out_bytes[o]) {
      e = hipMemcpyAsync(outputs[o], p->arena + P.buffers[P.outputs[o]].off, p->out_bytes[o], hipMemcpyDeviceToDevice, s);
      if (e != hipSuccess) return set_err(err, errlen, VMRT_INTERNAL, "output copy: " + hip_msg(e));
    }
  }
  // no per-launch event: a command between back-to-back launches costs
  // microseconds of gap; status waits on the launch's stream instead
  p->last_stream = s;
  p->launched = true;
  return VMRT_OK;
}

static int check_status(vmrt_program* p, char* err, size_t errlen) {
  uint32_t st[4] = {0, 0, 0, 0};
  hipError_t e = hipMemcpy(st, p->ctl, sizeof st, hipMemcpyDeviceToHost);
  if (e != hipSuccess) return set_err(err, errlen, VMRT_INTERNAL, "status read: " + hip_msg(e));
  if (st[BAR_ERROR] == VM_OK) return VMRT_OK;
  hipMemset(p->ctl, 0, BAR_WORDS * 4);
  // an aborted launch can leave arrival counters part-way
  if (p->scratch) hipMemset(p->scratch, 0, std::max<uint64_t>(p->scratch_bytes, 256));
  return set_err(err, errlen, VMRT_INTERNAL,
                 fmt("VM aborted: %s (code %u, detail %u)", vmrt_host::vm_error_text(st[BAR_ERROR]), st[BAR_ERROR],
                     st[BAR_ERRINFO]));
}

int vmrt_enqueue(vmrt_program* p, const void* const* inputs, size_t n_in, void* const* outputs, size_t n_out,
                 void* stream, char* err, size_t errlen) {
  if (!p) return set_err(err, errlen, VMRT_INVALID_ARGUMENT, "null program");
  std::lock_guard<std::mutex> g(p->rt->mu);
  hipSetDevice(p->rt->device);
  return enqueue_locked(p, inputs, n_in, outputs, n_out, stream ? static_cast<hipStream_t>(stream) : p->rt->stream,
                        err, errlen);
}

int vmrt_execute(vmrt_program* p, const void* const* inputs, size_t n_in, void* const* outputs, size_t n_out, char* err,
                 size_t errlen) {
  if (!p) return set_err(err, errlen, VMRT_INVALID_ARGUMENT, "null program");
  std::lock_guard<std::mutex> g(p->rt->mu);
  hipSetDevice(p->rt->device);
  int rc = enqueue_locked(p, inputs, n_in, outputs, n_out, p->rt->stream, err, errlen);
  if (rc != VMRT_OK) return rc;
  hipError_t e = hipStreamSynchronize(p->rt->stream);
  if (e != hipSuccess) return set_err(err, errlen, VMRT_INTERNAL, "VM execution: " + hip_msg(e));
  return check_status(p, err, errlen);
}

int vmrt_submit(vmrt_program* p, const void* const* inputs, size_t n_in, void* const* outputs, size_t n_out,
                vmrt_launch** out, char* err, size_t errlen) {
  if (!p || !out) return set_err(err, errlen, VMRT_INVALID_ARGUMENT, "null argument");
  vmrt_runtime* rt = p->rt;
  std::lock_guard<std::mutex> g(rt->mu);
  hipSetDevice(rt->device);
  auto l = std::make_unique<vmrt_launch>();
  l->rt = rt;
  l->slot = rt->slots.take();
  if (!l->slot) return set_err(err, errlen, VMRT_RESOURCE_EXHAUSTED, "launch status slot: pinned host allocation failed");
  uint32_t* slot_dev = nullptr;
  hipError_t e = hipHostGetDevicePointer(reinterpret_cast<void**>(&slot_dev), l->slot, 0);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&l->ev, hipEventDisableTiming);
  if (e != hipSuccess) {
    rt->slots.give(l->slot);
    return set_err(err, errlen, VMRT_INTERNAL, "launch status: " + hip_msg(e));
  }
  int rc = enqueue_locked(p, inputs, n_in, outputs, n_out, rt->stream, err, errlen);
  if (rc == VMRT_OK) {
    e = vm_status_epilogue_launch(p->ctl, slot_dev, p->scratch, std::max<uint64_t>(p->scratch_bytes, 256), rt->stream);
    if (e == hipSuccess) e = hipEventRecord(l->ev, rt->stream);
    if (e != hipSuccess) rc = set_err(err, errlen, VMRT_INTERNAL, "launch status epilogue: " + hip_msg(e));
  }
  if (rc != VMRT_OK) {
    // nothing of this launch may still write the slot when it is handed out again
    hipStreamSynchronize(rt->stream);
    hipEventDestroy(l->ev);
    rt->slots.give(l->slot);
    return rc;
  }
  *out = l.release();
  return VMRT_OK;
}

int vmrt_launch_query(vmrt_launch* l) {
  if (!l) return VMRT_INVALID_ARGUMENT;
  const hipError_t e = hipEventQuery(l->ev);
  return e == hipSuccess ? VMRT_OK : e == hipErrorNotReady ? VMRT_UNAVAILABLE : VMRT_INTERNAL;
}

int vmrt_launch_wait(vmrt_launch* l, char* err, size_t errlen) {
  if (!l) return set_err(err, errlen, VMRT_INVALID_ARGUMENT, "null launch");
  const hipError_t e = hipEventSynchronize(l->ev);
  if (e != hipSuccess) return set_err(err, errlen, VMRT_INTERNAL, "VM execution: " + hip_msg(e));
  std::string msg;
  const int rc = vmrt_host::slot_status(l->slot, &msg);
  return rc ? set_err(err, errlen, rc, msg) : VMRT_OK;
}

void vmrt_launch_release(vmrt_launch* l) {
  if (!l) return;
  hipSetDevice(l->rt->device);
  hipEventSynchronize(l->ev);     // the epilogue has written the slot before it is reused
  hipEventDestroy(l->ev);
  l->rt->slots.give(l->slot);
  delete l;
}

int vmrt_run_noalloc(vmrt_runtime* rt, const void* bytes, size_t len, uint32_t ew_ts, uint32_t mma_t,
                     const void* const* inputs, size_t n_in, void* const* outputs, size_t n_out, char* err,
                     size_t errlen) {
  if (!rt || !bytes) return set_err(err, errlen, VMRT_INVALID_ARGUMENT, "null argument");
  vmrt_program lp;
  Prepared pr;
  if (int rc = prepare_program(rt, &lp, bytes, len, ew_ts, mma_t, &pr, err, errlen)) return rc;
  const Program& P = lp.prog;
  // layout in the device's array: control words, task-scratch table, task
  // scratch, aux, tasks, entries, lane table, arena (each 256-byte aligned)
  size_t off = 0;
  auto place = [&](size_t n) {
    const size_t at = off;
    off += (std::max<size_t>(n, 64) + 255) & ~size_t(255);
    return at;
  };
  const size_t o_ctl = place(BAR_WORDS * 4);
  const size_t o_tsc = place(pr.task_scratch.size() * 4);
  const size_t o_scr = place(lp.scratch_bytes);
  const size_t o_aux = place(pr.aux.size() * 4);
  const size_t o_tasks = place(pr.tasks.size() * sizeof(Task));
  const size_t o_ent = place(pr.entries.size() * sizeof(Entry));
  const size_t o_lanes = place(P.lanes.size() * sizeof(LaneSpan));
  const size_t arena_n = size_t(P.arena_bytes) + 64;
  const size_t o_arena = place(arena_n);
  if (off > kNoAllocBytes)
    return set_err(err, errlen, VMRT_RESOURCE_EXHAUSTED,
                   fmt("vmrt_run_noalloc: the program needs %zu bytes of device memory (arena %llu, tables and "
                       "scratch); the allocation-free entry point holds at most %zu",
                       off, (unsigned long long)P.arena_bytes, kNoAllocBytes));
  std::lock_guard<std::mutex> g(rt->mu);
  hipSetDevice(rt->device);
  uint8_t* base = rt->device < kMaxDevices ? g_scratch_dev[rt->device] : nullptr;
  if (!base) return set_err(err, errlen, VMRT_FAILED_PRECONDITION, "no static scratch array on this device");
  hipStream_t s = rt->stream;
  // the array keeps the previous call's contents: clear what must start at zero
  // (barrier words, split counters and partials, the arena as vmrt_load leaves it)
  hipError_t e = hipMemsetAsync(base + o_ctl, 0, BAR_WORDS * 4, s);
  if (e == hipSuccess) e = hipMemsetAsync(base + o_scr, 0, std::max<uint64_t>(lp.scratch_bytes, 64), s);
  if (e == hipSuccess) e = hipMemsetAsync(base + o_arena, 0, arena_n, s);
  auto up = [&](size_t at, const void* src, size_t n) {
    if (e == hipSuccess && n) e = hipMemcpyAsync(base + at, src, n, hipMemcpyHostToDevice, s);
  };
  up(o_tsc, pr.task_scratch.data(), pr.task_scratch.size() * 4);
  up(o_aux, pr.aux.data(), pr.aux.size() * 4);
  up(o_tasks, pr.tasks.data(), pr.tasks.size() * sizeof(Task));
  up(o_ent, pr.entries.data(), pr.entries.size() * sizeof(Entry));
  const std::vector<LaneSpan> dlanes = device_lanes(P.lanes, pr.entries);
  up(o_lanes, dlanes.data(), dlanes.size() * sizeof(LaneSpan));
  for (auto& c : P.consts) up(o_arena + P.buffers[c.first].off, c.second.data(), c.second.size());
  if (e != hipSuccess) return set_err(err, errlen, VMRT_INTERNAL, "vmrt_run_noalloc upload: " + hip_msg(e));
  lp.arena = base + o_arena;
  lp.ctl = reinterpret_cast<uint32_t*>(base + o_ctl);
  lp.scratch = base + o_scr;
  VmArgs& a = lp.args;
  a.arena = lp.arena;
  a.aux = reinterpret_cast<const int32_t*>(base + o_aux);
  a.tasks = reinterpret_cast<const Task*>(base + o_tasks);
  a.entries = reinterpret_cast<const Entry*>(base + o_ent);
  a.lanes = reinterpret_cast<const LaneSpan*>(base + o_lanes);
  a.ctl = lp.ctl;
  a.n_lanes = uint32_t(P.lanes.size());
  a.ew_ts = lp.ew_ts;
  a.mma_t = lp.mma_t;
  a.timeout_ticks = rt->timeout_ticks;
  a.stats = nullptr;
  a.scratch = lp.scratch;
  a.task_scratch = reinterpret_cast<const uint32_t*>(base + o_tsc);
  a.flags = P.n_flags ? reinterpret_cast<uint64_t*>(lp.scratch + lp.flag_off) : nullptr;
  for (int k = 0; k < kMaxPorts; ++k) a.ports[k] = lp.arena;
  int rc = enqueue_locked(&lp, inputs, n_in, outputs, n_out, s, err, errlen);
  // the host tables above stay alive until the copies and the launch are done
  e = hipStreamSynchronize(s);
  if (rc != VMRT_OK) return rc;
  if (e != hipSuccess) return set_err(err, errlen, VMRT_INTERNAL, "VM execution: " + hip_msg(e));
  return check_status(&lp, err, errlen);
}

int vmrt_program_status(vmrt_program* p, char* err, size_t errlen) {
  if (!p) return set_err(err, errlen, VMRT_INVALID_ARGUMENT, "null program");
  std::lock_guard<std::mutex> g(p->rt->mu);
  hipSetDevice(p->rt->device);
  // the last launch of this program, on whichever stream it was enqueued
  hipError_t e = p->launched ? hipStreamSynchronize(p->last_stream) : hipSuccess;
  if (e != hipSuccess) return set_err(err, errlen, VMRT_INTERNAL, "synchronize: " + hip_msg(e));
  return check_status(p, err, errlen);
}

int vmrt_program_profile(vmrt_program* p, uint64_t* out, size_t n_words, int reset, char* err, size_t errlen) {
  if (!p) return set_err(err, errlen, VMRT_INVALID_ARGUMENT, "null program");
  if (!p->stats) return set_err(err, errlen, VMRT_FAILED_PRECONDITION, "profiling is off (load with PJRT_AMD_PROFILE=1)");
  if (!out || n_words < p->stats_words)
    return set_err(err, errlen, VMRT_INVALID_ARGUMENT, fmt("profile needs %zu words", p->stats_words));
  std::lock_guard<std::mutex> g(p->rt->mu);
  hipSetDevice(p->rt->device);
  hipError_t e = hipStreamSynchronize(p->rt->stream);
  if (e == hipSuccess) e = hipMemcpy(out, p->stats, p->stats_words * 8, hipMemcpyDeviceToHost);
  if (e == hipSuccess && reset) e = hipMemset(p->stats, 0, p->stats_words * 8);
  if (e != hipSuccess) return set_err(err, errlen, VMRT_INTERNAL, "profile read: " + hip_msg(e));
  return VMRT_OK;
}

int vmrt_alloc(vmrt_runtime* rt, size_t bytes, void** dptr, char* err, size_t errlen) {
  if (!rt || !dptr) return set_err(err, errlen, VMRT_INVALID_ARGUMENT, "null argument");
  hipSetDevice(rt->device);
  hipError_t e = rt->pool.alloc(bytes, dptr);
  if (e != hipSuccess) return set_err(err, errlen, VMRT_RESOURCE_EXHAUSTED, "device alloc: " + hip_msg(e));
  return VMRT_OK;
}

int vmrt_free(vmrt_runtime* rt, void* dptr) {
  if (!rt) return VMRT_INVALID_ARGUMENT;
  if (!dptr) return VMRT_OK;
  hipSetDevice(rt->device);
  return rt->pool.release(dptr) ? VMRT_OK : VMRT_INVALID_ARGUMENT;
}

static int copy(vmrt_runtime* rt, void* dst, const void* src, size_t n, hipMemcpyKind kind, char* err, size_t errlen) {
  if (!rt || (!dst && n) || (!src && n)) return set_err(err, errlen, VMRT_INVALID_ARGUMENT, "null argument");
  std::lock_guard<std::mutex> g(rt->mu);
  hipSetDevice(rt->device);
  hipError_t e = hipMemcpyAsync(dst, src, n, kind, rt->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(rt->stream);
  if (e != hipSuccess) return set_err(err, errlen, VMRT_INTERNAL, "copy: " + hip_msg(e));
  return VMRT_OK;
}

int vmrt_h2d(vmrt_runtime* rt, void* dst, const void* src, size_t n, char* err, size_t errlen) {
  return copy(rt, dst, src, n, hipMemcpyHostToDevice, err, errlen);
}
int vmrt_d2h(vmrt_runtime* rt, void* dst, const void* src, size_t n, char* err, size_t errlen) {
  return copy(rt, dst, src, n, hipMemcpyDeviceToHost, err, errlen);
}
int vmrt_d2d(vmrt_runtime* rt, void* dst, const void* src, size_t n, char* err, size_t errlen) {
  return copy(rt, dst, src, n, hipMemcpyDeviceToDevice, err, errlen);
}

int vmrt_synchronize(vmrt_runtime* rt, char* err, size_t errlen) {
  if (!rt) return set_err(err, errlen, VMRT_INVALID_ARGUMENT, "null runtime");
  hipSetDevice(rt->device);
  hipError_t e = hipStreamSynchronize(rt->stream);
  if (e != hipSuccess) return set_err(err, errlen, VMRT_INTERNAL, "synchronize: " + hip_msg(e));
  return VMRT_OK;
}

void* vmrt_stream(vmrt_runtime* rt) { return rt ? static_cast<void*>(rt->stream) : nullptr; }

int vmrt_event_create(vmrt_runtime* rt, void** event) {
  if (!rt || !event) return VMRT_INVALID_ARGUMENT;
  hipSetDevice(rt->device);
  hipEvent_t e;
  if (hipEventCreate(&e) != hipSuccess) return VMRT_INTERNAL;
  *event = e;
  return VMRT_OK;
}

int vmrt_event_record(vmrt_runtime* rt, void* event, void* stream) {
  if (!rt || !event) return VMRT_INVALID_ARGUMENT;
  hipSetDevice(rt->device);
  hipStream_t s = stream ? static_cast<hipStream_t>(stream) : rt->stream;
  return hipEventRecord(static_cast<hipEvent_t>(event), s) == hipSuccess ? VMRT_OK : VMRT_INTERNAL;
}

int vmrt_event_elapsed_ms(void* start, void* stop, float* ms) {
  if (!start || !stop || !ms) return VMRT_INVALID_ARGUMENT;
  if (hipEventSynchronize(static_cast<hipEvent_t>(stop)) != hipSuccess) return VMRT_INTERNAL;
  return hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)) == hipSuccess
             ? VMRT_OK
             : VMRT_INTERNAL;
}

void vmrt_event_destroy(void* event) {
  if (event) (void)hipEventDestroy(static_cast<hipEvent_t>(event));
}

int vmrt_event_query(void* event) {
  if (!event) return VMRT_INVALID_ARGUMENT;
  const hipError_t e = hipEventQuery(static_cast<hipEvent_t>(event));
  return e == hipSuccess ? VMRT_OK : e == hipErrorNotReady ? VMRT_UNAVAILABLE : VMRT_INTERNAL;
}

int vmrt_event_synchronize(void* event) {
  if (!event) return VMRT_INVALID_ARGUMENT;
  return hipEventSynchronize(static_cast<hipEvent_t>(event)) == hipSuccess ? VMRT_OK : VMRT_INTERNAL;
}

}  // extern "C"
