// CPU check of the runtime's per-launch status bookkeeping (launch_slots.h):
// each launch in flight holds its own slot, a slot is reused only after it is
// given back, the pool grows block by block without moving live slots, and a
// slot's words decode to that launch's outcome alone.  Built and run by
// tests/test_launch_slots.py; prints "ok" and exits 0, or names the failed check.
#include <cstdio>
#include <cstdlib>
#include <set>
#include <string>
#include <vector>

#include "launch_slots.h"

using namespace vmrt_host;

static int g_allocs = 0, g_frees = 0;
static void* counting_alloc(size_t n) {
  ++g_allocs;
  return std::malloc(n);
}
static void counting_free(void* p) {
  ++g_frees;
  std::free(p);
}

#define CHECK(c)                                                   \
  do {                                                             \
    if (!(c)) {                                                    \
      std::printf("FAILED %s (line %d)\n", #c, __LINE__);          \
      return 1;                                                    \
    }                                                              \
  } while (0)

// What the status epilogue writes for a finished launch.
static void finish(uint32_t* s, uint32_t code, uint32_t info) {
  s[SLOT_ERROR] = code;
  s[SLOT_ERRINFO] = info;
  s[SLOT_WRITTEN] = kSlotWritten;
}

int main() {
  {
    SlotPool pool(counting_alloc, counting_free, 4);
    CHECK(pool.blocks() == 0 && pool.live() == 0);
    // two launches of one program in flight: distinct, zeroed slots
    uint32_t* a = pool.take();
    uint32_t* b = pool.take();
    CHECK(a && b && a != b);
    for (uint32_t k = 0; k < SLOT_WORDS; ++k) CHECK(a[k] == 0 && b[k] == 0);
    std::string msg;
    // not finished yet: no status written
    CHECK(slot_status(a, &msg) == 13 && msg.find("not written") != std::string::npos);
    // the first launch aborts at a barrier, the second completes: each reports its own
    finish(a, vm::VM_ERR_BARRIER_TIMEOUT, 7);
    finish(b, vm::VM_OK, 0);
    CHECK(slot_status(b, &msg) == 0);
    CHECK(slot_status(a, &msg) == 13);
    CHECK(msg.find("grid barrier timed out") != std::string::npos && msg.find("detail 7") != std::string::npos);
    // reading a slot does not clear it (several events may ask)
    CHECK(slot_status(a, &msg) == 13 && slot_status(b, &msg) == 0);
    CHECK(pool.live() == 2);
    // a given-back slot is handed out again, zeroed
    pool.give(a);
    uint32_t* c = pool.take();
    CHECK(c == a);
    for (uint32_t k = 0; k < SLOT_WORDS; ++k) CHECK(c[k] == 0);
    CHECK(slot_status(b, &msg) == 0);              // b's outcome untouched by c's reuse
    // many launches in flight: the pool grows by blocks, every live slot distinct and stable
    std::vector<uint32_t*> live = {b, c};
    for (int i = 0; i < 13; ++i) live.push_back(pool.take());
    std::set<uint32_t*> uniq(live.begin(), live.end());
    CHECK(uniq.size() == live.size());
    CHECK(pool.blocks() == 4 && g_allocs == 4 && pool.live() == live.size());
    for (size_t i = 0; i < live.size(); ++i) finish(live[i], uint32_t(i % 3 == 0 ? vm::VM_ERR_FRAME_DEPTH : 0), uint32_t(i));
    for (size_t i = 0; i < live.size(); ++i) {
      const int rc = slot_status(live[i], &msg);
      CHECK(rc == (i % 3 == 0 ? 13 : 0));
      if (rc) CHECK(msg.find("frame stack overflow") != std::string::npos);
    }
    for (uint32_t* s : live) pool.give(s);
    CHECK(pool.live() == 0);
    // unknown codes still report an abort with their number
    uint32_t* d = pool.take();
    finish(d, 99, 1);
    CHECK(slot_status(d, &msg) == 13 && msg.find("code 99") != std::string::npos);
    pool.give(d);
  }
  CHECK(g_frees == g_allocs);                      // the pool frees its blocks
  std::printf("ok\n");
  return 0;
}
