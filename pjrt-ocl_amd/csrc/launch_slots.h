// Per-launch status of the runtime (host code only, no HIP types): the slots a
// launch's status is copied into, and their meaning.
//
// A program's status word (control word BAR_ERROR) is shared by all its
// launches.  A launch submitted with vmrt_submit is followed on its stream by a
// small status epilogue kernel that copies that word into a slot of its own and,
// when the launch aborted, clears the control words and task scratch before any
// later launch of the program starts.  The slot sits in host memory the device
// writes (pinned memory in the runtime), so a caller reads a finished launch's
// outcome without a device call, and no launch can see or clear another's.
#pragma once
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <mutex>
#include <string>
#include <vector>

#include "vm_abi.h"

namespace vmrt_host {

// Words of one slot.  SLOT_WRITTEN holds kSlotWritten once the epilogue ran.
enum : uint32_t { SLOT_ERROR = 0, SLOT_ERRINFO = 1, SLOT_WRITTEN = 2, SLOT_WORDS = 4 };
constexpr uint32_t kSlotWritten = 0x53544154u;

// What a nonzero VM status word means (vm_abi.h VmError).
inline const char* vm_error_text(uint32_t code) {
  switch (code) {
    case vm::VM_ERR_BARRIER_TIMEOUT:
      return "grid barrier timed out (lanes not co-resident, or non-uniform control across lanes)";
    case vm::VM_ERR_FRAME_DEPTH: return "control frame stack overflow";
    case vm::VM_ERR_BAD_TASK: return "unsupported tile op reached the device";
    default: return "VM error";
  }
}

// Outcome of a finished launch from its slot: 0 (OK), or 13 (INTERNAL, the
// PJRT_Error_Code the runtime reports VM aborts with) and a message.
inline int slot_status(const volatile uint32_t* s, std::string* msg) {
  if (s[SLOT_WRITTEN] != kSlotWritten) {
    *msg = "launch status was not written (the status epilogue did not run)";
    return 13;
  }
  const uint32_t code = s[SLOT_ERROR];
  if (code == vm::VM_OK) return 0;
  char buf[256];
  std::snprintf(buf, sizeof buf, "VM aborted: %s (code %u, detail %u)", vm_error_text(code), code,
                unsigned(s[SLOT_ERRINFO]));
  *msg = buf;
  return 13;
}

// Slots in blocks of `per_block`, allocated through `alloc` as launches need
// them and freed with the pool.  take() hands out a zeroed slot no other live
// launch holds; give() takes it back.  Thread-safe.
class SlotPool {
 public:
  typedef void* (*AllocFn)(size_t bytes);
  typedef void (*FreeFn)(void* p);
  SlotPool(AllocFn alloc, FreeFn free, size_t per_block = 256) : alloc_(alloc), free_(free), per_block_(per_block) {}
  SlotPool(const SlotPool&) = delete;
  SlotPool& operator=(const SlotPool&) = delete;
  ~SlotPool() {
    for (void* b : blocks_) free_(b);
  }
  uint32_t* take() {
    std::lock_guard<std::mutex> g(mu_);
    if (free_list_.empty()) {
      void* b = alloc_(per_block_ * SLOT_WORDS * sizeof(uint32_t));
      if (!b) return nullptr;
      blocks_.push_back(b);
      for (size_t i = per_block_; i-- > 0;) free_list_.push_back(static_cast<uint32_t*>(b) + i * SLOT_WORDS);
    }
    uint32_t* s = free_list_.back();
    free_list_.pop_back();
    for (uint32_t k = 0; k < SLOT_WORDS; ++k) s[k] = 0;
    ++live_;
    return s;
  }
  void give(uint32_t* s) {
    std::lock_guard<std::mutex> g(mu_);
    free_list_.push_back(s);
    --live_;
  }
  size_t live() const {
    std::lock_guard<std::mutex> g(mu_);
    return live_;
  }
  size_t blocks() const {
    std::lock_guard<std::mutex> g(mu_);
    return blocks_.size();
  }

 private:
  AllocFn alloc_;
  FreeFn free_;
  size_t per_block_;
  mutable std::mutex mu_;
  std::vector<void*> blocks_;
  std::vector<uint32_t*> free_list_;
  size_t live_ = 0;
};

}  // namespace vmrt_host
