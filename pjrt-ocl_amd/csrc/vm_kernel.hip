// The persistent VM: one workgroup per lane, each walking its own entry stream
// (reference: pjrt_plugin/kernels/vm_main.cl:107-258 `vm2`).
//
// Stream walk: a frame stack (depth 8) of {pc, end, owning control entry, phase}.
//   BARRIER  -> grid barrier across all lanes
//   WHILE    -> cond sub-list, barrier, read cond, body sub-list, barrier, repeat
//   FOR      -> body sub-list, barrier, x trip count (wait_flag)
//   IF       -> then / else sub-list chosen by the cond value
//   NOP      -> skip
//   task     -> run tiles [tile_lo, tile_hi) of tasks[task]; an entry may first
//               wait for completion flags and afterwards signal one (vm_device.h)
// Consecutive task entries of one lane form a fused chain: a block barrier with a
// workgroup fence separates them, because a tile op maps elements to threads
// differently from its producer (vm_main.cl:82-100).
#include <hip/hip_runtime.h>

#include "tile_attn.h"
#include "tile_decode.h"
#include "tile_ew.h"
#include "tile_gemv.h"
#include "tile_index.h"
#include "tile_mma.h"
#include "tile_reduce.h"

namespace vm {

constexpr int kMaxDepth = 8;
constexpr uint32_t kRootOwner = 0xFFFFFFFFu;

// LDS shared by the tile ops of one lane (the matmul's double-buffered operand
// slabs are the largest user).
constexpr int kSmemBytes0 = (kMmaLdsBytes > kAttnLdsBytes ? kMmaLdsBytes : kAttnLdsBytes);
constexpr int kSmemBytes = (kSmemBytes0 > int(kDecLdsBytes) ? kSmemBytes0 : int(kDecLdsBytes));

VM_DEV void exec_tiles(Args A, uint32_t ti, uint32_t lo, uint32_t hi) {
  switch (task_of(A, ti).tile_op & 0xFF) {
    case TOP_EW: ew_tile(A, ti, lo, hi); break;
    case TOP_MMA: mma_tiles(A, ti, lo, hi); break;
    case TOP_GATHER: gather_tiles(A, ti, lo, hi, false); break;
    case TOP_RED_PART: red_flat_tiles(A, ti, lo, hi, false); break;
    case TOP_RED_COMB: red_flat_tiles(A, ti, lo, hi, true); break;
    case TOP_IOTA_DIM: iota_tiles(A, ti, lo, hi); break;
    case TOP_SCATTER: gather_tiles(A, ti, lo, hi, true); break;
    case TOP_DYN_GATHER: dyn_tiles(A, ti, lo, hi, false); break;
    case TOP_DYN_SCATTER: dyn_tiles(A, ti, lo, hi, true); break;
    case TOP_RED_SEG: red_seg_tiles(A, ti, lo, hi); break;
    case TOP_SOFTMAX_SEG: softmax_tiles(A, ti, lo, hi); break;
    case TOP_LAYERNORM_SEG: layernorm_tiles(A, ti, lo, hi); break;
    case TOP_MAP_REGION: map_region_tiles(A, ti, lo, hi); break;
    case TOP_FLASH_ATTN: flash_attn_tiles(A, ti, lo, hi); break;
    case TOP_RED_STRIDED: red_strided_tiles(A, ti, lo, hi); break;
    case TOP_GATHER_INDEX: gather_index_tiles(A, ti, lo, hi); break;
    case TOP_ARGMAX_SEG: argmax_tiles(A, ti, lo, hi); break;
    case TOP_GEMV: gemv_tiles(A, ti, lo, hi); break;
    case TOP_DECODE_ATTN: decode_attn_tiles(A, ti, lo, hi); break;
    default: raise_error(A, VM_ERR_BAD_TASK, task_of(A, ti).tile_op); break;
  }
}

// Scalar-cache warm-up for the entry after a barrier: the entry, its task record
// and, for a GEMV, the fused layernorm's task record and the epilogue words --
// the dependent scalar loads a tile starts with.  Run between the lane's
// arrival and its wait, so the loads (about a microsecond of dependent misses
// after each barrier) overlap the wait instead of following it.  The values are
// kept live (an empty asm) so the loads are issued, then dropped.
VM_DEV void warm_entry(Args A, const VM_K Entry* ents, uint32_t i, uint32_t end) {
  if (i >= end) return;
  const Entry e = load_entry(ents + i);
  asm volatile("" ::"s"(e.tile_hi));
  if (e.task >= ENT_FOR) return;                          // a control entry
  const VM_K Task& t = task_of(A, e.task);
  const uint32_t top = t.tile_op, p5 = t.p[5], p6 = t.p[6];
  asm volatile("" ::"s"(t.dst), "s"(t.a), "s"(t.b), "s"(t.p[0]), "s"(t.p[4]), "s"(t.p[7]));
  if ((top & 0xFF) != TOP_GEMV) return;
  if (p5) {
    const VM_K Task& L = task_of(A, p5 - 1);
    asm volatile("" ::"s"(L.a), "s"(L.b), "s"(L.p[3]), "s"(L.p[4]));
  }
  if (p6) asm volatile("" ::"s"(aux_of(A)[p6 - 1]));   // the epilogue's count word (checked at load)
}

// grid_barrier, with the lane's wait added to the profiling counters when on;
// the entry at `next` (when inside [.., end)) is warmed while the lane waits
VM_DEV bool timed_barrier(Args A, const VM_K Entry* ents, uint32_t next, uint32_t end) {
  auto pre = [&] { warm_entry(A, ents, next, end); };
  if (!A->stats) return grid_barrier(A, pre);
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  const bool ok = grid_barrier(A, pre);
  if (threadIdx.x == 0) {
    __hip_atomic_fetch_add(A->stats, __builtin_amdgcn_s_memrealtime() - t0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_fetch_add(A->stats + 1, uint64_t(1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  return ok;
}

__global__ __launch_bounds__(kBlock, 1) void vm_main(VmArgs args) {
  // The VmArgs block is the kernel's only explicit argument: offset 0 of the
  // kernarg segment, read in place through the constant address space.
  (void)args;
  const Args A = (Args)__builtin_amdgcn_kernarg_segment_ptr();
  const uint32_t lane = blockIdx.x;
  const uint64_t t_launch = A->stats ? __builtin_amdgcn_s_memrealtime() : 0;   // profiling: the lane's span
  grid_barrier_init(A);
  const LaneSpan span = load_span((const VM_K LaneSpan*)A->lanes + lane);
  const VM_K Entry* ents = (const VM_K Entry*)A->entries + span.off;
  // the loader put the task of the lane's first entry in span.pad: request the
  // entry and that task record together (one scalar round trip, not two)
  if (span.pad != 0xFFFFFFFFu) {
    const Entry e0 = load_entry(ents);
    const VM_K Task& t0 = task_of(A, span.pad);
    asm volatile("" ::"s"(e0.tile_hi), "s"(t0.tile_op), "s"(t0.dst), "s"(t0.a), "s"(t0.b), "s"(t0.p[0]), "s"(t0.p[4]),
                 "s"(t0.p[7]));
  }

  uint32_t f_pc[kMaxDepth], f_end[kMaxDepth], f_own[kMaxDepth], f_phase[kMaxDepth];
  int sp = 0;
  f_pc[0] = 0;
  f_end[0] = span.root_len;
  f_own[0] = kRootOwner;
  f_phase[0] = 0;
  bool pub = false;     // a tile entry ran since the last barrier
  uint32_t nbar = 0;    // grid barriers this lane has passed in this launch (completion flag values)

  for (;;) {
    if (f_pc[sp] >= f_end[sp]) {
      if (f_own[sp] == kRootOwner) break;
      const Entry w = load_entry(ents + f_own[sp]);
      if (w.task == ENT_IF) {                 // branch done
        --sp;
        ++f_pc[sp];
        continue;
      }
      // loop bodies end with a grid barrier that publishes the carries
      // (warming a FOR body's first entry when another trip follows)
      const bool again = w.task == ENT_FOR && f_phase[sp] > 1;
      if (!timed_barrier(A, ents, again ? w.tile_lo : 0u, again ? w.tile_lo + w.tile_hi : 0u)) return;
      ++nbar;
      pub = false;
      if (w.task == ENT_FOR) {
        if (--f_phase[sp] != 0) {
          f_pc[sp] = w.tile_lo;
          f_end[sp] = w.tile_lo + w.tile_hi;
        } else {
          --sp;
          ++f_pc[sp];
        }
        continue;
      }
      if (f_phase[sp] == 0) {                 // while-cond done: test
        if (read_cond(resolve(A, w.signal_flag), w.pad)) {
          f_pc[sp] = w.wait_flag;
          f_end[sp] = w.wait_flag + w.wait_count;
          f_phase[sp] = 1;
        } else {
          --sp;
          ++f_pc[sp];
        }
      } else {                                // while-body done: re-test
        f_pc[sp] = w.tile_lo;
        f_end[sp] = w.tile_lo + w.tile_hi;
        f_phase[sp] = 0;
      }
      continue;
    }

    const uint32_t epc = f_pc[sp];
    const Entry en = load_entry(ents + epc);
    if (en.task == ENT_BARRIER) {
      if (!timed_barrier(A, ents, epc + 1, f_end[sp])) return;
      ++nbar;
      pub = false;
      ++f_pc[sp];
      continue;
    }
    if (en.task == ENT_WHILE || en.task == ENT_FOR || en.task == ENT_IF) {
      uint32_t start, len, phase;
      if (en.task == ENT_WHILE) {
        start = en.tile_lo;
        len = en.tile_hi;
        phase = 0;
      } else if (en.task == ENT_FOR) {
        if (en.wait_flag == 0) {
          ++f_pc[sp];
          continue;
        }
        start = en.tile_lo;
        len = en.tile_hi;
        phase = en.wait_flag;
      } else {
        const bool c = read_cond(resolve(A, en.signal_flag), en.pad);
        start = c ? en.tile_lo : en.wait_flag;
        len = c ? en.tile_hi : en.wait_count;
        phase = 2;
        if (len == 0) {
          ++f_pc[sp];
          continue;
        }
      }
      if (sp + 1 >= kMaxDepth) {
        raise_error(A, VM_ERR_FRAME_DEPTH, lane);
        return;
      }
      ++sp;
      f_pc[sp] = start;
      f_end[sp] = start + len;
      f_own[sp] = epc;
      f_phase[sp] = phase;
      continue;
    }
    if (en.task != ENT_NOP) {
      if (pub) __syncthreads();
      pub = true;
      // the loader sets wait_count 0 and signal_flag FLAG_NONE on entries without flags
      if (en.wait_count) {
        const uint64_t tw = A->stats ? __builtin_amdgcn_s_memrealtime() : 0;
        if (!flag_wait(A, en.wait_flag, en.wait_count, phase_tag(A, nbar))) return;
        if (A->stats && threadIdx.x == 0)
          __hip_atomic_fetch_add(A->stats + 3, __builtin_amdgcn_s_memrealtime() - tw, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
      }
      // One call site: the dispatch switch is inlined once, with the register
      // saving around each of its calls (two copies, one per stats mode, made
      // the kernel 79 KB instead of 46 KB and cost C5 7 %).
      const uint64_t t0 = A->stats ? __builtin_amdgcn_s_memrealtime() : 0;
      exec_tiles(A, en.task, en.tile_lo, en.tile_hi);
      if (A->stats) {
        __syncthreads();
        if (threadIdx.x == 0) {
          const uint64_t dt = __builtin_amdgcn_s_memrealtime() - t0;
          uint64_t* st = A->stats + kStatTask + 4ull * en.task;
          __hip_atomic_fetch_add(st, dt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_fetch_max(st + 1, dt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_fetch_add(st + 2, uint64_t(1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      if (en.signal_flag != FLAG_NONE) flag_signal(A, en.signal_flag, phase_tag(A, nbar));
    }
    ++f_pc[sp];
  }
  if (A->stats && threadIdx.x == 0)
    __hip_atomic_fetch_add(A->stats + 2, __builtin_amdgcn_s_memrealtime() - t_launch, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}

// Status epilogue of a launch submitted with vmrt_submit, run after it on the
// same stream: copies the program's status words into the launch's own slot (host
// memory, slot layout in launch_slots.h) and, when the launch aborted, clears
// the control words and the task scratch, so a later launch of the program
// queued behind this one starts from the state the loader leaves (an aborted
// launch can leave arrival flags and split counters part-way).  One block:
// every thread reads the status before the block barrier, and only then may
// any thread clear it.
__global__ __launch_bounds__(1024) void vm_status_epilogue(uint32_t* ctl, uint32_t* slot, uint32_t* scratch,
                                                          uint64_t scratch_words) {
  const uint32_t err = __hip_atomic_load(&ctl[BAR_ERROR], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint32_t info = __hip_atomic_load(&ctl[BAR_ERRINFO], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (threadIdx.x == 0) {
    __hip_atomic_store(&slot[0], err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __hip_atomic_store(&slot[1], info, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __hip_atomic_store(&slot[2], 0x53544154u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
  }
  if (err == VM_OK) return;
  for (uint32_t i = threadIdx.x; i < uint32_t(BAR_WORDS); i += blockDim.x) ctl[i] = 0;
  for (uint64_t i = threadIdx.x; i < scratch_words; i += blockDim.x) scratch[i] = 0;
}

}  // namespace vm

// ---- host side of the launch (called by the runtime) ------------------------------------
extern "C" hipError_t vm_status_epilogue_launch(uint32_t* ctl, uint32_t* slot, uint8_t* scratch,
                                                uint64_t scratch_bytes, hipStream_t stream) {
  uint32_t* words = reinterpret_cast<uint32_t*>(scratch);
  uint64_t n_words = scratch_bytes / 4;
  void* args[] = {&ctl, &slot, &words, &n_words};
  return hipLaunchKernel(reinterpret_cast<const void*>(&vm::vm_status_epilogue), dim3(1), dim3(1024), args, 0, stream);
}
extern "C" int vm_kernel_smem_bytes() { return vm::kSmemBytes; }

extern "C" hipError_t vm_kernel_prepare() {
  return hipFuncSetAttribute(reinterpret_cast<const void*>(&vm::vm_main), hipFuncAttributeMaxDynamicSharedMemorySize,
                             vm::kSmemBytes);
}

extern "C" hipError_t vm_kernel_occupancy(int* blocks_per_cu) {
  return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, reinterpret_cast<const void*>(&vm::vm_main),
                                                      vm::kBlock, vm::kSmemBytes);
}

// cooperative != 0: hipLaunchCooperativeKernel (co-residency of every lane is
// guaranteed or the launch fails); otherwise a plain launch, used only when the
// lane count fits the occupancy the runtime verified.
extern "C" hipError_t vm_kernel_launch(const vm::VmArgs* args, hipStream_t stream, int cooperative) {
  vm::VmArgs a = *args;
  void* params[] = {&a};
  if (cooperative)
    return hipLaunchCooperativeKernel(reinterpret_cast<const void*>(&vm::vm_main), dim3(a.n_lanes), dim3(vm::kBlock),
                                      params, vm::kSmemBytes, stream);
  return hipLaunchKernel(reinterpret_cast<const void*>(&vm::vm_main), dim3(a.n_lanes), dim3(vm::kBlock), params,
                         vm::kSmemBytes, stream);
}
