// Device-side helpers of the persistent VM: address spaces, buffer handle
// resolution, element conversions, wave64 DPP reductions, the grid barrier.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vm_abi.h"

namespace vm {

constexpr int kBlock = 256;              // threads per lane (4 wave64s)
constexpr int kWaves = kBlock / 64;

#define VM_DEV __device__ __forceinline__
// Tile-op entry points and their large specialisations are real device functions:
// each gets its own register allocation and instruction schedule (the kernel
// reserves the maximum), which keeps the one-kernel build tractable.
#define VM_TILE __device__ __attribute__((noinline))
// The matrix-core tiles (GEMM, flash attention) fill all 512 registers.  As
// ordinary callees they would save and restore every callee-saved VGPR and AGPR
// they touch (over 300 dwords per thread) around each call.  Called from the
// kernel itself and never as a tail call, the compiler's interprocedural
// register allocation lets them skip that, and the kernel keeps what it needs
// instead (a few values).  Measured on MI355X: C3 bf16 151 -> 133 us, C4 116 ->
// 94 us.  Their dispatchers are inlined into the kernel for the same reason.
#define VM_LEAF __device__ __attribute__((noinline, not_tail_called))

// Address spaces: tensor data is global memory (global_load/store with an SGPR
// base), the kernel-argument block and the read-only program tables (tasks,
// entries, lane table, aux) are read through the constant address space so
// wave-uniform reads become scalar loads.
#define VM_G __attribute__((address_space(1)))
#define VM_K __attribute__((address_space(4)))
typedef VM_G uint8_t gbyte;
typedef const VM_K VmArgs* Args;

// The lane's LDS: one dynamic allocation shared by every tile op (the largest
// user sizes it).  Declared at namespace scope so non-inlined tile functions
// address it as LDS directly.
extern __shared__ __align__(16) uint8_t vm_smem[];

// Base of the dynamic LDS block, read once into a scalar register.  In the tile
// functions (not the kernel itself) the compiler finds the block through the
// kernel's dynamic-LDS offset table; that table read is a global load which,
// under register pressure, it repeats at every use inside a loop, each with a
// full memory wait.  An empty asm that owns the value in an SGPR makes it opaque,
// so it is kept (or spilled) instead of re-derived.
template <typename T>
VM_DEV T* lds_ptr() {
  typedef __attribute__((address_space(3))) uint8_t lds_u8;
  uint32_t off = uint32_t(reinterpret_cast<uintptr_t>((lds_u8*)vm_smem));
  asm("" : "+s"(off));
  return (T*)(lds_u8*)(uintptr_t)off;
}

VM_DEV uint32_t uni(uint32_t x) { return __builtin_amdgcn_readfirstlane(x); }

// A pointer argument of a non-inlined function arrives in VGPRs; make it
// wave-uniform again so reads through it are scalar.
template <typename T>
VM_DEV T* uni_ptr(T* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint64_t lo = uni(uint32_t(v)), hi = uni(uint32_t(v >> 32));
  return reinterpret_cast<T*>((hi << 32) | lo);
}
VM_DEV Args uargs(Args A) { return uni_ptr(A); }

template <typename T>
VM_DEV VM_G T* gcast(gbyte* p) { return (VM_G T*)p; }
template <typename T>
VM_DEV const VM_G T* gcast(const gbyte* p) { return (const VM_G T*)p; }

// Builtin vector types (clang ext vectors load and store through address-space
// qualified pointers, unlike HIP's float4 class).
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));
VM_DEV v4f v4f_make(float a, float b, float c, float d) { return v4f{a, b, c, d}; }
VM_DEV v4u v4u_make(uint32_t a, uint32_t b, uint32_t c, uint32_t d) { return v4u{a, b, c, d}; }
VM_DEV v2u v2u_make(uint32_t a, uint32_t b) { return v2u{a, b}; }

// Value load through a typed global pointer (an rvalue without the address space).
template <typename T>
VM_DEV T gld(const VM_G T* p) { return *p; }

// Control records read field by field from the constant address space.
VM_DEV Entry load_entry(const VM_K Entry* p) {
  Entry e;
  e.task = p->task;
  e.tile_lo = p->tile_lo;
  e.tile_hi = p->tile_hi;
  e.wait_flag = p->wait_flag;
  e.wait_count = p->wait_count;
  e.signal_flag = p->signal_flag;
  e.slots = p->slots;
  e.pad = p->pad;
  return e;
}
VM_DEV LaneSpan load_span(const VM_K LaneSpan* p) {
  LaneSpan s;
  s.off = p->off;
  s.count = p->count;
  s.root_len = p->root_len;
  s.pad = p->pad;
  return s;
}

VM_DEV const VM_K int32_t* aux_of(Args A) { return (const VM_K int32_t*)A->aux; }
VM_DEV const VM_K Task& task_of(Args A, uint32_t i) { return ((const VM_K Task*)A->tasks)[uni(i)]; }

// Handles are wave-uniform: an arena byte offset, or PORT_BIT | port index.
VM_DEV gbyte* resolve(Args A, uint32_t h) {
  h = uni(h);
  uint8_t* p = (h & PORT_BIT) ? A->ports[h & (kMaxPorts - 1)] : A->arena + h;
  return (gbyte*)p;
}

// ---- element formats ------------------------------------------------------------------
VM_DEV float bf16_to_f32(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }

// Round-to-nearest-even f32 -> bf16 (vm_common.cl:66-70).  A NaN keeps a NaN
// pattern (quiet bit set) instead of the carry the bit formula would produce.
VM_DEV uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return uint16_t((u >> 16) | 0x40u);
  return uint16_t((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
// Two f32 -> packed bf16 pair (low half = a) with gfx950's v_cvt_pk_bf16_f32:
// round-to-nearest-even, the same result as f32_to_bf16 (checked bit-exact over
// 2^24 patterns including NaN / Inf / denormals by the GPU tests).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
VM_DEV uint32_t pack_bf16x2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{a, b}), bf16x2_t));
}
VM_DEV float f16_to_f32(uint16_t h) { return float(__builtin_bit_cast(_Float16, h)); }
VM_DEV uint16_t f32_to_f16(float f) { return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f)); }

// Element size in bytes of a dtype.
VM_DEV uint32_t dt_size(uint32_t dt) {
  return (dt == DT_I64 || dt == DT_F64) ? 8u : dt == DT_BOOL ? 1u
       : (dt == DT_F16 || dt == DT_BF16) ? 2u : 4u;
}

// Load element i of a buffer as f32 (the VM's arithmetic domain).
VM_DEV float load_f(const gbyte* base, uint32_t dt, uint64_t i) {
  switch (dt) {
    case DT_BF16: return bf16_to_f32(gcast<uint16_t>(base)[i]);
    case DT_F16: return f16_to_f32(gcast<uint16_t>(base)[i]);
    case DT_I32: return float(gcast<int32_t>(base)[i]);
    case DT_U32: return float(gcast<uint32_t>(base)[i]);
    case DT_BOOL: return float(base[i]);
    case DT_I64: return float(gcast<int64_t>(base)[i]);
    case DT_F64: return float(gcast<double>(base)[i]);
    default: return gcast<float>(base)[i];
  }
}
VM_DEV void store_f(gbyte* base, uint32_t dt, uint64_t i, float v) {
  switch (dt) {
    case DT_BF16: gcast<uint16_t>(base)[i] = f32_to_bf16(v); break;
    case DT_F16: gcast<uint16_t>(base)[i] = f32_to_f16(v); break;
    case DT_F64: gcast<double>(base)[i] = double(v); break;
    case DT_I32: gcast<int32_t>(base)[i] = int32_t(v); break;
    case DT_U32: gcast<uint32_t>(base)[i] = uint32_t(int64_t(v)); break;
    case DT_I64: gcast<int64_t>(base)[i] = int64_t(v); break;
    case DT_BOOL: base[i] = v != 0.0f; break;
    default: gcast<float>(base)[i] = v; break;
  }
}

// Four f32 / bf16 / f16 elements e..e+3 as f32 (e a multiple of 4, base 16-byte
// aligned) and back.
VM_DEV v4f ld4(const gbyte* p, uint32_t dt, uint64_t e) {   // e: element index (multiple of 4)
  if (dt == DT_F32) return *(const VM_G v4f*)(gcast<float>(p) + e);
  const v2u w = *(const VM_G v2u*)(gcast<uint16_t>(p) + e);
  if (dt == DT_BF16)
    return v4f_make(__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xFFFF0000u),
                       __uint_as_float(w.y << 16), __uint_as_float(w.y & 0xFFFF0000u));
  return v4f_make(f16_to_f32(w.x & 0xFFFF), f16_to_f32(w.x >> 16), f16_to_f32(w.y & 0xFFFF),
                     f16_to_f32(w.y >> 16));
}
VM_DEV void st4(gbyte* p, uint32_t dt, uint64_t e, v4f v) {
  if (dt == DT_F32) {
    *(VM_G v4f*)(gcast<float>(p) + e) = v;
  } else if (dt == DT_BF16) {
    *(VM_G v2u*)(gcast<uint16_t>(p) + e) = v2u_make(pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w));
  } else {
    *(VM_G v2u*)(gcast<uint16_t>(p) + e) = v2u_make(f32_to_f16(v.x) | (uint32_t(f32_to_f16(v.y)) << 16),
                                                         f32_to_f16(v.z) | (uint32_t(f32_to_f16(v.w)) << 16));
  }
}

// ---- wave64 reductions through DPP ----------------------------------------------
// quad_perm [1,0,3,2] and [2,3,0,1], then row_ror 4 and 8: every lane of a
// 16-lane row holds the row total; four v_readlane_b32 combine the rows.
template <int CTRL>
VM_DEV float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
VM_DEV float lane_read(float x, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l));
}

struct OpSum { VM_DEV float operator()(float a, float b) const { return a + b; } };
struct OpMax { VM_DEV float operator()(float a, float b) const { return fmaxf(a, b); } };
struct OpMin { VM_DEV float operator()(float a, float b) const { return fminf(a, b); } };
struct OpProd { VM_DEV float operator()(float a, float b) const { return a * b; } };

// Reduce over the 64 lanes of a wave; the result is wave-uniform.
template <class Op>
VM_DEV float wave_reduce(float x, Op op) {
  x = op(x, dpp<0xB1>(x));     // quad_perm [1,0,3,2]
  x = op(x, dpp<0x4E>(x));     // quad_perm [2,3,0,1]
  x = op(x, dpp<0x124>(x));    // row_ror:4
  x = op(x, dpp<0x128>(x));    // row_ror:8
  return op(op(lane_read(x, 0), lane_read(x, 16)), op(lane_read(x, 32), lane_read(x, 48)));
}
VM_DEV float wave_sum(float x) { return wave_reduce(x, OpSum()); }
VM_DEV float wave_max(float x) { return wave_reduce(x, OpMax()); }

// ---- grid barrier ----------------------------------------------------------------------
// Grid barrier: arrival flags and a master lane.  Barrier number k of a launch
// has epoch e0 + k, where e0 is ctl[BAR_GEN] when the launch starts (equal for all
// lanes: the previous launch ended with every lane past its last barrier).  A lane
// arrives by storing the epoch into its own word ctl[BAR_FLAGS + lane] with
// release semantics -- a plain store to a private word, so arrivals never queue
// on one atomic -- then spins until its XCD's copy of the release epoch reaches the
// epoch.  Lane 0 is the master: its 256 threads poll the other lanes' words until
// all have reached the epoch and then publish it in one word per XCD (so each
// polled line is shared by one XCD's lanes only) and in ctl[BAR_GEN].  The release before each arrival and
// the acquire after the wait make every lane's writes before the barrier visible
// to every lane after it across the XCDs' L2s (the reference's device-scope fence
// pair, vm_common.cl:231-300).  Every wait gives up after `timeout_ticks` of the
// 100 MHz constant clock, so a broken schedule ends the launch with an error
// instead of hanging.  Returns false when the launch must abort.
__shared__ uint32_t vm_bar_epoch;      // epoch of this lane's last barrier
__shared__ uint32_t vm_bar_ready;      // vm_bar_epoch is set (this lane passed a barrier)

// The launch's base epoch is read at the lane's first barrier, not here: until
// this lane has arrived there, lane 0 cannot advance ctl[BAR_GEN], so the read
// still sees the base -- and a program without barriers never waits on it
// (the read is a memory round trip ahead of every lane's first tile).
VM_DEV void grid_barrier_init(Args A) {
  (void)A;
  if (threadIdx.x == 0) vm_bar_ready = 0;   // read after grid_barrier's first block sync
}

// Every poll checks the clock; only every 32nd also reads the error word (a
// memory round trip that would otherwise double the latency of each poll).
VM_DEV bool barrier_timed_out(Args A, uint64_t t0, uint32_t poll) {
  uint32_t* ctl = A->ctl;
  if ((poll & 31) == 31 && __hip_atomic_load(&ctl[BAR_ERROR], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return true;
  if (__builtin_amdgcn_s_memrealtime() - t0 > A->timeout_ticks) {
    uint32_t expect = 0;
    __hip_atomic_compare_exchange_strong(&ctl[BAR_ERROR], &expect, uint32_t(VM_ERR_BARRIER_TIMEOUT), __ATOMIC_RELAXED,
                                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
  }
  return false;
}

// `pre` runs on every thread of the lane once its arrival is published and
// before it waits (on lane 0, the master, after the release): work that does
// not depend on the phase before, such as warming the scalar cache with the
// next entry's task records, then overlaps the wait.
struct NoPre {
  VM_DEV void operator()() const {}
};

template <typename Pre>
VM_DEV bool grid_barrier(Args A, Pre&& pre) {
  __shared__ uint32_t s_ok;
  __syncthreads();
  uint32_t* ctl = A->ctl;
  if (!vm_bar_ready) {       // block-uniform: vm_bar_ready changes only after the last sync below
    if (threadIdx.x == 0)
      vm_bar_epoch = __hip_atomic_load(&ctl[BAR_GEN], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
  }
  const uint32_t epoch = vm_bar_epoch + 1;
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  if (blockIdx.x == 0) {
    if (threadIdx.x == 0) s_ok = 1;
    for (uint32_t poll = 0;; ++poll) {
      bool mine = true;
      for (uint32_t l = threadIdx.x + 1; l < A->n_lanes; l += kBlock)
        if (int32_t(__hip_atomic_load(&ctl[BAR_FLAGS + l], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - epoch) < 0)
          mine = false;
      if (__syncthreads_and(mine)) break;
      if (threadIdx.x == 0 && barrier_timed_out(A, t0, poll)) s_ok = 0;
      __syncthreads();
      if (!s_ok) break;
      __builtin_amdgcn_s_sleep(1);
    }
    if (threadIdx.x < kXcds && s_ok) {
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      __hip_atomic_store(&ctl[BAR_XGEN + 32 * threadIdx.x], epoch, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
      if (threadIdx.x == 0) __hip_atomic_store(&ctl[BAR_GEN], epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    pre();
  } else {
    if (threadIdx.x == 0)
      __hip_atomic_store(&ctl[BAR_FLAGS + blockIdx.x], epoch, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    pre();
    if (threadIdx.x == 0) {
      uint32_t ok = 1;
      const uint32_t* gen = &ctl[BAR_XGEN + 32 * (blockIdx.x % kXcds)];
      for (uint32_t poll = 0;
           int32_t(__hip_atomic_load(gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - epoch) < 0; ++poll) {
        if (barrier_timed_out(A, t0, poll)) {
          ok = 0;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      s_ok = ok;
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {        // read again only after the next barrier's block sync
    vm_bar_epoch = epoch;
    vm_bar_ready = 1;
  }
  return s_ok != 0;
}

VM_DEV bool grid_barrier(Args A) { return grid_barrier(A, NoPre()); }

// ---- completion flags (extension of the entries' reserved WAIT / SIGNAL fields) ------
// A tile entry may signal one flag when its tiles are done, and wait for a range of
// flags before it starts: a point-to-point dependency inside one barrier phase in
// place of a grid barrier (the scheduler uses it where a consumer's tiles read the
// output of only a few producer tiles, such as one head's q, k and v).  A flag is a
// 64-bit word holding the identity of the phase instance that last signaled it:
// the launch's sequence number in the high half, the count of grid barriers the
// lane has passed in this launch, plus one, in the low half.  Every lane passes
// the same barriers, so producer and consumer compute the same identity; a value
// left by an earlier launch, loop trip or phase never equals it, so flags need no
// reset.  The loader checks that every waited flag has exactly one signaling
// entry in the same barrier segment and that, in each lane's segment, no entry
// signals after one that waits: signals never wait, so every wait ends.
VM_DEV uint64_t phase_tag(Args A, uint32_t nbar) { return (uint64_t(A->seq) << 32) | (nbar + 1u); }

// After the entry's tiles: the block's stores are complete (block barrier), and
// thread 0's agent-scope release publishes them with the flag, as a lane's
// arrival at the grid barrier does.
VM_DEV void flag_signal(Args A, uint32_t f, uint64_t tag) {
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_store(&A->flags[f], tag, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
}

// Before the entry's tiles: thread i polls flags f0 + i, f0 + i + 256, ... until
// each holds `tag`, then an agent-scope acquire and a block barrier order the
// tiles' reads after the producers' writes.  Polls give up after the barrier's
// time-out (the VM error word then ends the launch).  Returns false to abort.
VM_DEV bool flag_wait(Args A, uint32_t f0, uint32_t n, uint64_t tag) {
  __shared__ uint32_t s_fok;
  if (threadIdx.x == 0) s_fok = 1;
  __syncthreads();
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  bool ok = true;
  for (uint32_t i = threadIdx.x; ok && i < n; i += kBlock) {
    uint64_t* p = &A->flags[f0 + i];
    for (uint32_t poll = 0; __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != tag; ++poll) {
      if (barrier_timed_out(A, t0, poll)) {
        ok = false;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
  if (!ok) s_fok = 0;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  __syncthreads();
  return s_fok != 0;
}

// Record an error from a lane (first error wins) so the host can report it.
VM_DEV void raise_error(Args A, uint32_t code, uint32_t info) {
  if (threadIdx.x == 0) {
    uint32_t expect = 0;
    if (__hip_atomic_compare_exchange_strong(&A->ctl[BAR_ERROR], &expect, code, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT))
      __hip_atomic_store(&A->ctl[BAR_ERRINFO], info, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Coherent read of a control-flow condition (a value another lane may have written
// in the previous phase).  `fmt` = byte width | 0x100 for float types (the sign bit
// alone does not make a float condition true).
VM_DEV bool read_cond(const gbyte* p, uint32_t fmt) {
  const uint32_t w = fmt & 0xFF;
  uint64_t bits;
  if (w == 8) {
    bits = __hip_atomic_load((const uint64_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (fmt & 0x100) bits &= 0x7FFFFFFFFFFFFFFFull;
  } else {
    // aligned 4-byte word that holds the value (buffers are 64-byte aligned)
    const uint32_t word = __hip_atomic_load((const uint32_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    bits = w == 1 ? (word & 0xFFu) : w == 2 ? (word & 0xFFFFu) : word;
    if (fmt & 0x100) bits &= (w == 2 ? 0x7FFFull : 0x7FFFFFFFull);
  }
  return bits != 0;
}

// Coherent read of a runtime index scalar (dynamic-slice starts).
VM_DEV int64_t read_index(const gbyte* p, bool is64) {
  if (is64) return __hip_atomic_load((const int64_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return __hip_atomic_load((const int32_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace vm
