// TOP_MMA: C[g] = A[g] (MxK) . B[g] (KxN) (+ store epilogue), f32 accumulate on
// CDNA4 matrix cores (reference semantics: ops/mma.cl:362-434, epilogue 74-96).
// Task: p0 M, p1 N, p2 K, p3 G (bits 0-23) | tile-edge code (bits 24-27) |
// log2 of the K split (bits 28-31, extension), p4 A view+1, p5 B view+1, p6
// epilogue descriptor+1, p7 residual handle.
//
// K split (extension, for matmuls whose output tiles leave most lanes idle):
// with S = 2^(p3 >> 28) > 1, tile t is split t % S of output tile t / S and
// covers K slabs [k0, k1) of width ceil(K / S) rounded up to whole slabs.  It
// publishes its f32 partial tile in the task's scratch and counts its arrival;
// the split that arrives last sums the S partials in split order (deterministic,
// whichever arrives last), applies the epilogue and stores the tile.
//
// One output tile of T x T (T = 64/128/256) per tile index.  The block's four
// wave64s split it 2 x 2; each wave owns (T/2)^2 outputs as (T/64)^2 blocks of
// 32 x 32 MFMA accumulators (v_mfma_f32_32x32x16_{bf16,f16}; f32 operands use
// v_mfma_f32_32x32x2_f32).  K advances in slabs of 32 (16-bit) / 16 (f32)
// elements staged through double-buffered LDS: global -> registers for slab s+1
// while the matrix cores consume slab s.
//
// 32 x 32 accumulator layout (16 floats per lane): lane l holds column l % 32,
// rows 8*(v/4) + 4*(l/32) + v%4 for v = 0..15.  A operand: lane l holds row
// l % 32 and 8 (16-bit) or 1 (f32) K values of k-group l / 32; B operand: column
// l % 32, same K values.  Any K order works as long as A and B agree.
#pragma once
#include "tile_ew.h"
#include "vm_math.h"

namespace vm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

struct MmaDesc {
  uint32_t M, N, K, G;
  uint32_t tm, tn;          // tiles along M / N
  const gbyte* a;
  const gbyte* b;
  gbyte* d;
  const gbyte* res;         // epilogue second input
  uint32_t av, bv, epi;     // view / epilogue aux offsets + 1 (0 = none)
  uint32_t dt, adt;
  uint32_t k0, k1;          // K range of this tile (a K split's share; else 0, K)
  uint32_t S, split, ti;    // K split count, this tile's split, task index
};

// Store epilogue micro-program (mma.cl:67-96): {n, n x {kind, src, s, t}}, src 0
// = the accumulator itself, 1 = residual [G,M,N] per element, 2 = per column.
VM_TILE float apply_epilogue(Args A, uint32_t epi, const gbyte* res, uint64_t elem, uint32_t col, float v) {
  A = uargs(A);
  res = uni_ptr(res);
  const VM_K int32_t* e = aux_of(A) + (uni(epi) - 1);
  const int nm = e[0];
  for (int k = 0; k < nm; ++k) {
    const uint32_t kind = uint32_t(e[1 + 4 * k]), src = uint32_t(e[2 + 4 * k]);
    const float s = __int_as_float(e[3 + 4 * k]), t = __int_as_float(e[4 + 4 * k]);
    float y = v;
    if (src == 1) y = gcast<float>(res)[elem];
    else if (src == 2) y = gcast<float>(res)[col];
    else if (src == 3) y = s;          // constant operand (extension: relu as max(v, 0))
    v = micro(kind, v, y, s, t);
  }
  return v;
}

template <int T>
struct MmaCfg {
  static constexpr int kBM = T / 64;         // 32x32 blocks per wave along M
  static constexpr int kBN = T / 64;
};

// Epilogue kinds the lowering fuses into a matmul store (affine, GELU, a binary op
// with the residual or a per-column operand), evaluated inline by the fast path:
// a call would force the 256 live accumulator AGPRs through scratch.
// micro-ops a fast tile's store applies from registers (decoded once per tile)
constexpr int kFastEpi = 4;

VM_DEV bool epi_inline_ok(Args A, uint32_t epi) {
  if (!epi) return true;
  const VM_K int32_t* e = aux_of(A) + (epi - 1);
  const int nm = e[0];
  if (nm > kFastEpi) return false;
  for (int k = 0; k < nm; ++k) {
    const uint32_t kind = uint32_t(e[1 + 4 * k]);
    if (!(kind == SUB_AFFINE || kind == SUB_GELU || kind == SUB_COPY || kind <= SUB_DIV || kind == SUB_MAX ||
          kind == SUB_MIN))
      return false;
  }
  return true;
}

// epi_inline on four values with one dispatch on the (uniform) kind
VM_DEV v4f epi_inline4(uint32_t kind, v4f x, v4f y, float s, float t) {
  switch (kind) {
    case SUB_AFFINE: return v4f_make(fmaf(x.x, s, t), fmaf(x.y, s, t), fmaf(x.z, s, t), fmaf(x.w, s, t));
    case SUB_GELU: return v4f_make(gelu(x.x), gelu(x.y), gelu(x.z), gelu(x.w));
    case SUB_ADD: return v4f_make(x.x + y.x, x.y + y.y, x.z + y.z, x.w + y.w);
    case SUB_MUL: return v4f_make(x.x * y.x, x.y * y.y, x.z * y.z, x.w * y.w);
    case SUB_SUB: return v4f_make(x.x - y.x, x.y - y.y, x.z - y.z, x.w - y.w);
    case SUB_DIV: return v4f_make(x.x / y.x, x.y / y.y, x.z / y.z, x.w / y.w);
    case SUB_MAX: return v4f_make(fmaxf(x.x, y.x), fmaxf(x.y, y.y), fmaxf(x.z, y.z), fmaxf(x.w, y.w));
    case SUB_MIN: return v4f_make(fminf(x.x, y.x), fminf(x.y, y.y), fminf(x.z, y.z), fminf(x.w, y.w));
    default: return x;
  }
}

VM_DEV float epi_inline(uint32_t kind, float x, float y, float s, float t) {
  switch (kind) {
    case SUB_AFFINE: return fmaf(x, s, t);
    case SUB_GELU: return gelu(x);
    case SUB_ADD: return x + y;
    case SUB_MUL: return x * y;
    case SUB_SUB: return x - y;
    case SUB_DIV: return x / y;
    case SUB_MAX: return fmaxf(x, y);
    case SUB_MIN: return fminf(x, y);
    default: return x;
  }
}

// One 32 x 32 block through the epilogue program, element by element (the
// general path for epilogue kinds the store cannot evaluate inline).  A function
// of its own, taking the block by value: the caller's loop over blocks then
// unrolls, so its accumulators stay in registers.
VM_TILE void store_block_epi(Args A, uint32_t epi, const gbyte* res, gbyte* d, uint32_t dt, uint32_t M, uint32_t N,
                             f32x16 blk, uint32_t g, uint32_t rbase, uint32_t col) {
#pragma unroll 1
  for (int v = 0; v < 16; ++v) {
    const uint32_t row = rbase + 8 * (v >> 2) + (v & 3);
    if (row < M && col < N) {
      const uint64_t elem = (uint64_t(g) * M + row) * N + col;
      store_f(d, dt, elem, apply_epilogue(A, epi, res, elem, col, blk[v]));
    }
  }
}

template <int T>
VM_DEV void store_acc(Args A, const MmaDesc& D, const f32x16 (&acc)[MmaCfg<T>::kBM][MmaCfg<T>::kBN], uint32_t g,
                      uint32_t m0, uint32_t n0) {
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t wm = wave >> 1, wn = wave & 1;
  // 64-wide tiles (the small matmuls' tile, one 32 x 32 block per wave): an
  // epilogue of the inline kinds (affine, GELU, binary ops; the fast paths' set)
  // gets its operands loaded before the first is used -- the column value once,
  // the block's 16 residual values together (indices clamped into the output,
  // results past it not stored) -- so the store costs one memory round trip, not
  // one per element (config 1's bias + relu matmuls).  Larger tiles and other
  // kinds evaluate per element: unrolled over four or more blocks, the inline
  // evaluation pushes the accumulators of a 128-wide tile into scratch.
  const bool inl = T == 64 && D.epi && epi_inline_ok(A, D.epi);
  const VM_K int32_t* e = aux_of(A) + (D.epi ? D.epi - 1 : 0);
  const int nm = inl ? e[0] : 0;
  bool need_res = false, need_col = false;
  for (int k = 0; k < nm; ++k) {
    need_res |= e[2 + 4 * k] == 1;
    need_col |= e[2 + 4 * k] == 2;
  }
  const VM_G float* res = (const VM_G float*)D.res;
#pragma unroll
  for (int bm = 0; bm < MmaCfg<T>::kBM; ++bm) {
#pragma unroll
    for (int bn = 0; bn < MmaCfg<T>::kBN; ++bn) {
      const uint32_t col = n0 + wn * (T / 2) + bn * 32 + (lane & 31);
      const uint32_t rbase = m0 + wm * (T / 2) + bm * 32 + 4 * (lane >> 5);
      if (T == 64 && inl) {
        const uint32_t cc = min(col, D.N - 1);
        const float yc = need_col ? res[cc] : 0.0f;
        float yr[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const uint32_t row = min(rbase + 8 * (v >> 2) + (v & 3), D.M - 1);
          yr[v] = need_res ? res[(uint64_t(g) * D.M + row) * D.N + cc] : 0.0f;
        }
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const uint32_t row = rbase + 8 * (v >> 2) + (v & 3);
          float x = acc[bm][bn][v];
          for (int k = 0; k < nm; ++k) {
            const uint32_t kind = uint32_t(e[1 + 4 * k]), src = uint32_t(e[2 + 4 * k]);
            const float sv = __int_as_float(e[3 + 4 * k]), tv = __int_as_float(e[4 + 4 * k]);
            x = epi_inline(kind, x, src == 1 ? yr[v] : src == 2 ? yc : src == 3 ? sv : x, sv, tv);
          }
          if (row < D.M && col < D.N) store_f(D.d, D.dt, (uint64_t(g) * D.M + row) * D.N + col, x);
        }
      } else if (D.epi) {
        store_block_epi(A, D.epi, D.res, D.d, D.dt, D.M, D.N, acc[bm][bn], g, rbase, col);
      } else {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const uint32_t row = rbase + 8 * (v >> 2) + (v & 3);
          if (row < D.M && col < D.N) store_f(D.d, D.dt, (uint64_t(g) * D.M + row) * D.N + col, acc[bm][bn][v]);
        }
      }
    }
  }
}

__shared__ uint32_t vm_mma_last;       // this lane's split arrived last (K-split combine)

// Store of a general tile: the tile itself, or (K split) its f32 partial.  A
// partial is written in register order, 16 bytes per thread and step (values
// 4q .. 4q + 3 of thread x at [(tile S + split) NQ + q] kBlock + x, NQ = T^2 /
// (4 kBlock)), coalesced.  Each thread waits for its own stores to complete, the
// block barrier orders them before thread 0's arrival, an agent-scope
// acquire-release add on the tile's counter: its release writes this XCD's L2
// back (the partial included), its acquire (in the last arriver) invalidates the
// reader's caches, and the block barrier after it orders the other threads'
// reads after the invalidation -- the grid barrier's publish / acquire pattern.
// The last arriver resets the counter (the next run of the task is ordered after
// this one by a grid barrier) and sums partials 0 .. S-1 in that order, loading
// several splits' partials before the first add (one memory round trip per
// batch, not per value).
template <int T>
VM_DEV void mma_store(Args A, const MmaDesc& D, f32x16 (&acc)[MmaCfg<T>::kBM][MmaCfg<T>::kBN], uint32_t tile,
                      uint32_t g, uint32_t m0, uint32_t n0) {
  if (D.S <= 1) return store_acc<T>(A, D, acc, g, m0, n0);
  using C = MmaCfg<T>;
  constexpr uint32_t NQ = C::kBM * C::kBN * 4;             // float4 steps per thread
  constexpr uint32_t B = NQ <= 4 ? 8 : NQ <= 16 ? 2 : 1;   // splits per load batch (<= 32 float4)
  v4f* sp = reinterpret_cast<v4f*>(A->scratch + A->task_scratch[D.ti]);
  const uint64_t nbase = uint64_t(D.tm) * D.tn * D.G;
  uint32_t* arrivals = reinterpret_cast<uint32_t*>(sp + nbase * D.S * NQ * kBlock);
  v4f* mine = sp + (uint64_t(tile) * D.S + D.split) * NQ * kBlock + threadIdx.x;
#pragma unroll
  for (int bm = 0; bm < C::kBM; ++bm)
#pragma unroll
    for (int bn = 0; bn < C::kBN; ++bn)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x16& x = acc[bm][bn];
        mine[((bm * C::kBN + bn) * 4 + q) * kBlock] = v4f_make(x[4 * q], x[4 * q + 1], x[4 * q + 2], x[4 * q + 3]);
      }
  __builtin_amdgcn_s_waitcnt(0x0F70);                 // vmcnt(0): this thread's stores are done
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t before = __hip_atomic_fetch_add(arrivals + tile, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = before == D.S - 1;
    if (last) __hip_atomic_store(arrivals + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    vm_mma_last = last;
  }
  __syncthreads();
  if (!vm_mma_last) return;
  const v4f* hp = sp + uint64_t(tile) * D.S * NQ * kBlock + threadIdx.x;
  for (uint32_t s0 = 0; s0 < D.S; s0 += B) {
    v4f part[B][NQ];
#pragma unroll
    for (uint32_t u = 0; u < B; ++u)             // past S: re-read the last split (not added)
#pragma unroll
      for (uint32_t q = 0; q < NQ; ++q) part[u][q] = hp[(uint64_t(min(s0 + u, D.S - 1)) * NQ + q) * kBlock];
#pragma unroll
    for (uint32_t u = 0; u < B; ++u)
      if (s0 + u < D.S) {
#pragma unroll
        for (int bm = 0; bm < C::kBM; ++bm)
#pragma unroll
          for (int bn = 0; bn < C::kBN; ++bn)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const v4f y = part[u][(bm * C::kBN + bn) * 4 + q];
              f32x16& x = acc[bm][bn];
              if (s0 + u == 0) {
                x[4 * q] = y.x; x[4 * q + 1] = y.y; x[4 * q + 2] = y.z; x[4 * q + 3] = y.w;
              } else {
                x[4 * q] += y.x; x[4 * q + 1] += y.y; x[4 * q + 2] += y.z; x[4 * q + 3] += y.w;
              }
            }
      }
  }
  store_acc<T>(A, D, acc, g, m0, n0);
}

// Operand element (g, m, k) with a view or an unaligned row: 8 (16-bit) or 4
// (f32) consecutive logical elements starting at `lin`, the first `nvalid` real.
VM_TILE v4u gather_chunk(Args A, const gbyte* base, uint32_t view, uint64_t lin, uint32_t nvalid, uint32_t esz) {
  A = uargs(A);
  base = uni_ptr(base);
  const VM_K int32_t* aux = aux_of(A);
  uint32_t w[4] = {0, 0, 0, 0};
  const uint32_t n = esz == 2 ? 8u : 4u;
  for (uint32_t q = 0; q < n && q < nvalid; ++q) {
    const uint64_t idx = view ? uint64_t(view_index(aux, view - 1, lin + q)) : lin + q;
    if (esz == 2) w[q >> 1] |= uint32_t(gcast<uint16_t>(base)[idx]) << (16 * (q & 1));
    else w[q] = gcast<uint32_t>(base)[idx];
  }
  return v4u_make(w[0], w[1], w[2], w[3]);
}

// ---------------------------------------------------------------------------------
// 16-bit operands (bf16 / f16)
// ---------------------------------------------------------------------------------
constexpr int kBK16 = 32;                 // K-split granularity (elements)
// K slab of a general tile: every tile edge stages T * kBK = 8192 elements per
// operand and slab (four 16-byte loads per thread), so the small tiles of
// skinny products (a few hundred rows, prefill-style) take one memory round
// trip, LDS store and block barrier per 128 k rather than per 32.  With 32-deep
// slabs a 64 x 64 tile of a 512 x 768 x 3072 bf16 product took 93 us.
template <int T>
struct Lds16 {
  static constexpr int kBK = T == 64 ? 128 : T == 128 ? 64 : 32;
  static constexpr int kLdA = kBK + 8;    // A row stride (elements): 16-byte aligned, padded against bank conflicts
  // B row stride (elements): 8-byte aligned rows, (T + 32) / 2 = 16 or 48 dwords
  // mod 64, so the four rows x two 16-column halves a half wave's transposed
  // read touches fall on eight distinct 8-bank groups
  static constexpr int kLdB = T + 32;
  static constexpr int kA = T * kLdA;     // elements
  static constexpr int kB = kBK * kLdB;
  static constexpr int kBuf = kA + kB;
  static constexpr int kBytes = 2 * kBuf * 2;   // double buffered, 2 bytes each
};

// How a general tile reads one operand's chunks of `per` consecutive logical
// elements (8 16-bit or 4 f32, one 16-byte access): mode 0, straight from the
// row-major operand (no view, rows a multiple of `per`, 16-byte aligned base);
// mode 1, from the view's index of the chunk start (a view of rank <=
// kViewRank whose innermost dim is contiguous, with that extent, the other
// strides and the offset multiples of `per`, so each chunk is one aligned run:
// the lowered decoder's attention output read as [tokens, heads * head_dim]);
// mode 2, element by element (anything else).  Mode 1 (taken for A only) took
// the lowered C5 prefill's output projection from 151 to 40 us per entry.
struct OperandRead {
  uint32_t mode;
  ViewMap map;
};
VM_DEV OperandRead operand_read(const VM_K int32_t* aux, uint32_t view, const gbyte* base, uint32_t row_len,
                                uint64_t n_elems, uint32_t per) {
  OperandRead r;
  r.map = view_map(aux, 0);
  const bool aligned = (uintptr_t(base) & 15) == 0 && row_len % per == 0;
  if (!view) {
    r.mode = aligned ? 0u : 2u;
    return r;
  }
  r.map = view_map(aux, view);
  bool ok = aligned && n_elems <= 0xFFFFFFFFull && r.map.rank >= 1 && r.map.rank <= kViewRank &&
            r.map.stride[0] == 1 && r.map.dim[0].d % per == 0 && r.map.off % per == 0;
#pragma unroll
  for (int k = 1; k < kViewRank; ++k)
    if (k < r.map.rank && r.map.stride[k] % int32_t(per) != 0) ok = false;
  r.mode = ok ? 1u : 2u;
  return r;
}

template <int T>
struct Stage16 {
  // A: T rows x kBK k in chunks of 8 elements; B: kBK rows x T cols, the same count.
  static constexpr int kBK = Lds16<T>::kBK, kRowChunks = kBK / 8;
  static constexpr int kChunks = T * kRowChunks / kBlock;
  v4u ra[kChunks];
  v4u rb[kChunks];

  VM_DEV void load(Args A, const MmaDesc& D, uint32_t g, uint32_t m0, uint32_t n0, uint32_t k0, const OperandRead& ar,
                   const OperandRead& br) {
    const VM_K int32_t* aux = aux_of(A);
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
      const uint32_t c = threadIdx.x + j * kBlock;
      const uint32_t m = m0 + c / kRowChunks, k = k0 + (c % kRowChunks) * 8;
      const uint64_t lin = (uint64_t(g) * D.M + m) * D.K + k;
      const bool in = m < D.M && k < D.k1;
      if (ar.mode != 2)   // modes 0 and 1: view_at is the identity without a view
        ra[j] = in ? gld((const VM_G v4u*)(gcast<uint16_t>(D.a) + (ar.mode ? view_at(ar.map, aux, D.av, uint32_t(lin)) : lin)))
                   : v4u_make(0, 0, 0, 0);
      else
        ra[j] = in ? gather_chunk(A, D.a, D.av, lin, D.k1 - k, 2) : v4u_make(0, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
      const uint32_t c = threadIdx.x + j * kBlock;
      const uint32_t k = k0 + c / (T / 8), n = n0 + (c % (T / 8)) * 8;
      const uint64_t lin = (uint64_t(g) * D.K + k) * D.N + n;
      const bool in = k < D.k1 && n < D.N;
      if (br.mode == 0)
        rb[j] = in ? gld((const VM_G v4u*)(gcast<uint16_t>(D.b) + lin)) : v4u_make(0, 0, 0, 0);
      else
        rb[j] = in ? gather_chunk(A, D.b, D.bv, lin, D.N - n, 2) : v4u_make(0, 0, 0, 0);
    }
  }
  VM_DEV void store(uint16_t* lds) const {
    uint16_t* la = lds;
    uint16_t* lb = lds + Lds16<T>::kA;
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
      const uint32_t c = threadIdx.x + j * kBlock;
      *reinterpret_cast<v4u*>(la + (c / kRowChunks) * Lds16<T>::kLdA + (c % kRowChunks) * 8) = ra[j];
    }
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
      const uint32_t c = threadIdx.x + j * kBlock;
      v2u* p = reinterpret_cast<v2u*>(lb + (c / (T / 8)) * Lds16<T>::kLdB + (c % (T / 8)) * 8);
      p[0] = v2u_make(rb[j].x, rb[j].y);
      p[1] = v2u_make(rb[j].z, rb[j].w);
    }
  }
};

typedef __attribute__((address_space(3))) uint8_t lds_u8;
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
typedef __attribute__((address_space(3))) u16x8 lds_u16x8;

template <bool BF16>
VM_DEV f32x16 mfma16(const u16x8& a, const u16x8& b, const f32x16& c) {
  if constexpr (BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
}

// The descriptor arrives through a pointer; every field is wave-uniform.
VM_DEV MmaDesc load_desc(const MmaDesc* p) {
  MmaDesc D;
  D.M = uni(p->M);
  D.N = uni(p->N);
  D.K = uni(p->K);
  D.G = uni(p->G);
  D.tm = uni(p->tm);
  D.tn = uni(p->tn);
  D.a = uni_ptr(p->a);
  D.b = uni_ptr(p->b);
  D.d = uni_ptr(p->d);
  D.res = uni_ptr(p->res);
  D.av = uni(p->av);
  D.bv = uni(p->bv);
  D.epi = uni(p->epi);
  D.dt = uni(p->dt);
  D.adt = uni(p->adt);
  D.k0 = uni(p->k0);
  D.k1 = uni(p->k1);
  D.S = uni(p->S);
  D.split = uni(p->split);
  D.ti = uni(p->ti);
  return D;
}

VM_DEV void tile_origin(const MmaDesc& D, uint32_t tile, uint32_t T, uint32_t* g, uint32_t* m0, uint32_t* n0) {
  const uint32_t per = D.tm * D.tn;
  *g = tile / per;
  const uint32_t loc = tile % per;
  *m0 = (loc / D.tn) * T;
  *n0 = (loc % D.tn) * T;
}

template <int T, bool BF16>
VM_TILE void mma_tile16(Args A, const MmaDesc* Dp, uint32_t tile) {
  A = uargs(A);
  const MmaDesc D = load_desc(Dp);
  uint16_t* lds = lds_ptr<uint16_t>();
  using C = MmaCfg<T>;
  uint32_t g, m0, n0;
  tile_origin(D, uni(tile), T, &g, &m0, &n0);
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t wm = wave >> 1, wn = wave & 1;
  const OperandRead ar = operand_read(aux_of(A), D.av, D.a, D.K, uint64_t(D.G) * D.M * D.K, 8);
  // B (the weight, in every program seen) has no mode 1: viewed weights are
  // transposes, whose innermost dim is not contiguous
  OperandRead br = operand_read(aux_of(A), D.bv, D.b, D.N, uint64_t(D.G) * D.K * D.N, 8);
  if (br.mode == 1) br.mode = 2;

  f32x16 acc[C::kBM][C::kBN];
#pragma unroll
  for (int i = 0; i < C::kBM; ++i)
#pragma unroll
    for (int j = 0; j < C::kBN; ++j) acc[i][j] = f32x16{};

  constexpr int kBK = Lds16<T>::kBK;
  const uint32_t nk = (D.k1 - D.k0 + kBK - 1) / kBK;
  Stage16<T> st;
  st.load(A, D, g, m0, n0, D.k0, ar, br);
  __syncthreads();                      // previous user of the LDS is done
  st.store(lds);
  __syncthreads();
  for (uint32_t ks = 0; ks < nk; ++ks) {
    const uint16_t* cur = lds + (ks & 1) * Lds16<T>::kBuf;
    if (ks + 1 < nk) st.load(A, D, g, m0, n0, D.k0 + (ks + 1) * kBK, ar, br);
    const uint16_t* la = cur;
    const uint16_t* lb = cur + Lds16<T>::kA;
#pragma unroll
    for (int kk = 0; kk < kBK; kk += 16) {
      const uint32_t kq = kk + (lane >> 5) * 8;
      u16x8 af[C::kBM], bf[C::kBN];
#pragma unroll
      for (int bm = 0; bm < C::kBM; ++bm)
        af[bm] = *reinterpret_cast<const u16x8*>(la + (wm * (T / 2) + bm * 32 + (lane & 31)) * Lds16<T>::kLdA + kq);
      // B fragment: column lane % 32, k = kq .. kq + 7, as two ds_read_b64_tr_b16.
      // In each group of 16 lanes, lane 4e + q points at row kq + e (+ 4),
      // columns c0 + 4q .. + 3 (c0: the group's 16 columns); the transposed read
      // gives lane i column c0 + i at the four rows.  (Eight 16-bit LDS reads
      // per fragment made the LDS the bound of the small tiles.)
#pragma unroll
      for (int bn = 0; bn < C::kBN; ++bn) {
        const uint32_t j = lane & 15;
        const uint32_t col = wn * (T / 2) + bn * 32 + (lane & 16) + 4 * (j & 3);
        const uint16_t* p = lb + (kq + (j >> 2)) * Lds16<T>::kLdB + col;
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p);
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p + 4 * Lds16<T>::kLdB));
        bf[bn] = __builtin_bit_cast(u16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      }
#pragma unroll
      for (int bm = 0; bm < C::kBM; ++bm)
#pragma unroll
        for (int bn = 0; bn < C::kBN; ++bn) acc[bm][bn] = mfma16<BF16>(af[bm], bf[bn], acc[bm][bn]);
    }
    if (ks + 1 < nk) st.store(lds + ((ks + 1) & 1) * Lds16<T>::kBuf);
    __syncthreads();
  }
  mma_store<T>(A, D, acc, uni(tile), g, m0, n0);
}

// ---------------------------------------------------------------------------------
// 16-bit fast path: 256 x 256 output tiles, K slabs of 64
// ---------------------------------------------------------------------------------
// For unviewed row-major operands with M and N multiples of 256 and K a multiple of
// 64 (the big square GEMMs).  Each wave owns a 128 x 128 quadrant as 4 x 4 blocks
// of 32 x 32 accumulators (all 256 AGPRs).  Both operand slabs go from global
// memory straight into LDS (global_load_lds_dwordx4, no register staging), two
// stages of 64 KiB:
//   A slab, 256 rows x 64 k: rows of 128 B, dense.  The eight 16-byte k chunks of
//     row r sit at slots chunk ^ aswz(r), so that a fragment's ds_read_b128 hits
//     distinct bank groups both in any 16 consecutive lanes (16 rows, one chunk)
//     and in lanes 0-7 with 32-39 (8 rows, chunks c and c + 1).
//   B slab, 64 k rows x 256 n, as B is laid out (rows of 512 B).  The 32 chunks of
//     row k sit at slots chunk ^ 4 (k & 3).  A fragment (8 k values of one column
//     per lane) is read with two ds_read_b64_tr_b16: in each group of 16 lanes,
//     lane 4e + q points at row k0 + e, columns n0 + 4q .. +3, and the transposed
//     read gives lane i column n0 + i at rows k0 .. k0 + 3.  The 32 lanes of a half
//     wave read four rows, 64 B each, whose swizzled slots cover the 64 banks once.
constexpr int kFBK = 64;                                // K slab (elements)
constexpr uint32_t kFStage = 65536;                     // bytes per stage: A 32 KiB + B 32 KiB
constexpr uint32_t kFStageB = 32768;                    // B's offset in a stage
constexpr int kFStoreBytes = 128 * (256 + 4) * 4;       // store_fast's staging tile
constexpr int kFastLdsBytes = 2 * int(kFStage) > kFStoreBytes ? 2 * int(kFStage) : kFStoreBytes;

// A-slab slot swizzle of row r: ((r >> 1) & 3) << 1 | ((r >> 3) & 1).  Rows of one
// parity among 16 consecutive rows get 8 distinct values; among 8 consecutive
// rows (aligned), 4 values whose halves (bits 1-2) differ, so chunks c and c ^ 1
// of those rows land on 8 distinct slots.  A 128-byte row spans half the banks,
// so rows of opposite parity never meet.
VM_DEV uint32_t aswz(uint32_t r) { return (((r >> 1) & 3) << 1) | ((r >> 3) & 1); }


// One 16-byte global -> LDS transfer per lane: lane l of the wave writes LDS bytes
// [lds + 16 l, +16) with base[voff].  Issued from asm: the compiler, which cannot
// tell which LDS bytes the transfer writes, would otherwise wait for it before
// every LDS read.  The tile waits for its transfers itself (vmcnt) before the
// block barrier that publishes a stage.  The transfer takes its LDS address from
// M0, which the compiler reserves and does not let an asm statement declare as
// clobbered, so the statement leaves M0 as it found it: it saves M0 in an SGPR
// of its own, loads the address, waits the one state the M0 write needs before
// the transfer reads it, issues the transfer (which takes M0 at issue) and puts
// the saved value back.
VM_DEV void dma16(const gbyte* base, uint32_t voff, uint32_t lds) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %2, %3\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(lds), "v"(voff), "s"(base)
      : "memory");
}
VM_DEV void wait_vm0() { __builtin_amdgcn_s_waitcnt(0x0F70); }    // s_waitcnt vmcnt(0)
VM_DEV void wait_vm8() { __builtin_amdgcn_s_waitcnt(0x0F78); }    // s_waitcnt vmcnt(8)

// The transfers of one slab: 8 rounds for A, 8 for B, one dwordx4 per thread each.
// A round j fills stage bytes [4096 j, +4096): wave w rows 32 j + 8 w + l / 8; B
// round j fills [32768 + 4096 j, +4096): wave w k rows 8 j + 2 w + l / 32.  Each
// lane fetches the chunk whose swizzled slot is its own 16 bytes.
struct FastDma {
  uint32_t oa, ob;        // per-lane byte offsets of round 0 in the A and B slabs
  uint32_t wo;            // the wave's 1 KiB within a round (wave-uniform)
  VM_DEV void init(uint32_t K, uint32_t N) {
    const uint32_t l = threadIdx.x & 63, w = threadIdx.x >> 6;
    const uint32_t ra = 8 * w + (l >> 3);
    oa = ra * K * 2 + (((l & 7) ^ aswz(ra)) * 16);
    const uint32_t rb = 2 * w + (l >> 5);
    ob = rb * N * 2 + (((l & 31) ^ (4 * (rb & 3))) * 16);
    wo = uni(1024 * w);
  }
  // round r of 16 (A rounds 0-7, B rounds 8-15) of the slab at a (A[m0, k0]) and
  // b (B[k0, n0]) into the stage at LDS address st
  VM_DEV void round(const gbyte* a, const gbyte* b, uint32_t K, uint32_t N, uint32_t st, int r) const {
    if (r < 8) dma16(a + uint64_t(r) * 64 * K, oa, st + wo + 4096 * r);
    else dma16(b + uint64_t(r - 8) * 16 * N, ob, st + kFStageB + wo + 4096 * (r - 8));
  }
};

// The same transfers for a ragged tile (M or N not a multiple of 256, or K not a
// multiple of 64; K and N multiples of 8): every address is clamped into the
// operand -- A rows past M re-read row M - 1, B columns past N the last 8, k past
// K the last 8 columns of A / the last row of B -- so no transfer leaves the
// buffers, and each lane's LDS slot is where the aligned tile puts it.  Rows and
// columns past M / N are computed but not stored; the k past K are zeroed in LDS
// (RaggedDma::zero) before the stage is published, in both operands, so that
// they add 0 whatever the clamped data holds.
struct RaggedDma {
  uint32_t ra, ca, rb, cb;  // per lane: A row within a round and its k chunk; B k row within a round and n chunk
  uint32_t wo;
  const gbyte* a;           // A[g, m0, 0]
  const gbyte* b;           // B[g, 0, n0]
  uint32_t M, N, K, m0, n0;
  VM_DEV void init(const gbyte* a_, const gbyte* b_, uint32_t M_, uint32_t N_, uint32_t K_, uint32_t m0_, uint32_t n0_) {
    const uint32_t l = threadIdx.x & 63, w = threadIdx.x >> 6;
    ra = 8 * w + (l >> 3);
    ca = (l & 7) ^ aswz(ra);
    rb = 2 * w + (l >> 5);
    cb = (l & 31) ^ (4 * (rb & 3));
    wo = uni(1024 * w);
    a = a_;
    b = b_;
    M = M_;
    N = N_;
    K = K_;
    m0 = m0_;
    n0 = n0_;
  }
  // round r of slab s into the stage at st
  VM_DEV void round(uint32_t s, uint32_t st, int r) const {
    if (r < 8) {
      const uint32_t row = min(m0 + 32 * uint32_t(r) + ra, M - 1) - m0;
      const uint32_t k = min(s * kFBK + 8 * ca, K - 8);
      dma16(a, row * K * 2 + k * 2, st + wo + 4096 * r);
    } else {
      // the slab's rows from a scalar base, so the lane offset stays below 64 rows
      const uint32_t k = min(s * kFBK + 8 * uint32_t(r - 8) + rb, K - 1) - s * kFBK;
      const uint32_t n = min(n0 + 8 * cb, N - 8) - n0;
      dma16(b + uint64_t(s) * kFBK * N * 2, k * N * 2 + n * 2, st + kFStageB + wo + 4096 * (r - 8));
    }
  }
  // zero this lane's slots that hold k >= K of the last slab s (after the lane's
  // transfers into st have landed, before the block barrier that publishes st)
  VM_DEV void zero(uint32_t s, uint32_t st) const {
    const uint32_t kv = K - s * kFBK;                    // valid k of the slab, a multiple of 8
    typedef __attribute__((address_space(3))) v4u lds_v4u;
    const uint32_t l = threadIdx.x & 63;
    if (8 * ca >= kv) {
#pragma unroll
      for (int r = 0; r < 8; ++r) *(lds_v4u*)uintptr_t(st + wo + 4096 * r + 16 * l) = v4u_make(0, 0, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < 8; ++r)
      if (8 * uint32_t(r) + rb >= kv)
        *(lds_v4u*)uintptr_t(st + kFStageB + wo + 4096 * r + 16 * l) = v4u_make(0, 0, 0, 0);
  }
};

// Tile index -> origin.  When the tile grid splits evenly over the 8 XCDs, tile t
// (which the scheduler places on lane t, and the dispatcher on XCD t % 8) is
// mapped so that each XCD owns a compact band of 4-row groups: its tiles share A
// and B panels in that XCD's L2.  Any bijection is correct; this one is faster.
VM_DEV void fast_origin(const MmaDesc& D, uint32_t tile, uint32_t* g, uint32_t* m0, uint32_t* n0) {
  const uint32_t per = D.tm * D.tn;
  *g = tile / per;
  uint32_t loc = tile % per;
  if (per % 8 == 0 && D.tm % 4 == 0) {
    loc = (loc % 8) * (per / 8) + loc / 8;
    const uint32_t grp = loc / (4 * D.tn), in = loc % (4 * D.tn);
    *m0 = (grp * 4 + in % 4) * 256;
    *n0 = (in / 4) * 256;
  } else {
    *m0 = (loc / D.tn) * 256;
    *n0 = (loc % D.tn) * 256;
  }
}

// Tile store through LDS: the accumulators of half the tile (rows 0-63 and
// 128-191 of every wave's quadrant) are scattered into a 128 x 256 f32 staging
// tile, then the whole block writes full rows with 16-byte (f32) or 8-byte
// (16-bit) stores, applying the epilogue on the way.  No call is made while the
// accumulators are live.
template <bool F32, bool RAG>
VM_DEV void store_fast(Args A, const MmaDesc& D, const f32x16 (&acc)[4][4], uint32_t g, uint32_t m0, uint32_t n0) {
  constexpr int LD = 256 + 4;
  float* st = lds_ptr<float>();
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t wm = wave >> 1, wn = wave & 1;
  const uint64_t tile0 = (uint64_t(g) * D.M + m0) * D.N + n0;
  gbyte* d = D.d + tile0 * (F32 ? 4 : 2);
  const bool bf = D.dt == DT_BF16;
  const VM_K int32_t* e = aux_of(A) + (D.epi ? D.epi - 1 : 0);
  const int nm = D.epi ? uni(e[0]) : 0;                   // <= kFastEpi (epi_inline_ok)
  // the micro-ops, decoded once: scalar registers, not a descriptor read and a
  // branch per component in every step (bias + GELU on 512x2304x768 bf16: the
  // store loop held 2561 branches)
  uint32_t ek[kFastEpi], esrc[kFastEpi];
  float es4[kFastEpi], et4[kFastEpi];
  bool src1 = false, src2 = false;
#pragma unroll
  for (int k = 0; k < kFastEpi; ++k) {
    ek[k] = esrc[k] = 0;
    es4[k] = et4[k] = 0.0f;
    if (k < nm) {                                         // uniform: never reads past the descriptor
      ek[k] = uni(e[1 + 4 * k]);
      esrc[k] = uni(e[2 + 4 * k]);
      es4[k] = __int_as_float(uni(e[3 + 4 * k]));
      et4[k] = __int_as_float(uni(e[4 + 4 * k]));
      src1 |= esrc[k] == 1;
      src2 |= esrc[k] == 2;
    }
  }
  // Epilogue operands are read ahead of the stores: loads and stores share one
  // in-order counter, so a load issued after a store makes its wait drain the
  // store too (read inside the store loop, a bias took 512x2304x768 bf16 from
  // 31.5 to 57.4 us).  The per-column operand (src 2) covers the same 4 columns
  // of a thread in every step, so it is read once; the per-element one (src 1)
  // is read one step ahead.  Ragged edges read clamped (valid) addresses; their
  // results are not stored.  The step loop stays rolled, one copy per half:
  // unrolled with the micro-op dispatch in every copy, the tile grew past the
  // 128 KiB reach of a short branch, and the compiler's long branches reused the
  // return address registers (s[30:31]) of this leaf without saving them.
  const uint32_t cth = (threadIdx.x & 63) * 4;                       // the thread's columns in every step
  v4f ycol = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  if (src2) ycol = *(const VM_G v4f*)(D.res + uint64_t(RAG ? min(n0 + cth, D.N - 4) : n0 + cth) * 4);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    __syncthreads();
#pragma unroll
    for (int ii = 0; ii < 2; ++ii)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t c = wn * 128 + j * 32 + (lane & 31);
        const uint32_t r0 = wm * 64 + ii * 32 + 4 * (lane >> 5);
#pragma unroll
        for (int v = 0; v < 16; ++v) st[(r0 + 8 * (v >> 2) + (v & 3)) * LD + c] = acc[2 * h + ii][j][v];
      }
    __syncthreads();
    // step it: idx = it kBlock + threadIdx.x -> row (rs >> 6) 128 + h 64 + rs % 64, columns c .. c + 3;
    // the residual (src 1) of step it + 1 is read before step it's store
    auto res_at = [&](uint32_t it) -> v4f {
      const uint32_t rs = (it * kBlock + threadIdx.x) >> 6;
      uint32_t row = (rs >> 6) * 128 + h * 64 + (rs & 63), col = cth;
      if constexpr (RAG) {
        row = min(row, D.M - 1 - m0);
        col = min(col, D.N - 4 - n0);
      }
      return *(const VM_G v4f*)(D.res + (tile0 + uint64_t(row) * D.N + col) * 4);
    };
    if (nm == 0) {
      // no epilogue: the plain store (C3)
#pragma unroll 4
      for (uint32_t it = 0; it < 32; ++it) {
        const uint32_t idx = it * kBlock + threadIdx.x;
        const uint32_t rs = idx >> 6, c = (idx & 63) * 4;
        const uint32_t row = (rs >> 6) * 128 + h * 64 + (rs & 63);
        if constexpr (RAG) {
          if (m0 + row >= D.M || n0 + c >= D.N) continue;
        }
        const v4f x = *reinterpret_cast<const v4f*>(st + rs * LD + c);
        const uint32_t off = row * D.N + c;
        if constexpr (F32) {
          *(VM_G v4f*)(d + off * 4u) = x;
        } else {
          const uint32_t lo = bf ? pack_bf16x2(x.x, x.y) : (uint32_t(f32_to_f16(x.x)) | uint32_t(f32_to_f16(x.y)) << 16);
          const uint32_t hi = bf ? pack_bf16x2(x.z, x.w) : (uint32_t(f32_to_f16(x.z)) | uint32_t(f32_to_f16(x.w)) << 16);
          *(VM_G v2u*)(d + off * 2u) = v2u_make(lo, hi);
        }
      }
      continue;
    }
    v4f ynext = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    if (src1) ynext = res_at(0);
#pragma unroll 2
    for (uint32_t it = 0; it < 32; ++it) {
      const v4f ycur = ynext;
      if (src1 && it + 1 < 32) ynext = res_at(it + 1);
      const uint32_t idx = it * kBlock + threadIdx.x;
      const uint32_t rs = idx >> 6, c = (idx & 63) * 4;
      const uint32_t row = (rs >> 6) * 128 + h * 64 + (rs & 63);
      if constexpr (RAG) {
        if (m0 + row >= D.M || n0 + c >= D.N) continue;   // N % 4 == 0: 4 columns all in or all out
      }
      v4f x = *reinterpret_cast<const v4f*>(st + rs * LD + c);
      const uint32_t off = row * D.N + c;
#pragma unroll
      for (int k = 0; k < kFastEpi; ++k) {
        if (k < nm) {
          const v4f y = esrc[k] == 1 ? ycur : esrc[k] == 2 ? ycol
                      : esrc[k] == 3 ? v4f_make(es4[k], es4[k], es4[k], es4[k]) : x;
          x = epi_inline4(ek[k], x, y, es4[k], et4[k]);
        }
      }
      if constexpr (F32) {
        *(VM_G v4f*)(d + off * 4u) = x;
      } else {
        const uint32_t lo = bf ? pack_bf16x2(x.x, x.y) : (uint32_t(f32_to_f16(x.x)) | uint32_t(f32_to_f16(x.y)) << 16);
        const uint32_t hi = bf ? pack_bf16x2(x.z, x.w) : (uint32_t(f32_to_f16(x.z)) | uint32_t(f32_to_f16(x.w)) << 16);
        *(VM_G v2u*)(d + off * 2u) = v2u_make(lo, hi);
      }
    }
  }
}

template <bool BF16, bool RAG>
VM_LEAF void mma_tile16_fast(Args A, const MmaDesc* Dp, uint32_t tile) {
  A = uargs(A);
  const MmaDesc D = load_desc(Dp);
  const uint32_t lds0 = uni(uint32_t(reinterpret_cast<uintptr_t>(lds_ptr<lds_u8>())));
  const lds_u8* L = (const lds_u8*)uintptr_t(lds0);
  uint32_t g, m0, n0;
  fast_origin(D, uni(tile), &g, &m0, &n0);
  const uint32_t K = D.K, N = D.N;
  const gbyte* a = D.a + (uint64_t(g) * D.M + m0) * K * 2;        // A[g, m0, 0]
  const gbyte* b = D.b + (uint64_t(g) * K * N + n0) * 2;           // B[g, 0, n0]
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t wm = wave >> 1, wn = wave & 1;
  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};
  const uint32_t nk = RAG ? (K + kFBK - 1) / kFBK : K / kFBK;
  FastDma dm;
  RaggedDma rd;
  if constexpr (RAG) rd.init(a, b, D.M, N, K, m0, n0);
  else dm.init(K, N);
  auto slab_a = [&](uint32_t s) { return a + uint64_t(s) * kFBK * 2; };
  auto slab_b = [&](uint32_t s) { return b + uint64_t(s) * kFBK * N * 2; };
  // Fragment addresses within a stage.  A, block i, k step kk: row wm 128 + 32 i +
  // (l & 31), chunk 2 kk + (l >> 5).  B, block j, k step kk: this lane points at
  // row 16 kk + 8 (g >> 1) + e (+ 4 for the second read), column wn 128 + 32 j +
  // 16 (g & 1) + 4 q, where g = l >> 4, e = (l >> 2) & 3, q = l & 3.
  uint32_t fa[4], fb[4];
  {
    const uint32_t r = wm * 128 + (lane & 31), sw = aswz(r);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) fa[kk] = r * 128 + (((2 * kk + (lane >> 5)) ^ sw) * 16);
    const uint32_t gq = lane >> 4, e = (lane >> 2) & 3, q = lane & 3;
    const uint32_t row = 8 * (gq >> 1) + e;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      fb[j] = kFStageB + row * 512 + ((wn * 16 + 4 * (uint32_t(j) ^ e) + 2 * (gq & 1) + (q >> 1)) * 16) + (q & 1) * 8;
  }
  u16x8 af[2][4], bfr[2][4];
  auto frags = [&](int p, uint32_t st, int kk) {
    const lds_u8* S = L + (st - lds0);
#pragma unroll
    for (int i = 0; i < 4; ++i) af[p][i] = *(const lds_u16x8*)(S + fa[kk] + 4096 * i);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(S + fb[j] + 8192 * kk));
      const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(S + fb[j] + 8192 * kk + 2048));
      bfr[p][j] = __builtin_bit_cast(u16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    }
  };
  auto mfmas = [&](int p) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = mfma16<BF16>(af[p][i], bfr[p][j], acc[i][j]);
  };
  const uint32_t st0 = lds0, st1 = lds0 + kFStage;
  __syncthreads();                      // the previous user of the LDS is done
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    if constexpr (RAG) rd.round(0, st0, r);
    else dm.round(slab_a(0), slab_b(0), K, N, st0, r);
  }
  if (nk > 1) {
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      if constexpr (RAG) rd.round(1, st1, r);
      else dm.round(slab_a(1), slab_b(1), K, N, st1, r);
    }
    wait_vm8();                         // slab 0 landed; slab 1's A rounds may be in flight
  } else {
    wait_vm0();
    if constexpr (RAG) {
      if (K % kFBK) rd.zero(0, st0);
    }
  }
  __syncthreads();
  frags(0, st0, 0);
  // Per slab: k steps 0-2 read the next step's fragments while their MFMAs run,
  // and k step 0 issues the B rounds of slab ks+1 (one per two MFMAs) into the
  // other stage; then this lane's transfers of slab ks+1 are waited for and the
  // block barrier publishes that stage (and retires every read of the current
  // one); k step 3's MFMAs then run beside the A rounds of slab ks+2 into the
  // stage just retired, after the first fragments of slab ks+1 are requested (past
  // the last slab they read a stale stage and go unused).  Each slab is one basic
  // block, so the accumulators stay in their AGPRs: the last two slabs, which
  // transfer less, run outside the main loop.
  auto mfma_r = [&](int p, int r) {
    acc[r >> 2][r & 3] = mfma16<BF16>(af[p][r >> 2], bfr[p][r & 3], acc[r >> 2][r & 3]);
  };
  auto slab = [&](uint32_t ks, auto da, auto db) {
    const uint32_t cur = (ks & 1) ? st1 : st0, nxt = (ks & 1) ? st0 : st1;
    __builtin_amdgcn_sched_barrier(0);
    frags(1, cur, 1);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (decltype(db)::value) {
      const gbyte* bn = slab_b(ks + 1);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        mfma_r(0, r);
        __builtin_amdgcn_sched_barrier(0);
        if (r & 1) {
          if constexpr (RAG) rd.round(ks + 1, nxt, 8 + (r >> 1));
          else dm.round(a, bn, K, N, nxt, 8 + (r >> 1));
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      mfmas(0);
    }
    __builtin_amdgcn_sched_barrier(0);
    frags(0, cur, 2);
    __builtin_amdgcn_sched_barrier(0);
    mfmas(1);
    __builtin_amdgcn_sched_barrier(0);
    frags(1, cur, 3);
    __builtin_amdgcn_sched_barrier(0);
    mfmas(0);
    __builtin_amdgcn_sched_barrier(0);
    wait_vm0();
    if constexpr (RAG) {
      if (ks + 2 == nk && (K % kFBK)) rd.zero(ks + 1, nxt);     // the last slab's k past K
    }
    __syncthreads();
    frags(0, nxt, 0);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (decltype(da)::value) {
      const gbyte* an = slab_a(ks + 2);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        mfma_r(1, r);
        __builtin_amdgcn_sched_barrier(0);
        if (r & 1) {
          if constexpr (RAG) rd.round(ks + 2, cur, r >> 1);
          else dm.round(an, b, K, N, cur, r >> 1);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      mfmas(1);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  uint32_t ks = 0;
  for (; ks + 2 < nk; ++ks) slab(ks, std::true_type(), std::true_type());
  if (ks + 1 < nk) slab(ks++, std::false_type(), std::true_type());
  if (ks < nk) slab(ks, std::false_type(), std::false_type());
  if (D.dt == DT_F32) store_fast<true, RAG>(A, D, acc, g, m0, n0);
  else store_fast<false, RAG>(A, D, acc, g, m0, n0);
}

// ---------------------------------------------------------------------------------
// f32 operands
// ---------------------------------------------------------------------------------
constexpr int kBK32 = 16;
constexpr int kLdA32 = kBK32 + 1;           // odd stride: conflict-free column reads
template <int T>
struct Lds32 {
  static constexpr int kLdB = T + 1;
  static constexpr int kA = T * kLdA32;
  static constexpr int kB = kBK32 * kLdB;
  static constexpr int kBuf = kA + kB;
  static constexpr int kBytes = 2 * kBuf * 4;
};

template <int T>
struct Stage32 {
  static constexpr int kChunks = T * 4 / kBlock;   // T rows x 16 k = T*4 chunks of 4
  v4u ra[kChunks];
  v4u rb[kChunks];
  VM_DEV void load(Args A, const MmaDesc& D, uint32_t g, uint32_t m0, uint32_t n0, uint32_t k0, bool vec) {
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
      const uint32_t c = threadIdx.x + j * kBlock;
      const uint32_t m = m0 + (c >> 2), k = k0 + (c & 3) * 4;
      const uint64_t lin = (uint64_t(g) * D.M + m) * D.K + k;
      const bool in = m < D.M && k < D.k1;
      if (vec) ra[j] = in ? gld((const VM_G v4u*)(gcast<float>(D.a) + lin)) : v4u_make(0, 0, 0, 0);
      else ra[j] = in ? gather_chunk(A, D.a, D.av, lin, D.k1 - k, 4) : v4u_make(0, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
      const uint32_t c = threadIdx.x + j * kBlock;
      const uint32_t k = k0 + c / (T / 4), n = n0 + (c % (T / 4)) * 4;
      const uint64_t lin = (uint64_t(g) * D.K + k) * D.N + n;
      const bool in = k < D.k1 && n < D.N;
      if (vec) rb[j] = in ? gld((const VM_G v4u*)(gcast<float>(D.b) + lin)) : v4u_make(0, 0, 0, 0);
      else rb[j] = in ? gather_chunk(A, D.b, D.bv, lin, D.N - n, 4) : v4u_make(0, 0, 0, 0);
    }
  }
  VM_DEV void store(float* lds) const {
    float* la = lds;
    float* lb = lds + Lds32<T>::kA;
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
      const uint32_t c = threadIdx.x + j * kBlock;
      float* p = la + (c >> 2) * kLdA32 + (c & 3) * 4;
      p[0] = __uint_as_float(ra[j].x);
      p[1] = __uint_as_float(ra[j].y);
      p[2] = __uint_as_float(ra[j].z);
      p[3] = __uint_as_float(ra[j].w);
    }
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
      const uint32_t c = threadIdx.x + j * kBlock;
      float* p = lb + (c / (T / 4)) * Lds32<T>::kLdB + (c % (T / 4)) * 4;
      p[0] = __uint_as_float(rb[j].x);
      p[1] = __uint_as_float(rb[j].y);
      p[2] = __uint_as_float(rb[j].z);
      p[3] = __uint_as_float(rb[j].w);
    }
  }
};

template <int T>
VM_TILE void mma_tile32(Args A, const MmaDesc* Dp, uint32_t tile) {
  A = uargs(A);
  const MmaDesc D = load_desc(Dp);
  float* lds = lds_ptr<float>();
  using C = MmaCfg<T>;
  uint32_t g, m0, n0;
  tile_origin(D, uni(tile), T, &g, &m0, &n0);
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t wm = wave >> 1, wn = wave & 1;
  const bool vec = !D.av && !D.bv && (D.K % 4) == 0 && (D.N % 4) == 0 && ((uintptr_t(D.a) | uintptr_t(D.b)) & 15) == 0;
  f32x16 acc[C::kBM][C::kBN];
#pragma unroll
  for (int i = 0; i < C::kBM; ++i)
#pragma unroll
    for (int j = 0; j < C::kBN; ++j) acc[i][j] = f32x16{};
  const uint32_t nk = (D.k1 - D.k0 + kBK32 - 1) / kBK32;
  Stage32<T> st;
  st.load(A, D, g, m0, n0, D.k0, vec);
  __syncthreads();
  st.store(lds);
  __syncthreads();
  for (uint32_t ks = 0; ks < nk; ++ks) {
    const float* cur = lds + (ks & 1) * Lds32<T>::kBuf;
    if (ks + 1 < nk) st.load(A, D, g, m0, n0, D.k0 + (ks + 1) * kBK32, vec);
    const float* la = cur;
    const float* lb = cur + Lds32<T>::kA;
#pragma unroll
    for (int kk = 0; kk < kBK32 / 2; ++kk) {
      // lanes 0-31 take k = kk, lanes 32-63 take k = 8 + kk of this slab
      const uint32_t kq = kk + (lane >> 5) * (kBK32 / 2);
      float af[C::kBM], bf[C::kBN];
#pragma unroll
      for (int bm = 0; bm < C::kBM; ++bm) af[bm] = la[(wm * (T / 2) + bm * 32 + (lane & 31)) * kLdA32 + kq];
#pragma unroll
      for (int bn = 0; bn < C::kBN; ++bn) bf[bn] = lb[kq * Lds32<T>::kLdB + wn * (T / 2) + bn * 32 + (lane & 31)];
#pragma unroll
      for (int bm = 0; bm < C::kBM; ++bm)
#pragma unroll
        for (int bn = 0; bn < C::kBN; ++bn)
          acc[bm][bn] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[bm], bf[bn], acc[bm][bn], 0, 0, 0);
    }
    if (ks + 1 < nk) st.store(lds + ((ks + 1) & 1) * Lds32<T>::kBuf);
    __syncthreads();
  }
  mma_store<T>(A, D, acc, uni(tile), g, m0, n0);
}

// ---- f32 fast path ---------------------------------------------------------------
// 256 x 256 tiles of f32 operands (M, N multiples of 256, K of 16, no views,
// 16-byte aligned): the wave split, accumulator layout (4 x 4 blocks of 32 x 32
// per wave, in AGPRs) and store of the 16-bit fast path, with
// v_mfma_f32_32x32x2_f32.  K goes in slabs of 16 through double-buffered LDS:
//   A [m][k], row stride 20 floats: the 16 lanes of one 16-byte LDS read step
//     read 16 consecutive rows at the same k, 80 bytes apart, which covers the 64
//     banks once; a lane reads the 4 k values of 4 consecutive k steps with one
//     ds_read_b128 per block;
//   B [k][n], row stride 260: a lane reads one value per block and k step; the
//     two half-waves read rows k and k + 8, whose banks are 32 apart.
// Lanes 0-31 take k = kk and lanes 32-63 k = 8 + kk of the slab at k step kk,
// the assignment of mma_tile32, so the two paths sum in the same order.  The
// next slab's global loads are issued before the slab's MFMAs and written to
// the idle buffer after them; a k step's B values are read while the previous
// step's MFMAs run.
constexpr int kF32BK = 16, kF32LdA = 20, kF32LdB = 256 + 4;
constexpr int kF32A = 256 * kF32LdA, kF32Buf = kF32A + kF32BK * kF32LdB;
constexpr int kF32FastLdsBytes = 2 * kF32Buf * 4;

struct F32Stage {
  // A: 256 rows x 16 k as 1024 chunks of 4 (thread t: row t / 4 + 64 j, k 4 (t % 4));
  // B: 16 k x 256 n as 1024 chunks (thread t: k t / 64 + 4 j, n 4 (t % 64))
  v4f ra[4], rb[4];
  VM_DEV void load(const gbyte* a, const gbyte* b, uint32_t K, uint32_t N) {
    const uint32_t t = threadIdx.x;
#pragma unroll
    for (int j = 0; j < 4; ++j) ra[j] = *(const VM_G v4f*)(a + (uint64_t(t / 4 + 64 * j) * K + (t % 4) * 4) * 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) rb[j] = *(const VM_G v4f*)(b + (uint64_t(t / 64 + 4 * j) * N + (t % 64) * 4) * 4);
  }
  // The same chunks of slab s for a ragged tile (K, N multiples of 4): rows past
  // M re-read row M - 1 and columns past N the last 4 (computed, not stored); k
  // past K re-read the last k and are zeroed in registers, in both operands.
  // a = A[g, m0, 0], b = B[g, 0, n0].  The loads are not predicated, so none of
  // them waits behind a branch.
  VM_DEV void load_ragged(const gbyte* a, const gbyte* b, uint32_t s, uint32_t M, uint32_t K, uint32_t N, uint32_t m0,
                          uint32_t n0) {
    const uint32_t t = threadIdx.x, k0 = s * kF32BK;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t row = min(m0 + t / 4 + 64 * j, M - 1) - m0, k = k0 + (t % 4) * 4;
      const v4f v = *(const VM_G v4f*)(a + (uint64_t(row) * K + min(k, K - 4)) * 4);
      ra[j] = k < K ? v : v4f{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t k = k0 + t / 64 + 4 * j, n = min(n0 + (t % 64) * 4, N - 4) - n0;
      const v4f v = *(const VM_G v4f*)(b + (uint64_t(min(k, K - 1)) * N + n) * 4);
      rb[j] = k < K ? v : v4f{0.0f, 0.0f, 0.0f, 0.0f};
    }
  }
  VM_DEV void store(float* s) const {
    const uint32_t t = threadIdx.x;
#pragma unroll
    for (int j = 0; j < 4; ++j) *reinterpret_cast<v4f*>(s + (t / 4 + 64 * j) * kF32LdA + (t % 4) * 4) = ra[j];
#pragma unroll
    for (int j = 0; j < 4; ++j) *reinterpret_cast<v4f*>(s + kF32A + (t / 64 + 4 * j) * kF32LdB + (t % 64) * 4) = rb[j];
  }
};

template <bool RAG>
VM_LEAF void mma_tile32_fast(Args A, const MmaDesc* Dp, uint32_t tile) {
  A = uargs(A);
  const MmaDesc D = load_desc(Dp);
  float* lds = lds_ptr<float>();
  uint32_t g, m0, n0;
  fast_origin(D, uni(tile), &g, &m0, &n0);
  const uint32_t K = D.K, N = D.N;
  const gbyte* a = D.a + (uint64_t(g) * D.M + m0) * K * 4;        // A[g, m0, 0]
  const gbyte* b = D.b + (uint64_t(g) * K * N + n0) * 4;           // B[g, 0, n0]
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t wm = wave >> 1, wn = wave & 1;
  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};
  const uint32_t nk = RAG ? (K + kF32BK - 1) / kF32BK : K / kF32BK;
  F32Stage st;
  if constexpr (RAG) st.load_ragged(a, b, 0, D.M, K, N, m0, n0);
  else st.load(a, b, K, N);
  __syncthreads();                      // the previous user of the LDS is done
  st.store(lds);
  __syncthreads();
  const uint32_t fa = (wm * 128 + (lane & 31)) * kF32LdA + (lane >> 5) * 8;
  const uint32_t fb = kF32A + (lane >> 5) * 8 * kF32LdB + wn * 128 + (lane & 31);
  for (uint32_t ks = 0; ks < nk; ++ks) {
    const float* cur = lds + (ks & 1) * kF32Buf;
    if (ks + 1 < nk) {
      if constexpr (RAG) st.load_ragged(a, b, ks + 1, D.M, K, N, m0, n0);
      else st.load(a + uint64_t(ks + 1) * kF32BK * 4, b + uint64_t(ks + 1) * kF32BK * N * 4, K, N);
    }
    float bfr[2][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) bfr[0][j] = cur[fb + j * 32];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      v4f af[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) af[i] = *reinterpret_cast<const v4f*>(cur + fa + i * 32 * kF32LdA + q * 4);
#pragma unroll
      for (int kq = 0; kq < 4; ++kq) {
        const int kk = 4 * q + kq, p = kk & 1;
        if (kk + 1 < 8)
#pragma unroll
          for (int j = 0; j < 4; ++j) bfr[p ^ 1][j] = cur[fb + (kk + 1) * kF32LdB + j * 32];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][kq], bfr[p][j], acc[i][j], 0, 0, 0);
      }
    }
    if (ks + 1 < nk) st.store(lds + ((ks + 1) & 1) * kF32Buf);
    __syncthreads();
  }
  if (D.dt == DT_F32) store_fast<true, RAG>(A, D, acc, g, m0, n0);
  else store_fast<false, RAG>(A, D, acc, g, m0, n0);
}

// LDS bytes the matmul tile op needs at its largest tile.
constexpr int kMaxI(int a, int b) { return a > b ? a : b; }
constexpr int kMmaLdsBytes0 = kMaxI(kMaxI(Lds16<256>::kBytes, Lds16<128>::kBytes), kMaxI(Lds16<64>::kBytes, Lds32<256>::kBytes));
constexpr int kMmaLdsBytes1 = kFastLdsBytes > kMmaLdsBytes0 ? kFastLdsBytes : kMmaLdsBytes0;
constexpr int kMmaLdsBytes = kF32FastLdsBytes > kMmaLdsBytes1 ? kF32FastLdsBytes : kMmaLdsBytes1;

VM_DEV void mma_tiles(Args A, uint32_t ti, uint32_t lo, uint32_t hi) {
  A = uargs(A);
  const VM_K Task& t = task_of(A, ti);
  MmaDesc D;
  D.M = t.p[0];
  D.N = t.p[1];
  D.K = t.p[2];
  D.G = max(1u, t.p[3] & 0xFFFFFFu);
  const uint32_t code = (t.p[3] >> 24) & 0xF;
  const uint32_t T = code == 1 ? 64u : code == 2 ? 128u : code == 3 ? 256u : A->mma_t;
  D.tm = (D.M + T - 1) / T;
  D.tn = (D.N + T - 1) / T;
  D.a = resolve(A, t.a);
  D.b = resolve(A, t.b);
  D.d = resolve(A, t.dst);
  D.av = t.p[4];
  D.bv = t.p[5];
  D.epi = t.p[6];
  D.res = t.p[6] ? resolve(A, t.p[7]) : D.a;
  D.dt = (t.tile_op >> 8) & 0xFF;
  D.adt = (t.tile_op >> 16) & 0xFF;
  D.S = 1u << ((t.p[3] >> 28) & 0xF);
  D.ti = ti;
  D.k0 = 0;
  D.k1 = D.K;
  D.split = 0;
  hi = min(hi, D.tm * D.tn * D.G * D.S);
  const bool h16 = D.adt == DT_BF16 || D.adt == DT_F16, bf = D.adt == DT_BF16;
  // a K split's share: whole slabs of the general tiles (32 16-bit or 16 f32 k)
  const uint32_t bk = h16 ? uint32_t(kBK16) : uint32_t(kBK32);
  const uint32_t ksh = ((D.K + D.S - 1) / D.S + bk - 1) / bk * bk;
  const bool fast = D.S == 1 && h16 && T == 256 && !D.av && !D.bv && D.M % 256 == 0 && D.N % 256 == 0 && D.K % kFBK == 0 &&
                    D.N < (1u << 22) && ((uintptr_t(D.a) | uintptr_t(D.b)) & 15) == 0 &&
                    (D.dt == DT_F32 || D.dt == DT_BF16 || D.dt == DT_F16) && epi_inline_ok(A, D.epi);
  // the same tile for ragged shapes: 16-byte rows (K, N multiples of 8), offsets
  // within 32 bits (RaggedDma)
  const bool fastr = !fast && D.S == 1 && h16 && T == 256 && !D.av && !D.bv && D.K >= 8 && D.K % 8 == 0 && D.N % 8 == 0 &&
                     D.K < (1u << 22) && D.N < (1u << 22) && ((uintptr_t(D.a) | uintptr_t(D.b)) & 15) == 0 &&
                     (D.dt == DT_F32 || D.dt == DT_BF16 || D.dt == DT_F16) && epi_inline_ok(A, D.epi);
  const bool fast32 = D.S == 1 && D.adt == DT_F32 && T == 256 && !D.av && !D.bv && D.M % 256 == 0 && D.N % 256 == 0 &&
                      D.K % kF32BK == 0 && D.N < (1u << 22) && ((uintptr_t(D.a) | uintptr_t(D.b)) & 15) == 0 &&
                      (D.dt == DT_F32 || D.dt == DT_BF16 || D.dt == DT_F16) && epi_inline_ok(A, D.epi);
  const bool fast32r = !fast32 && D.S == 1 && D.adt == DT_F32 && T == 256 && !D.av && !D.bv && D.K >= 4 &&
                       D.K % 4 == 0 && D.N % 4 == 0 && D.N < (1u << 22) && ((uintptr_t(D.a) | uintptr_t(D.b)) & 15) == 0 &&
                       (D.dt == DT_F32 || D.dt == DT_BF16 || D.dt == DT_F16) && epi_inline_ok(A, D.epi);
  for (uint32_t ts = lo; ts < hi; ++ts) {
    uint32_t tile = ts;
    if (D.S > 1) {                      // split ts % S of output tile ts / S
      tile = ts / D.S;
      D.split = ts % D.S;
      D.k0 = min(D.split * ksh, D.K);
      D.k1 = min(D.k0 + ksh, D.K);
    }
    if (fast32) {
      mma_tile32_fast<false>(A, &D, tile);
    } else if (fast32r) {
      mma_tile32_fast<true>(A, &D, tile);
    } else if (fast) {
      if (bf) mma_tile16_fast<true, false>(A, &D, tile);
      else mma_tile16_fast<false, false>(A, &D, tile);
    } else if (fastr) {
      if (bf) mma_tile16_fast<true, true>(A, &D, tile);
      else mma_tile16_fast<false, true>(A, &D, tile);
    } else if (h16) {
      if (T == 256) { if (bf) mma_tile16<256, true>(A, &D, tile); else mma_tile16<256, false>(A, &D, tile); }
      else if (T == 128) { if (bf) mma_tile16<128, true>(A, &D, tile); else mma_tile16<128, false>(A, &D, tile); }
      else { if (bf) mma_tile16<64, true>(A, &D, tile); else mma_tile16<64, false>(A, &D, tile); }
    } else {
      if (T == 256) mma_tile32<256>(A, &D, tile);
      else if (T == 128) mma_tile32<128>(A, &D, tile);
      else mma_tile32<64>(A, &D, tile);
    }
  }
}

}  // namespace vm
