// TOP_MMA: C[g] = A[g] (MxK) . B[g] (KxN) (+ store epilogue), f32 accumulate on
// CDNA4 matrix cores (reference semantics: ops/mma.cl:362-434, epilogue 74-96).
// Task: p0 M, p1 N, p2 K, p3 G (bits 0-23) | tile-edge code (bits 24-27),
// p4 A view+1, p5 B view+1, p6 epilogue descriptor+1, p7 residual handle.
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
    v = micro(kind, v, y, s, t);
  }
  return v;
}

template <int T>
struct MmaCfg {
  static constexpr int kBM = T / 64;         // 32x32 blocks per wave along M
  static constexpr int kBN = T / 64;
};

template <int T>
VM_DEV void store_acc(Args A, const MmaDesc& D, const f32x16 (&acc)[MmaCfg<T>::kBM][MmaCfg<T>::kBN], uint32_t g,
                      uint32_t m0, uint32_t n0) {
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t wm = wave >> 1, wn = wave & 1;
#pragma unroll
  for (int bm = 0; bm < MmaCfg<T>::kBM; ++bm) {
#pragma unroll
    for (int bn = 0; bn < MmaCfg<T>::kBN; ++bn) {
      const uint32_t col = n0 + wn * (T / 2) + bn * 32 + (lane & 31);
      const uint32_t rbase = m0 + wm * (T / 2) + bm * 32 + 4 * (lane >> 5);
      if (D.epi) {
#pragma unroll 1
        for (int v = 0; v < 16; ++v) {
          const uint32_t row = rbase + 8 * (v >> 2) + (v & 3);
          if (row < D.M && col < D.N) {
            const uint64_t elem = (uint64_t(g) * D.M + row) * D.N + col;
            store_f(D.d, D.dt, elem, apply_epilogue(A, D.epi, D.res, elem, col, acc[bm][bn][v]));
          }
        }
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
constexpr int kBK16 = 32;                 // K slab (elements)
constexpr int kLdA16 = kBK16 + 8;         // A row stride in LDS (elements): 80 B
template <int T>
struct Lds16 {
  static constexpr int kLdB = T + 4;      // B row stride (elements): 8-byte aligned rows
  static constexpr int kA = T * kLdA16;   // elements
  static constexpr int kB = kBK16 * kLdB;
  static constexpr int kBuf = kA + kB;
  static constexpr int kBytes = 2 * kBuf * 2;   // double buffered, 2 bytes each
};

template <int T>
struct Stage16 {
  // A: T rows x 32 k = T*4 chunks of 8 elements; B: 32 rows x T cols = 4T chunks.
  static constexpr int kChunks = T * 4 / kBlock;
  v4u ra[kChunks];
  v4u rb[kChunks];

  VM_DEV void load(Args A, const MmaDesc& D, uint32_t g, uint32_t m0, uint32_t n0, uint32_t k0, bool vec) {
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
      const uint32_t c = threadIdx.x + j * kBlock;
      const uint32_t m = m0 + (c >> 2), k = k0 + (c & 3) * 8;
      const uint64_t lin = (uint64_t(g) * D.M + m) * D.K + k;
      const bool in = m < D.M && k < D.K;
      if (vec) ra[j] = in ? gld((const VM_G v4u*)(gcast<uint16_t>(D.a) + lin)) : v4u_make(0, 0, 0, 0);
      else ra[j] = in ? gather_chunk(A, D.a, D.av, lin, D.K - k, 2) : v4u_make(0, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
      const uint32_t c = threadIdx.x + j * kBlock;
      const uint32_t k = k0 + c / (T / 8), n = n0 + (c % (T / 8)) * 8;
      const uint64_t lin = (uint64_t(g) * D.K + k) * D.N + n;
      const bool in = k < D.K && n < D.N;
      if (vec) rb[j] = in ? gld((const VM_G v4u*)(gcast<uint16_t>(D.b) + lin)) : v4u_make(0, 0, 0, 0);
      else rb[j] = in ? gather_chunk(A, D.b, D.bv, lin, D.N - n, 2) : v4u_make(0, 0, 0, 0);
    }
  }
  VM_DEV void store(uint16_t* lds) const {
    uint16_t* la = lds;
    uint16_t* lb = lds + Lds16<T>::kA;
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
      const uint32_t c = threadIdx.x + j * kBlock;
      *reinterpret_cast<v4u*>(la + (c >> 2) * kLdA16 + (c & 3) * 8) = ra[j];
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
  uint16_t* lds = reinterpret_cast<uint16_t*>(vm_smem);
  using C = MmaCfg<T>;
  uint32_t g, m0, n0;
  tile_origin(D, uni(tile), T, &g, &m0, &n0);
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t wm = wave >> 1, wn = wave & 1;
  const bool vec = !D.av && !D.bv && (D.K % 8) == 0 && (D.N % 8) == 0 && ((uintptr_t(D.a) | uintptr_t(D.b)) & 15) == 0;

  f32x16 acc[C::kBM][C::kBN];
#pragma unroll
  for (int i = 0; i < C::kBM; ++i)
#pragma unroll
    for (int j = 0; j < C::kBN; ++j) acc[i][j] = f32x16{};

  const uint32_t nk = (D.K + kBK16 - 1) / kBK16;
  Stage16<T> st;
  st.load(A, D, g, m0, n0, 0, vec);
  __syncthreads();                      // previous user of the LDS is done
  st.store(lds);
  __syncthreads();
  for (uint32_t ks = 0; ks < nk; ++ks) {
    const uint16_t* cur = lds + (ks & 1) * Lds16<T>::kBuf;
    if (ks + 1 < nk) st.load(A, D, g, m0, n0, (ks + 1) * kBK16, vec);
    const uint16_t* la = cur;
    const uint16_t* lb = cur + Lds16<T>::kA;
#pragma unroll
    for (int kk = 0; kk < kBK16; kk += 16) {
      const uint32_t kq = kk + (lane >> 5) * 8;
      u16x8 af[C::kBM], bf[C::kBN];
#pragma unroll
      for (int bm = 0; bm < C::kBM; ++bm)
        af[bm] = *reinterpret_cast<const u16x8*>(la + (wm * (T / 2) + bm * 32 + (lane & 31)) * kLdA16 + kq);
#pragma unroll
      for (int bn = 0; bn < C::kBN; ++bn) {
        const uint32_t cidx = wn * (T / 2) + bn * 32 + (lane & 31);
        u16x8 v;
#pragma unroll
        for (int q = 0; q < 8; ++q) v[q] = lb[(kq + q) * Lds16<T>::kLdB + cidx];
        bf[bn] = v;
      }
#pragma unroll
      for (int bm = 0; bm < C::kBM; ++bm)
#pragma unroll
        for (int bn = 0; bn < C::kBN; ++bn) acc[bm][bn] = mfma16<BF16>(af[bm], bf[bn], acc[bm][bn]);
    }
    if (ks + 1 < nk) st.store(lds + ((ks + 1) & 1) * Lds16<T>::kBuf);
    __syncthreads();
  }
  store_acc<T>(A, D, acc, g, m0, n0);
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
      const bool in = m < D.M && k < D.K;
      if (vec) ra[j] = in ? gld((const VM_G v4u*)(gcast<float>(D.a) + lin)) : v4u_make(0, 0, 0, 0);
      else ra[j] = in ? gather_chunk(A, D.a, D.av, lin, D.K - k, 4) : v4u_make(0, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
      const uint32_t c = threadIdx.x + j * kBlock;
      const uint32_t k = k0 + c / (T / 4), n = n0 + (c % (T / 4)) * 4;
      const uint64_t lin = (uint64_t(g) * D.K + k) * D.N + n;
      const bool in = k < D.K && n < D.N;
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
  float* lds = reinterpret_cast<float*>(vm_smem);
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
  const uint32_t nk = (D.K + kBK32 - 1) / kBK32;
  Stage32<T> st;
  st.load(A, D, g, m0, n0, 0, vec);
  __syncthreads();
  st.store(lds);
  __syncthreads();
  for (uint32_t ks = 0; ks < nk; ++ks) {
    const float* cur = lds + (ks & 1) * Lds32<T>::kBuf;
    if (ks + 1 < nk) st.load(A, D, g, m0, n0, (ks + 1) * kBK32, vec);
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
  store_acc<T>(A, D, acc, g, m0, n0);
}

// LDS bytes the matmul tile op needs at its largest tile.
constexpr int kMmaLdsBytes = Lds16<256>::kBytes > Lds32<256>::kBytes ? Lds16<256>::kBytes : Lds32<256>::kBytes;

VM_TILE void mma_tiles(Args A, uint32_t ti, uint32_t lo, uint32_t hi) {
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
  hi = min(hi, D.tm * D.tn * D.G);
  const bool h16 = D.adt == DT_BF16 || D.adt == DT_F16, bf = D.adt == DT_BF16;
  for (uint32_t tile = lo; tile < hi; ++tile) {
    if (h16) {
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
