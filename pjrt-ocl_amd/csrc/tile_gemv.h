// TOP_GEMV: C[g] = A[g] (M x K) . B[g] (K x N) for skinny M (decode-time matmuls:
// one token's activations against a weight matrix), the weight stream being the
// whole cost.  The reference sends these through its matmul tiles
// (ops/dot.py:94-161, mma.cl:362-434); here each tile is a narrow column strip of
// B with the full K, so a launch has a tile per CU even for N = 768 and no tile
// ever exchanges partial sums with another (no cross-CU synchronisation, no
// scratch, deterministic).
//
// Task: p0 M (<= kGemvMaxM), p1 N (multiple of 8), p2 K, p3 G, p4 CW (columns
// per tile: 8 x a power of two, at most 256), p5 layernorm prologue (index + 1
// of a LAYERNORM_SEG task over the M rows of K that no lane runs: each tile
// normalises x while staging it, rounded to A's dtype as the layernorm's store
// would, which saves the phase between the two), p6 epilogue descriptor + 1, p7
// residual handle.  Operands contiguous row-major, A/B of one dtype (bf16 / f16 /
// f32), f32 accumulation.
//
// Tile t = g * ceil(N / CW) + nb covers columns [CW nb, CW nb + CW) of batch g.
// Threads: CW / 8 column groups (one 16-byte bf16 load per row each) x RP =
// 2048 / CW row phases; thread (cg, rp) accumulates rows rp, rp + RP, ... with up
// to 16 row loads in flight.  The RP row-phase sums are added in a fixed order
// through LDS.
#pragma once
#include "tile_mma.h"
#include "tile_reduce.h"

namespace vm {

// Rows rp, rp + RP, ... of this thread's 8 columns.  Loads run in chunks of U rows
// into two register buffers: chunk c+1 is in flight while chunk c is consumed.
// Rows past K re-read row K - 1 and are not accumulated; col is always a valid
// column group (callers clamp it), so no load sits behind a branch; xs rows past
// M re-read row M - 1 (results unused).
template <uint32_t ADT>
struct GemvRaw {
  typedef v4u T;                          // 8 x 16-bit
};
template <>
struct GemvRaw<DT_F32> {
  struct T {
    v4f lo, hi;
  };
};

template <uint32_t ADT>
VM_DEV typename GemvRaw<ADT>::T gemv_ld(const gbyte* b, uint64_t elem) {
  if constexpr (ADT == DT_F32)
    return {*(const VM_G v4f*)(b + elem * 4), *(const VM_G v4f*)(b + elem * 4 + 16)};
  else
    return *(const VM_G v4u*)(b + elem * 2);
}

template <uint32_t ADT>
VM_DEV void gemv_cvt(const typename GemvRaw<ADT>::T& r, float (&w)[8]) {
  if constexpr (ADT == DT_F32) {
    w[0] = r.lo.x; w[1] = r.lo.y; w[2] = r.lo.z; w[3] = r.lo.w;
    w[4] = r.hi.x; w[5] = r.hi.y; w[6] = r.hi.z; w[7] = r.hi.w;
  } else {
    const uint32_t u[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (ADT == DT_BF16) {
        w[2 * i] = __uint_as_float(u[i] << 16);
        w[2 * i + 1] = __uint_as_float(u[i] & 0xFFFF0000u);
      } else {
        w[2 * i] = f16_to_f32(uint16_t(u[i] & 0xFFFF));
        w[2 * i + 1] = f16_to_f32(uint16_t(u[i] >> 16));
      }
    }
  }
}

constexpr int kGemvU = 8;                 // rows per load chunk and thread

// f32 value as stored in dtype DT and read back
template <uint32_t DT>
VM_DEV float gemv_round(float z) {
  if constexpr (DT == DT_BF16) return bf16_to_f32(f32_to_bf16(z));
  else if constexpr (DT == DT_F16) return f16_to_f32(f32_to_f16(z));
  else return z;
}

// Stage the M x K rows of x normalised by the layernorm task `lti` (the
// LAYERNORM_SEG semantics: mean, two-pass or one-pass variance per its flags,
// rsqrt(var + eps), affine, GELU), rounded to DT, into xs.  Each thread keeps the
// same columns in every pass, so the in-place update needs no extra barrier.
template <uint32_t DT>
VM_DEV void gemv_ln_stage(Args A, uint32_t lti, uint32_t M, uint32_t K, float* xs, float* red) {
  const VM_K Task& L = task_of(A, lti);
  const uint32_t flags = L.p[3];
  const float eps = __uint_as_float(L.p[2]);
  const uint32_t xdt = (L.tile_op >> 16) & 0xFF;
  const bool affine = flags & LN_AFFINE, do_gelu = flags & LN_GELU, two_pass = flags & LN_TWO_PASS;
  const gbyte* x = resolve(A, L.a);
  const gbyte* gp = resolve(A, affine ? L.b : L.a);
  const gbyte* bp = resolve(A, affine ? L.p[4] : L.a);
  const float inv_n = 1.0f / float(K);
  for (uint32_t m = 0; m < M; ++m)
    for (uint32_t j = threadIdx.x; j < K; j += kBlock) xs[m * K + j] = load_f(x, xdt, uint64_t(m) * K + j);
  for (uint32_t m = 0; m < M; ++m) {
    float* row = xs + m * K;
    float s = 0.0f, s2 = 0.0f;
    for (uint32_t j = threadIdx.x; j < K; j += kBlock) {
      const float v = row[j];
      s += v;
      s2 = fmaf(v, v, s2);
    }
    const float mean = block_reduce(s, OpSum(), red) * inv_n;
    float var;
    if (two_pass) {
      float q = 0.0f;
      for (uint32_t j = threadIdx.x; j < K; j += kBlock) {
        const float dv = row[j] - mean;
        q = fmaf(dv, dv, q);
      }
      var = block_reduce(q, OpSum(), red + kWaves) * inv_n;
    } else {
      var = block_reduce(s2, OpSum(), red + kWaves) * inv_n - mean * mean;
    }
    const float rstd = rsqrtf(var + eps);
    const float shift = -mean * rstd;
    for (uint32_t j = threadIdx.x; j < K; j += kBlock) {
      float z = fmaf(row[j], rstd, shift);
      if (affine) z = fmaf(z, load_f(gp, DT_F32, j), load_f(bp, DT_F32, j));
      if (do_gelu) z = gelu(z);
      row[j] = gemv_round<DT>(z);
    }
  }
}

template <uint32_t ADT>
VM_DEV void gemv_issue(typename GemvRaw<ADT>::T (&raw)[kGemvU], const gbyte* b, uint32_t N, uint32_t K, uint32_t k,
                       uint32_t RP, uint32_t col) {
#pragma unroll
  for (int u = 0; u < kGemvU; ++u) raw[u] = gemv_ld<ADT>(b, uint64_t(min(k + u * RP, K - 1)) * N + col);
}

template <uint32_t ADT, int MM>
VM_DEV void gemv_consume(const typename GemvRaw<ADT>::T (&raw)[kGemvU], uint32_t M, uint32_t K, uint32_t k,
                         uint32_t RP, const float* xs, float (&acc)[MM][8]) {
#pragma unroll
  for (int u = 0; u < kGemvU; ++u) {
    const uint32_t kk = k + u * RP;
    if (kk < K) {
      float w[8];
      gemv_cvt<ADT>(raw[u], w);
#pragma unroll
      for (int m = 0; m < MM; ++m) {
        const float xv = xs[min(uint32_t(m), M - 1) * K + kk];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[m][j] = fmaf(xv, w[j], acc[m][j]);
      }
    }
  }
}

template <uint32_t ADT, int MM>
VM_TILE void gemv_tile(Args A, uint32_t ti, uint32_t tile) {
  A = uargs(A);
  const VM_K Task& t = task_of(A, ti);
  const uint32_t M = t.p[0], N = t.p[1], K = t.p[2], CW = t.p[4];
  const uint32_t ncb = (N + CW - 1) / CW;
  tile = uni(tile);
  const uint32_t nb = tile % ncb, g = tile / ncb;
  const uint32_t esz = ADT == DT_F32 ? 4 : 2;
  const gbyte* a = resolve(A, t.a) + uint64_t(g) * M * K * esz;
  const gbyte* b = resolve(A, t.b) + uint64_t(g) * K * N * esz;
  const uint32_t cgs = CW / 8, RP = kBlock / cgs;
  // LDS: x [M][K], then the row-phase sums [RP][M][CW] (= 2048 M floats), then the
  // first-pass sums; the loader checks that M * K + 4096 M floats fit
  float* xs = reinterpret_cast<float*>(vm_smem);
  float* red = xs + ((M * K + 3) & ~3u);
  float* tmp = red + 2048 * M;

  const uint32_t cg = threadIdx.x % cgs, rp = threadIdx.x / cgs;
  // column groups past N (the last strip's tail) read the last group instead
  const uint32_t col = min(nb * CW + cg * 8, N - 8);
  // the first weight chunk is in flight while x is staged
  typename GemvRaw<ADT>::T r0[kGemvU], r1[kGemvU];
  gemv_issue<ADT>(r0, b, N, K, rp, RP, col);
  __syncthreads();                       // the previous user of the LDS is done
  if (t.p[5]) gemv_ln_stage<ADT>(A, t.p[5] - 1, M, K, xs, red);
  else
    for (uint32_t i = threadIdx.x; i < M * K; i += kBlock) xs[i] = load_f(a, ADT, i);
  __syncthreads();

  float acc[MM][8];
#pragma unroll
  for (int m = 0; m < MM; ++m)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[m][j] = 0.0f;
  // uniform loop over chunk pairs; the prefetch is unconditional (clamped rows)
  const uint32_t step = kGemvU * RP;
  for (uint32_t kb = 0; kb < K; kb += 2 * step) {
    gemv_issue<ADT>(r1, b, N, K, kb + step + rp, RP, col);
    gemv_consume<ADT, MM>(r0, M, K, kb + rp, RP, xs, acc);
    if (kb + step >= K) break;
    gemv_issue<ADT>(r0, b, N, K, kb + 2 * step + rp, RP, col);
    gemv_consume<ADT, MM>(r1, M, K, kb + step + rp, RP, xs, acc);
  }
#pragma unroll
  for (int m = 0; m < MM; ++m)
    if (m < int(M))
#pragma unroll
      for (int j = 0; j < 8; ++j) red[(rp * M + m) * CW + cg * 8 + j] = acc[m][j];
  __syncthreads();

  // Sum the RP row phases of each of the M * CW outputs in a fixed order: J
  // threads per output each add every J-th phase, then one thread adds the J.
  const uint32_t outs = M * CW;
  const uint32_t J = outs >= kBlock ? 1u : kBlock / outs;
  for (uint32_t i = threadIdx.x; i < outs * J; i += kBlock) {
    const uint32_t o = i % outs, j = i / outs;
    float v = 0.0f;
    for (uint32_t r = j; r < RP; r += J) v += red[r * outs + o];
    tmp[j * outs + o] = v;
  }
  __syncthreads();

  const uint32_t dt = (t.tile_op >> 8) & 0xFF;
  const uint32_t epi = t.p[6];
  gbyte* d = resolve(A, t.dst);
  const VM_K int32_t* e = aux_of(A) + (epi ? epi - 1 : 0);
  const int nm = epi ? e[0] : 0;
  const gbyte* res = epi ? resolve(A, t.p[7]) : nullptr;
  for (uint32_t o = threadIdx.x; o < outs; o += kBlock) {
    const uint32_t m = o / CW, n = nb * CW + o % CW;
    if (n >= N) continue;
    float x = 0.0f;
    for (uint32_t j = 0; j < J; ++j) x += tmp[j * outs + o];
    const uint64_t elem = (uint64_t(g) * M + m) * N + n;
    for (int k = 0; k < nm; ++k) {
      const uint32_t kind = uint32_t(e[1 + 4 * k]), src = uint32_t(e[2 + 4 * k]);
      float y = x;
      if (src == 1) y = gcast<float>(res)[elem];
      else if (src == 2) y = gcast<float>(res)[n];
      x = epi_inline(kind, x, y, __int_as_float(e[3 + 4 * k]), __int_as_float(e[4 + 4 * k]));
    }
    store_f(d, dt, elem, x);
  }
}

VM_TILE void gemv_tiles(Args A, uint32_t ti, uint32_t lo, uint32_t hi) {
  A = uargs(A);
  const VM_K Task& t = task_of(A, ti);
  const uint32_t M = t.p[0], adt = (t.tile_op >> 16) & 0xFF;
  const uint32_t total = max(1u, t.p[3]) * ((t.p[1] + t.p[4] - 1) / t.p[4]);
  hi = min(hi, total);
  for (uint32_t tile = lo; tile < hi; ++tile) {
    if (adt == DT_BF16) {
      if (M == 1) gemv_tile<DT_BF16, 1>(A, ti, tile);
      else gemv_tile<DT_BF16, kGemvMaxM>(A, ti, tile);
    } else if (adt == DT_F16) {
      gemv_tile<DT_F16, kGemvMaxM>(A, ti, tile);
    } else {
      gemv_tile<DT_F32, kGemvMaxM>(A, ti, tile);
    }
  }
}

}  // namespace vm
