// TOP_GEMV: C[g] = A[g] (M x K) . B[g] (K x N) for skinny M (decode-time matmuls:
// one token's activations against a weight matrix), the weight stream being the
// whole cost.  The reference sends these through its matmul tiles
// (ops/dot.py:94-161, mma.cl:362-434), whose K loop runs serially inside one
// tile; here K is split so every CU streams a slice of the weights at once.
//
// Task: p0 M (<= kGemvMaxM), p1 N (multiple of 8), p2 K, p3 G, p4 S (K splits),
// p5 scratch byte offset (assigned by the loader), p6 epilogue descriptor + 1,
// p7 residual handle.  Operands contiguous row-major, A/B of one dtype
// (bf16 / f16 / f32), f32 accumulation.
//
// Tile t = ((g * S) + s) * NCB + nb covers output columns [256 nb, 256 nb + 256)
// of batch g over the K rows of split s.  Threads: 32 column groups of 8 columns
// (one 16-byte bf16 load per row) x 8 row phases.  The 8 row phases are summed
// through LDS into the split's partial [M][256], stored in the scratch area;
// a per-(g, nb) arrival counter then elects the last split to finish, which sums
// the S partials in split order (deterministic), applies the store epilogue and
// writes C.  The counter is reset by that last tile, so the next execution (or
// loop trip) starts from zero.
#pragma once
#include "tile_mma.h"

namespace vm {

VM_DEV uint32_t gemv_ncb(uint32_t N) { return (N + kGemvCols - 1) / kGemvCols; }

// 8 consecutive elements of row k starting at column c, as f32.
template <uint32_t ADT>
VM_DEV void gemv_row8(const gbyte* b, uint64_t elem, float (&w)[8]) {
  if constexpr (ADT == DT_F32) {
    const v4f lo = *(const VM_G v4f*)(b + elem * 4), hi = *(const VM_G v4f*)(b + elem * 4 + 16);
    w[0] = lo.x; w[1] = lo.y; w[2] = lo.z; w[3] = lo.w;
    w[4] = hi.x; w[5] = hi.y; w[6] = hi.z; w[7] = hi.w;
  } else {
    const v4u q = *(const VM_G v4u*)(b + elem * 2);
    const uint32_t u[4] = {q.x, q.y, q.z, q.w};
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

// Rows k0 + rp, k0 + rp + 8, ... of this thread's 8 columns (rp = row phase),
// four rows in flight.  col is always a valid column group (callers clamp it), so
// no load sits behind a branch; xs rows past M re-read row M - 1 (results unused).
template <uint32_t ADT, int MM>
VM_DEV void gemv_accumulate(const gbyte* b, uint32_t N, uint32_t M, uint32_t k0, uint32_t k1, uint32_t col,
                            const float* xs, uint32_t kspan, float (&acc)[MM][8]) {
  const uint32_t rp = threadIdx.x >> 5;
  uint32_t k = k0 + rp;
  for (; k + 24 < k1; k += 32) {
    float w[4][8];
#pragma unroll
    for (int u = 0; u < 4; ++u) gemv_row8<ADT>(b, uint64_t(k + 8 * u) * N + col, w[u]);
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int m = 0; m < MM; ++m) {
        const float xv = xs[min(uint32_t(m), M - 1) * kspan + (k + 8 * u - k0)];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[m][j] = fmaf(xv, w[u][j], acc[m][j]);
      }
  }
  for (; k < k1; k += 8) {
    float w[8];
    gemv_row8<ADT>(b, uint64_t(k) * N + col, w);
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      const float xv = xs[min(uint32_t(m), M - 1) * kspan + (k - k0)];
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[m][j] = fmaf(xv, w[j], acc[m][j]);
    }
  }
}

template <uint32_t ADT, int MM>
VM_TILE void gemv_tile(Args A, uint32_t ti, uint32_t tile) {
  A = uargs(A);
  const VM_K Task& t = task_of(A, ti);
  const uint32_t M = t.p[0], N = t.p[1], K = t.p[2], S = t.p[4];
  const uint32_t ncb = gemv_ncb(N);
  tile = uni(tile);
  const uint32_t nb = tile % ncb, s = (tile / ncb) % S, g = tile / (ncb * S);
  const uint32_t esz = ADT == DT_F32 ? 4 : 2;
  const gbyte* a = resolve(A, t.a) + uint64_t(g) * M * K * esz;
  const gbyte* b = resolve(A, t.b) + uint64_t(g) * K * N * esz;
  const uint32_t k0 = uint32_t(uint64_t(s) * K / S), k1 = uint32_t(uint64_t(s + 1) * K / S);
  const uint32_t kspan = k1 - k0;
  // LDS: x slice [M][kspan] then the row-phase sums [8][M][256] (the loader
  // checks that (M * kspan rounded up to 4 + 2048 M) floats fit)
  float* xs = reinterpret_cast<float*>(vm_smem);
  float* red = xs + ((M * kspan + 3) & ~3u);

  __syncthreads();                       // the previous user of the LDS is done
  for (uint32_t i = threadIdx.x; i < M * kspan; i += kBlock) {
    const uint32_t m = i / kspan, k = k0 + i % kspan;
    xs[i] = load_f(a, ADT, uint64_t(m) * K + k);
  }
  __syncthreads();

  const uint32_t cg = threadIdx.x & 31, rp = threadIdx.x >> 5;
  // column groups past N (the last block's tail) read the last group instead
  const uint32_t col = min(nb * kGemvCols + cg * 8, N - 8);
  float acc[MM][8];
#pragma unroll
  for (int m = 0; m < MM; ++m)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[m][j] = 0.0f;
  if (kspan) gemv_accumulate<ADT, MM>(b, N, M, k0, k1, col, xs, kspan, acc);

  // sum the 8 row phases: red[rp][m][cg * 8 + j]
#pragma unroll
  for (int m = 0; m < MM; ++m)
    if (m < int(M))
#pragma unroll
      for (int j = 0; j < 8; ++j) red[(rp * M + m) * kGemvCols + cg * 8 + j] = acc[m][j];
  __syncthreads();

  const uint32_t dt = (t.tile_op >> 8) & 0xFF;
  const uint32_t epi = t.p[6];
  gbyte* d = resolve(A, t.dst);
  uint8_t* scratch = A->scratch + t.p[5];
  uint32_t* counters = reinterpret_cast<uint32_t*>(scratch);
  float* part = reinterpret_cast<float*>(scratch + ((uint64_t(t.p[3]) * ncb * 4 + 255) & ~uint64_t(255)));
  const uint32_t c = threadIdx.x;                                  // column within the tile
  const uint32_t n = nb * kGemvCols + c;
  // partial of this split, one column per thread
  float pm[kGemvMaxM];
#pragma unroll
  for (uint32_t m = 0; m < kGemvMaxM; ++m) {
    float v = 0.0f;
    if (m < M)
#pragma unroll
      for (int r = 0; r < 8; ++r) v += red[(r * M + m) * kGemvCols + c];
    pm[m] = v;
  }

  __shared__ uint32_t s_last;
  if (S > 1) {
    if (n < N)
      for (uint32_t m = 0; m < M; ++m) part[((uint64_t(g) * S + s) * M + m) * N + n] = pm[m];
    __threadfence();                     // partials visible device-wide before the arrival
    __syncthreads();
    if (threadIdx.x == 0) {
      uint32_t* cnt = counters + g * ncb + nb;
      const uint32_t old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
      const bool last = old == S - 1;
      if (last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = last;
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();                     // see every split's partial
    if (n < N)
      for (uint32_t m = 0; m < M; ++m) {
        float v = 0.0f;
        for (uint32_t q = 0; q < S; ++q) v += part[((uint64_t(g) * S + q) * M + m) * N + n];
        pm[m] = v;
      }
  }
  if (n >= N) return;
  const VM_K int32_t* e = aux_of(A) + (epi ? epi - 1 : 0);
  const int nm = epi ? e[0] : 0;
  const gbyte* res = epi ? resolve(A, t.p[7]) : nullptr;
  for (uint32_t m = 0; m < M; ++m) {
    const uint64_t elem = (uint64_t(g) * M + m) * N + n;
    float x = pm[m];
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
  const uint32_t total = max(1u, t.p[3]) * t.p[4] * gemv_ncb(t.p[1]);
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
