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
// to 16 row loads in flight.  The RP row-phase sums are added in a fixed order:
// by DPP row rotations inside each 16-lane row, then the row partials through LDS.
#pragma once
#include "tile_mma.h"
#include "tile_reduce.h"

namespace vm {

// Rows rp, rp + RP, ... of this thread's 8 columns.  Loads run in chunks of U rows
// into two register buffers: chunk c+1 is in flight while chunk c is consumed.
// Rows past K re-read row K - 1 and are not accumulated; col is always a valid
// column group (callers clamp it), so no load sits behind a branch (a load under
// a lane-dependent branch makes the compiler wait for it before the join); xs
// rows past M re-read row M - 1 (results unused).
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

// Weight rows per load chunk and thread (two chunks in flight), and x elements
// per thread staged from registers.
template <uint32_t ADT>
constexpr int gemv_u() { return 8; }
constexpr int kGemvXU = 12;

// f32 value as stored in dtype DT and read back
template <uint32_t DT>
VM_DEV float gemv_round(float z) {
  if constexpr (DT == DT_BF16) return bf16_to_f32(f32_to_bf16(z));
  else if constexpr (DT == DT_F16) return f16_to_f32(f32_to_f16(z));
  else return z;
}

// The first kGemvXU * kBlock elements of x (flat index threadIdx.x + u kBlock) as
// raw bits, all loads issued back to back and nothing converted yet, so that the
// weight loads issued next are in flight before the first wait.  Indices past n
// re-read element n - 1 (no load behind a branch); gemv_xcvt zeroes them.
VM_DEV bool gemv_x_raw_ok(uint32_t dt) { return dt == DT_F32 || dt == DT_BF16 || dt == DT_F16; }
VM_DEV void gemv_xraw(uint32_t (&r)[kGemvXU], const gbyte* src, uint32_t dt, uint32_t n) {
  if (dt == DT_F32) {
#pragma unroll
    for (int u = 0; u < kGemvXU; ++u) r[u] = gcast<uint32_t>(src)[min(threadIdx.x + u * kBlock, n - 1)];
  } else {
#pragma unroll
    for (int u = 0; u < kGemvXU; ++u) r[u] = gcast<uint16_t>(src)[min(threadIdx.x + u * kBlock, n - 1)];
  }
}
VM_DEV void gemv_xcvt(const uint32_t (&r)[kGemvXU], float (&x)[kGemvXU], uint32_t dt, uint32_t n) {
#pragma unroll
  for (int u = 0; u < kGemvXU; ++u) {
    const float v = dt == DT_F32 ? __uint_as_float(r[u]) : dt == DT_BF16 ? bf16_to_f32(uint16_t(r[u]))
                                                                         : f16_to_f32(uint16_t(r[u]));
    x[u] = threadIdx.x + u * kBlock < n ? v : 0.0f;
  }
}

// Normalise the M x K rows staged in xs in place by the layernorm task L (the
// LAYERNORM_SEG semantics: mean, two-pass or one-pass variance per its flags,
// rsqrt(var + eps), affine, GELU), rounded to DT as the layernorm's store would.
// gv / bv: gamma / beta of columns threadIdx.x + u kBlock (K <= kGemvXU kBlock),
// else read from memory.  Each thread keeps the same columns in every pass.
template <uint32_t DT>
VM_DEV void gemv_ln_rows(Args A, const VM_K Task& L, uint32_t M, uint32_t K, float* xs, float* red,
                         const float (&gv)[kGemvXU], const float (&bv)[kGemvXU]) {
  const uint32_t flags = L.p[3];
  const float eps = __uint_as_float(L.p[2]);
  const bool affine = flags & LN_AFFINE, do_gelu = flags & LN_GELU, two_pass = flags & LN_TWO_PASS;
  const gbyte* gp = resolve(A, affine ? L.b : L.a);
  const gbyte* bp = resolve(A, affine ? L.p[4] : L.a);
  const bool regs = K <= kGemvXU * kBlock;
  const float inv_n = 1.0f / float(K);
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
    if (regs) {
#pragma unroll
      for (int u = 0; u < kGemvXU; ++u) {
        const uint32_t j = threadIdx.x + u * kBlock;
        if (j < K) {
          float z = fmaf(row[j], rstd, shift);
          if (affine) z = fmaf(z, gv[u], bv[u]);
          if (do_gelu) z = gelu(z);
          row[j] = gemv_round<DT>(z);
        }
      }
    } else {
      for (uint32_t j = threadIdx.x; j < K; j += kBlock) {
        float z = fmaf(row[j], rstd, shift);
        if (affine) z = fmaf(z, load_f(gp, DT_F32, j), load_f(bp, DT_F32, j));
        if (do_gelu) z = gelu(z);
        row[j] = gemv_round<DT>(z);
      }
    }
  }
}

// The same layernorm for one row (M = 1) whose K <= kGemvXU kBlock elements are
// already in registers (element threadIdx.x + u kBlock in x[u], 0 past K),
// normalised in place.  The sums are the ones gemv_ln_rows forms (per thread in
// u order, DPP wave sums, the four waves added in order), so the results are the
// same bits, with one LDS exchange and block barrier per sum instead of two
// passes over the row in LDS and two barriers per sum.  st: 3 kWaves floats of
// LDS that no other stage of the tile uses.
template <uint32_t DT>
VM_DEV void gemv_ln_regs(const VM_K Task& L, uint32_t K, float (&x)[kGemvXU], const float (&gv)[kGemvXU],
                         const float (&bv)[kGemvXU], float* st) {
  const uint32_t flags = L.p[3];
  const float eps = __uint_as_float(L.p[2]);
  const bool affine = flags & LN_AFFINE, do_gelu = flags & LN_GELU, two_pass = flags & LN_TWO_PASS;
  const float inv_n = 1.0f / float(K);
  const uint32_t wave = threadIdx.x >> 6;
  const bool lead = (threadIdx.x & 63) == 0;
  float s = 0.0f, s2 = 0.0f;
#pragma unroll
  for (int u = 0; u < kGemvXU; ++u) {
    s += x[u];
    s2 = fmaf(x[u], x[u], s2);
  }
  s = wave_sum(s);
  if (!two_pass) s2 = wave_sum(s2);
  if (lead) {
    st[wave] = s;
    st[kWaves + wave] = s2;
  }
  __syncthreads();
  float ts = st[0], ts2 = st[kWaves];
#pragma unroll
  for (int k = 1; k < kWaves; ++k) {
    ts += st[k];
    ts2 += st[kWaves + k];
  }
  const float mean = ts * inv_n;
  float var;
  if (two_pass) {
    float q = 0.0f;
#pragma unroll
    for (int u = 0; u < kGemvXU; ++u) {
      const float dv = x[u] - mean;
      if (threadIdx.x + u * kBlock < K) q = fmaf(dv, dv, q);
    }
    q = wave_sum(q);
    if (lead) st[2 * kWaves + wave] = q;
    __syncthreads();
    float tq = st[2 * kWaves];
#pragma unroll
    for (int k = 1; k < kWaves; ++k) tq += st[2 * kWaves + k];
    var = tq * inv_n;
  } else {
    var = ts2 * inv_n - mean * mean;
  }
  const float rstd = rsqrtf(var + eps);
  const float shift = -mean * rstd;
#pragma unroll
  for (int u = 0; u < kGemvXU; ++u) {
    float z = fmaf(x[u], rstd, shift);
    if (affine) z = fmaf(z, gv[u], bv[u]);
    if (do_gelu) z = gelu(z);
    x[u] = gemv_round<DT>(z);
  }
}

template <uint32_t ADT, int U>
VM_DEV void gemv_issue(typename GemvRaw<ADT>::T (&raw)[U], const gbyte* b, uint32_t N, uint32_t K, uint32_t k,
                       uint32_t RP, uint32_t col) {
#pragma unroll
  for (int u = 0; u < U; ++u) raw[u] = gemv_ld<ADT>(b, uint64_t(min(k + u * RP, K - 1)) * N + col);
}

template <uint32_t ADT, int U, int MM>
VM_DEV void gemv_consume(const typename GemvRaw<ADT>::T (&raw)[U], uint32_t M, uint32_t K, uint32_t k,
                         uint32_t RP, const float* xs, float (&acc)[MM][8]) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
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

// One tile.  Latency is its cost, so every global read it needs is issued
// before the first wait: x (or the fused layernorm's input, gamma and beta),
// the epilogue's residual values, then two weight chunks; later chunks are
// issued as earlier ones are consumed.
template <uint32_t ADT, int MM>
VM_DEV void gemv_tile(Args A, uint32_t ti, uint32_t tile) {
  A = uargs(A);
  constexpr int U = gemv_u<ADT>();
  const VM_K Task& t = task_of(A, ti);
  const uint32_t M = t.p[0], N = t.p[1], K = t.p[2], CW = t.p[4];
  const uint32_t ncb = (N + CW - 1) / CW;
  tile = uni(tile);
  const uint32_t nb = tile % ncb, g = tile / ncb;
  const uint32_t esz = ADT == DT_F32 ? 4 : 2;
  const gbyte* a = resolve(A, t.a) + uint64_t(g) * M * K * esz;
  const gbyte* b = resolve(A, t.b) + uint64_t(g) * K * N * esz;
  const uint32_t cgs = CW / 8, RP = kBlock / cgs;
  // LDS: x [M][K], then the row partials [P][M][CW] (at most 2048 M floats), then
  // the layernorm's sums; the loader checks that M * K + 4096 M floats fit
  float* xs = lds_ptr<float>();
  float* red = xs + ((M * K + 3) & ~3u);
  float* st = red + 2048 * M;
  const uint32_t nx = M * K;

  // x, or the fused layernorm's input with its gamma / beta, as raw bits
  const bool lnp = t.p[5] != 0;
  const VM_K Task& L = task_of(A, lnp ? t.p[5] - 1 : ti);
  const gbyte* xsrc = lnp ? resolve(A, L.a) : a;
  const uint32_t xdt = lnp ? (L.tile_op >> 16) & 0xFF : ADT;
  const bool lnaff = lnp && (L.p[3] & LN_AFFINE);
  const bool xreg = gemv_x_raw_ok(xdt);
  uint32_t xr[kGemvXU], gr[kGemvXU], br[kGemvXU];
  if (xreg) gemv_xraw(xr, xsrc, xdt, nx);
  if (lnaff) {
    gemv_xraw(gr, resolve(A, L.b), DT_F32, K);
    gemv_xraw(br, resolve(A, L.p[4]), DT_F32, K);
  }
  // the epilogue's residual values of this thread's first output
  const uint32_t epi = t.p[6];
  const VM_K int32_t* e = aux_of(A) + (epi ? epi - 1 : 0);
  const int nm = epi ? e[0] : 0;
  const gbyte* res = epi ? resolve(A, t.p[7]) : nullptr;
  bool src1 = false, src2 = false;
  for (int k = 0; k < nm; ++k) {
    src1 |= e[2 + 4 * k] == 1;
    src2 |= e[2 + 4 * k] == 2;
  }
  const uint32_t outs = M * CW;
  float ry1 = 0.0f, ry2 = 0.0f;
  {
    // clamped to a valid output so the loads sit behind no branch
    const uint32_t o = min(uint32_t(threadIdx.x), outs - 1), m = o / CW, n = min(nb * CW + o % CW, N - 1);
    if (src1) ry1 = gcast<float>(res)[(uint64_t(g) * M + m) * N + n];
    if (src2) ry2 = gcast<float>(res)[n];
  }

  const uint32_t cg = threadIdx.x % cgs, rp = threadIdx.x / cgs;
  // column groups past N (the last strip's tail) read the last group instead
  const uint32_t col = min(nb * CW + cg * 8, N - 8);
  const uint32_t step = U * RP;
  typename GemvRaw<ADT>::T r0[U], r1[U];
  gemv_issue<ADT, U>(r0, b, N, K, rp, RP, col);
  if (step < K) gemv_issue<ADT, U>(r1, b, N, K, step + rp, RP, col);

  float xv[kGemvXU], gv[kGemvXU], bv[kGemvXU];
  if (xreg) gemv_xcvt(xr, xv, xdt, nx);
  if (lnaff) {
    gemv_xcvt(gr, gv, DT_F32, K);
    gemv_xcvt(br, bv, DT_F32, K);
  }
  // No block barrier before the first LDS write: the entry starts after one (a
  // grid barrier, a completion-flag wait or the block sync between entries), and
  // the previous tile of this entry reads only its row partials from here on,
  // which this stage does not write.
  const bool lnreg = lnp && xreg && M == 1 && K <= kGemvXU * kBlock;
  if (lnreg) gemv_ln_regs<ADT>(L, K, xv, gv, bv, st);
  if (xreg) {
#pragma unroll
    for (int u = 0; u < kGemvXU; ++u) {
      const uint32_t i = threadIdx.x + u * kBlock;
      if (i < nx) xs[i] = xv[u];
    }
  }
  if (xreg) {
    // rows longer than the register window: batches of kGemvXU loads in flight
    for (uint32_t i0 = kGemvXU * kBlock; i0 < nx; i0 += kGemvXU * kBlock) {
      gemv_xraw(xr, xsrc + uint64_t(i0) * (xdt == DT_F32 ? 4 : 2), xdt, nx - i0);
      gemv_xcvt(xr, xv, xdt, nx - i0);
#pragma unroll
      for (int u = 0; u < kGemvXU; ++u) {
        const uint32_t i = i0 + threadIdx.x + u * kBlock;
        if (i < nx) xs[i] = xv[u];
      }
    }
  } else {
    for (uint32_t i = threadIdx.x; i < nx; i += kBlock) xs[i] = load_f(xsrc, xdt, i);
  }
  __syncthreads();
  if (lnp && !lnreg) {
    gemv_ln_rows<ADT>(A, L, M, K, xs, st, gv, bv);
    __syncthreads();
  }

  float acc[MM][8];
#pragma unroll
  for (int m = 0; m < MM; ++m)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[m][j] = 0.0f;
  // uniform loop over chunk pairs, two chunks in flight
  for (uint32_t kb = 0; kb < K; kb += 2 * step) {
    gemv_consume<ADT, U, MM>(r0, M, K, kb + rp, RP, xs, acc);
    if (kb + 2 * step < K) gemv_issue<ADT, U>(r0, b, N, K, kb + 2 * step + rp, RP, col);
    if (kb + step >= K) break;
    gemv_consume<ADT, U, MM>(r1, M, K, kb + step + rp, RP, xs, acc);
    if (kb + 3 * step < K) gemv_issue<ADT, U>(r1, b, N, K, kb + 3 * step + rp, RP, col);
  }
  // Row-phase sums: the lanes of a 16-lane row that hold one column group (lanes
  // cg, cg + cgs, ...) add theirs by DPP row rotations (by cgs, 2 cgs, .. 8); the
  // P = kBlock / max(16, cgs) row partials then go through LDS, and one thread per
  // output adds them in row order.  (Alternating C5 runs: 1263.5 / 1260.8 ->
  // 1280.2 / 1280.9 tokens/s together with the register layernorm above.)
  const uint32_t rw = max(16u, cgs), P = kBlock / rw;
#pragma unroll
  for (int m = 0; m < MM; ++m)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float v = acc[m][j];
      if (cgs < 2) v += dpp<0x121>(v);
      if (cgs < 4) v += dpp<0x122>(v);
      if (cgs < 8) v += dpp<0x124>(v);
      if (cgs < 16) v += dpp<0x128>(v);
      acc[m][j] = v;
    }
  if ((threadIdx.x & 15) < cgs) {
    const uint32_t pr = threadIdx.x / rw;
#pragma unroll
    for (int m = 0; m < MM; ++m)
      if (m < int(M))
#pragma unroll
        for (int j = 0; j < 8; ++j) red[(pr * M + m) * CW + cg * 8 + j] = acc[m][j];
  }
  __syncthreads();

  const uint32_t dt = (t.tile_op >> 8) & 0xFF;
  gbyte* d = resolve(A, t.dst);
  for (uint32_t o = threadIdx.x; o < outs; o += kBlock) {
    const uint32_t m = o / CW, n = nb * CW + o % CW;
    if (n >= N) continue;
    float x = 0.0f;
    for (uint32_t q = 0; q < P; ++q) x += red[q * outs + o];
    const uint64_t elem = (uint64_t(g) * M + m) * N + n;
    const bool first = o == threadIdx.x;
    for (int k = 0; k < nm; ++k) {
      const uint32_t kind = uint32_t(e[1 + 4 * k]), src = uint32_t(e[2 + 4 * k]);
      float y = x;
      if (src == 1) y = first ? ry1 : gcast<float>(res)[elem];
      else if (src == 2) y = first ? ry2 : gcast<float>(res)[n];
      else if (src == 3) y = __int_as_float(e[3 + 4 * k]);     // constant operand s (extension)
      x = epi_inline(kind, x, y, __int_as_float(e[3 + 4 * k]), __int_as_float(e[4 + 4 * k]));
    }
    store_f(d, dt, elem, x);
  }
}

// One leaf per operand type and M class runs an entry's tiles with the tile
// inlined.  A wrapper that called the tile as a function would follow the
// calling convention around every call (its callee-saved registers to scratch
// on entry and back before it returns: a memory round trip at the end of each
// GEMV entry, and 7 KB of scratch writes per entry that the grid barrier's
// release writes back).  Called only from the kernel and never as a tail call,
// a leaf leaves the saving to the kernel, which keeps what it needs in
// registers the leaf does not touch.
template <uint32_t ADT, int MM>
VM_LEAF void gemv_run(Args A, uint32_t ti, uint32_t lo, uint32_t hi) {
  A = uargs(A);
  lo = uni(lo);
  hi = uni(hi);
  for (uint32_t tile = lo; tile < hi; ++tile) gemv_tile<ADT, MM>(A, ti, tile);
}

VM_DEV void gemv_tiles(Args A, uint32_t ti, uint32_t lo, uint32_t hi) {
  const VM_K Task& t = task_of(A, ti);
  const uint32_t M = t.p[0], adt = (t.tile_op >> 16) & 0xFF;
  const uint32_t total = max(1u, t.p[3]) * ((t.p[1] + t.p[4] - 1) / t.p[4]);
  hi = min(hi, total);
  if (adt == DT_BF16) {
    if (M == 1) gemv_run<DT_BF16, 1>(A, ti, lo, hi);
    else gemv_run<DT_BF16, kGemvMaxM>(A, ti, lo, hi);
  } else if (adt == DT_F16) {
    gemv_run<DT_F16, kGemvMaxM>(A, ti, lo, hi);
  } else {
    gemv_run<DT_F32, kGemvMaxM>(A, ti, lo, hi);
  }
}

}  // namespace vm
