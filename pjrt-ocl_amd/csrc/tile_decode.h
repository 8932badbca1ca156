// TOP_DECODE_ATTN (extension): one decode step of attention, one tile per head.
//
//   out[h] = softmax_j(scale q[h] . key_j) value_j,  j = 0 .. pos
//   key_j = K^T[h, :, j] and value_j = V[h, j, :] for j < pos (the cache prefix),
//   key_pos = k[h], value_pos = v[h] (the step's own key / value)
//
// The reference runs this step as the decomposed chain DOT(q K^T) -> mask ->
// softmax -> DOT(P V), three barrier-separated phases per layer
// (python/pjrt_ocl/lowering.py:2664-2690 describes the idiom and leaves the
// masked decode form unfused).  Here one CU streams a head's cache slices once:
// the score pass reads K^T rows as 16-byte runs of 8 keys, the P.V pass reads V
// rows as 16-byte runs of 8 channels, both with a batch of loads in flight per
// thread.  Keys are taken in chunks of 1024 with an online softmax (running
// maximum and sum), so any context length fits a fixed LDS budget.  The step's
// key and value are read from where the projection wrote them, which lets the
// cache update run after this op, beside the next matmul.
//
// A head's keys can be split S ways (tile = head * S + split): each split
// streams its slice of the cache with its own CU and leaves its partial result
// (running maximum, sum, unnormalised output) in the task's scratch; the split
// that arrives last at the head's counter combines the S partials in split
// order (deterministic whichever arrives last) and resets the counter.  One CU
// moves only so many bytes per microsecond, so spreading a head over CUs is
// what shortens the step.
//
// Task: a q, b K^T cache [H, hd, C], p0 V cache [H, C, hd], p1 k, p2 v, p3 pos
// (i32 scalar, clamped to [0, C]), p4 H | S << 16 (S <= 1: no split), p5 hd
// (multiple of 8, <= 256) | krow << 16 | masked << 17, p6 C (multiple of 8),
// p7 scale bits.  One dtype (bf16 / f16 / f32) for every operand and the
// output; f32 arithmetic.
//
// krow: the key cache holds rows [H, C, hd] (the layout a JAX decoder keeps,
// tools/bench_decode.py:44-52) instead of K^T.  The score pass then reads keys
// the way the P.V pass reads values: hd / 8 threads per key, each a 16-byte run
// of channels, summed by lane shuffles over the key's group of threads, which is
// rounded up to a power of two (the group's extra threads add 0).
// masked: the decoder stored k and v at column pos before attending over the
// keys up to pos (dynamic_update_slice, then a key <= pos mask): pos is clamped
// to [0, C - 1] as the store's start is, and a negative pos leaves every key
// masked, so the output is NaN as the decomposed softmax makes it.
// Scratch (S > 1): [H * S][hd + 2] partials {max, sum, hd channels}, then H
// arrival counters.
#pragma once
#include "tile_gemv.h"

namespace vm {

constexpr uint32_t kDecKU = 8;                      // K / V 16-byte loads per thread at most
// LDS, in floats: scores / probabilities [64], reduction slots [16], the P.V
// partials [2048], their first-pass sums [256]
constexpr uint32_t kDecS = 0, kDecRed = 64, kDecPart = 80, kDecTmp = kDecPart + 2048;
constexpr uint32_t kDecLdsBytes = (kDecTmp + 256) * 4;

VM_DEV float dec_block_sum(float x, float* red) {
  x = wave_sum(x);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[4 + (threadIdx.x >> 6)] = x;
  __syncthreads();
  return (red[4] + red[5]) + (red[6] + red[7]);
}

template <uint32_t DT>
VM_DEV void dec_cvt8(const typename GemvRaw<DT>::T& r, float (&w)[8]) { gemv_cvt<DT>(r, w); }

// One split of one head.  Every global read the tile needs is issued before
// the first wait (the split's key range is fixed by C and S, not by pos): pos,
// q, the step's own k and v, the split's K^T columns and V rows.  So the tile
// pays one memory round trip, then the scores, the softmax and P.V come out of
// registers, lane shuffles and LDS.
template <uint32_t DT>
VM_DEV void decode_attn_split(Args A, uint32_t ti, uint32_t tile) {
  A = uargs(A);
  const VM_K Task& t = task_of(A, ti);
  const uint32_t hd = t.p[5] & 0xFFFF, C = t.p[6];
  const bool krow = (t.p[5] >> 16) & 1, masked = (t.p[5] >> 17) & 1;
  const uint32_t H = t.p[4] & 0xFFFF, S = max(1u, t.p[4] >> 16);
  const float scale = __uint_as_float(t.p[7]);
  tile = uni(tile);
  const uint32_t h = tile / S, split = tile % S;
  constexpr uint32_t esz = DT == DT_F32 ? 4 : 2;
  typedef typename GemvRaw<DT>::T Raw;
  const gbyte* q = resolve(A, t.a) + uint64_t(h) * hd * esz;
  const gbyte* kt = resolve(A, t.b) + uint64_t(h) * hd * C * esz;
  const gbyte* vc = resolve(A, t.p[0]) + uint64_t(h) * C * hd * esz;
  const gbyte* kn = resolve(A, t.p[1]) + uint64_t(h) * hd * esz;
  const gbyte* vn = resolve(A, t.p[2]) + uint64_t(h) * hd * esz;
  // the split's cache keys [k0, k0 + nk): whole octets (C is a multiple of 8)
  const uint32_t per = ((C + S - 1) / S + 7) & ~7u;          // <= kDecSplitKeys (loader check)
  const uint32_t k0 = min(split * per, C), nk = min(per, C - k0);
  const uint32_t tid = threadIdx.x, lane = tid & 63;

  // ---- every read up front -----------------------------------------------------
  const int32_t praw = __hip_atomic_load((const int32_t*)resolve(A, t.p[3]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // scores: thread (octet o = tid / 32, channel group dg = tid % 32) holds
  // channels dg, dg + 32, ... of keys [k0 + 8 o, +8); octets past nk re-read
  // the last one (discarded), channels past hd re-read hd - 1 (not accumulated)
  const uint32_t o = tid >> 5, dg = tid & 31;
  const uint32_t oc = nk ? min(o, nk / 8 - 1) : 0;
  const uint32_t kcol = min(k0 + 8 * oc, C - 8);
  const uint32_t dpt = (hd + 31) / 32;                        // <= kDecKU
  // P.V (and the key rows of krow): thread (cg = tid % cgp, rg = tid / cgp)
  // holds channels [8 cg, +8) of rows rg, rg + rpp, ...; rows past nk re-read
  // the last row (not accumulated).  cgs = hd / 8 threads cover a row; krow
  // rounds the group up to cgp, a power of two (dividing 64: hd <= 256), whose
  // threads past cgs re-read the row's last channels and add nothing.
  const uint32_t cgs = hd / 8;
  const uint32_t cgp = krow && cgs > 1 ? 1u << (32 - __builtin_clz(cgs - 1)) : cgs;
  const uint32_t rpp = kBlock / cgp;
  const uint32_t cg = tid % cgp, rg = min(tid / cgp, rpp - 1);
  const bool cg_on = cg < cgs;
  const uint32_t cg8 = min(cg, cgs - 1) * 8;               // channel offset read
  const uint32_t vpt = (per + rpp - 1) / rpp;                 // <= kDecKU
  Raw kr[kDecKU];
  float qd[kDecKU];
  Raw qrow;
  if (krow) {
    qrow = gemv_ld<DT>(q, cg8);
#pragma unroll
    for (uint32_t u = 0; u < kDecKU; ++u)
      if (u < vpt) {
        const uint32_t r = nk ? min(rg + rpp * u, nk - 1) : 0;
        kr[u] = gemv_ld<DT>(kt, uint64_t(min(k0 + r, C - 1)) * hd + cg8);
      }
  } else {
#pragma unroll
    for (uint32_t u = 0; u < kDecKU; ++u)
      if (u < dpt) {                                          // uniform: dpt is
        const uint32_t d = min(dg + 32 * u, hd - 1);
        kr[u] = gemv_ld<DT>(kt, uint64_t(d) * C + kcol);
        qd[u] = load_f(q, DT, d);
      }
  }
  Raw vr[kDecKU];
#pragma unroll
  for (uint32_t u = 0; u < kDecKU; ++u)
    if (u < vpt) {
      const uint32_t r = nk ? min(rg + rpp * u, nk - 1) : 0;
      vr[u] = gemv_ld<DT>(vc, (uint64_t(min(k0 + r, C - 1)) * hd + cg8));
    }
  const Raw vnew = gemv_ld<DT>(vn, cg8);
  float qn = 0.0f;
  if (tid < hd) qn = load_f(q, DT, tid) * load_f(kn, DT, tid);

  float* lds = lds_ptr<float>();
  float* sc = lds + kDecS;
  float* red = lds + kDecRed;
  float* part = lds + kDecPart;
  float* tmp = lds + kDecTmp;
  __syncthreads();                                   // the previous user of the LDS is done
  const float s_new = dec_block_sum(qn, red) * scale;   // the step's own key
  const int32_t pmax = masked ? int32_t(C) - 1 : int32_t(C);
  const uint32_t pos = uni(uint32_t(praw < 0 ? 0 : praw > pmax ? pmax : praw));
  const bool no_key = masked && praw < 0;            // every key masked: NaN

  // ---- scores of the split's cache keys ---------------------------------------
  if (krow) {
    float qv[8];
    gemv_cvt<DT>(qrow, qv);
#pragma unroll
    for (uint32_t u = 0; u < kDecKU; ++u)
      if (u < vpt) {                                          // uniform: vpt is
        float w[8];
        gemv_cvt<DT>(kr[u], w);
        float sdot = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) sdot = fmaf(qv[j], w[j], sdot);
        if (!cg_on) sdot = 0.0f;
        // the cgp threads of a key are adjacent lanes of one wave
        for (uint32_t msk = cgp >> 1; msk >= 1; msk >>= 1) sdot += __shfl_xor(sdot, msk, 64);
        const uint32_t r = rg + rpp * u;
        if (cg == 0 && r < nk) sc[r] = sdot * scale;
      }
  } else {
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
#pragma unroll
    for (uint32_t u = 0; u < kDecKU; ++u)
      if (u < dpt && dg + 32 * u < hd) {
        float w[8];
        gemv_cvt<DT>(kr[u], w);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = fmaf(qd[u], w[j], acc[j]);
      }
#pragma unroll
    for (int j = 0; j < 8; ++j)
      for (int msk = 16; msk >= 1; msk >>= 1) acc[j] += __shfl_xor(acc[j], msk, 64);
    if (dg == 0 && 8 * o < nk)
#pragma unroll
      for (int j = 0; j < 8; ++j) sc[8 * o + j] = acc[j] * scale;
  }
  __syncthreads();

  // ---- softmax over the split's keys up to pos (wave 0) -----------------------
  // key pos is the step's own (its cache column is not written yet)
  float m = -INFINITY, l = 0.0f;
  if (tid < 64) {
    const uint32_t key = k0 + lane;
    float sv = -INFINITY;
    if (lane < nk && key <= pos) sv = key == pos ? s_new : sc[lane];
    m = wave_max(sv);
    const float p = sv == -INFINITY ? 0.0f : expf(sv - m);
    l = wave_sum(p);
    sc[lane] = p;
    if (lane == 0) {
      red[8] = m;
      red[9] = l;
    }
  }
  // the step's own key when it lies past the cache (pos == C) belongs to the
  // last split
  const bool own_extra = pos == C && split == S - 1;
  __syncthreads();
  m = red[8];
  l = red[9];
  float p_own = 0.0f;
  if (own_extra) {                                   // one more key: rescale
    const float mn = fmaxf(m, s_new);
    const float a = m == -INFINITY ? 0.0f : expf(m - mn);
    p_own = expf(s_new - mn);
    l = l * a + p_own;
    // the cache keys' probabilities are rescaled by a below
    for (uint32_t j = tid; j < 64; j += kBlock) sc[j] *= a;
    m = mn;
    __syncthreads();
  }

  // ---- P.V ----------------------------------------------------------------------
  float ov[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) ov[j] = 0.0f;
  if (tid / cgp < rpp && cg_on) {
#pragma unroll
    for (uint32_t u = 0; u < kDecKU; ++u) {
      const uint32_t r = rg + rpp * u;
      if (u < vpt && r < nk) {
        float w[8];
        gemv_cvt<DT>(k0 + r == pos ? vnew : vr[u], w);
        const float p = sc[r];
#pragma unroll
        for (int j = 0; j < 8; ++j) ov[j] = fmaf(p, w[j], ov[j]);
      }
    }
    if (own_extra && rg == 0) {
      float w[8];
      gemv_cvt<DT>(vnew, w);
#pragma unroll
      for (int j = 0; j < 8; ++j) ov[j] = fmaf(p_own, w[j], ov[j]);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) part[rg * hd + cg * 8 + j] = ov[j];
  }
  __syncthreads();
  // sum the rpp row groups in a fixed order: J threads per channel, then one
  const uint32_t J = kBlock / hd;
  {
    const uint32_t c = tid % hd, jj = tid / hd;
    if (jj < J) {
      float v = 0.0f;
      for (uint32_t r = jj; r < rpp; r += J) v += part[r * hd + c];
      tmp[jj * hd + c] = v;
    }
  }
  __syncthreads();
  float oacc = 0.0f;
  if (tid < hd)
    for (uint32_t jj = 0; jj < J; ++jj) oacc += tmp[jj * hd + tid];

  gbyte* out = resolve(A, t.dst) + uint64_t(h) * hd * esz;
  if (S == 1) {
    if (tid < hd) store_f(out, DT, tid, no_key ? __builtin_nanf("") : oacc / l);
    return;
  }
  // split: publish the partial, count the arrival; the last split combines.
  // The partials are agent-scope atomic stores; the workgroup barrier orders
  // every thread's stores before thread 0's arrival, an agent-scope
  // acquire-release read-modify-write: its release publishes this workgroup's
  // partials to the other XCDs, its acquire (observed by the last arriver)
  // makes every earlier split's partials visible before the combine reads them.
  uint32_t* sp = reinterpret_cast<uint32_t*>(A->scratch + A->task_scratch[ti]);
  uint32_t* arrivals = sp + uint64_t(H) * S * (hd + 2);
  uint32_t* mine = sp + uint64_t(h * S + split) * (hd + 2);
  if (tid < hd) __hip_atomic_store(mine + 2 + tid, __float_as_uint(oacc), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (tid == 0) {
    __hip_atomic_store(mine, __float_as_uint(m), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(mine + 1, __float_as_uint(l), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);                 // vmcnt(0): this thread's stores are done
  __syncthreads();
  uint32_t* flag = reinterpret_cast<uint32_t*>(red + 12);
  if (tid == 0) {
    const uint32_t before = __hip_atomic_fetch_add(arrivals + h, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = before == S - 1;
    // reset for the next run of this task (ordered before it by a grid barrier)
    if (last) __hip_atomic_store(arrivals + h, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag = last;
  }
  __syncthreads();
  if (!*flag) return;
  // combine in split order; every read issued in parallel
  const uint32_t* hp = sp + uint64_t(h) * S * (hd + 2);
  auto rd = [](const uint32_t* p) {
    return __uint_as_float(__hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  };
  float* ms = part;                                  // [S] maxima, then weights
  float* ls = part + kDecMaxSplits;                  // [S] sums
  for (uint32_t k = tid; k < S; k += kBlock) {
    ms[k] = rd(hp + k * (hd + 2));
    ls[k] = rd(hp + k * (hd + 2) + 1);
  }
  __syncthreads();
  float M = -INFINITY;
  for (uint32_t k = 0; k < S; ++k) M = fmaxf(M, ms[k]);
  __syncthreads();
  for (uint32_t k = tid; k < S; k += kBlock) ms[k] = ms[k] == -INFINITY ? 0.0f : expf(ms[k] - M);
  __syncthreads();
  if (tid < hd) {
    float L = 0.0f, O = 0.0f;
    constexpr int B = 8;
    for (uint32_t k0b = 0; k0b < S; k0b += B) {
      float o8[B];
#pragma unroll
      for (int u = 0; u < B; ++u) o8[u] = rd(hp + min(k0b + u, S - 1) * (hd + 2) + 2 + tid);
#pragma unroll
      for (int u = 0; u < B; ++u)
        if (k0b + u < S) {
          L = fmaf(ls[k0b + u], ms[k0b + u], L);
          O = fmaf(o8[u], ms[k0b + u], O);
        }
    }
    store_f(out, DT, tid, no_key ? __builtin_nanf("") : O / L);
  }
}

// One leaf per dtype with the split inlined, for the reason gemv_run gives.
template <uint32_t DT>
VM_LEAF void decode_attn_run(Args A, uint32_t ti, uint32_t lo, uint32_t hi) {
  A = uargs(A);
  lo = uni(lo);
  hi = uni(hi);
  for (uint32_t tile = lo; tile < hi; ++tile) decode_attn_split<DT>(A, ti, tile);
}

VM_DEV void decode_attn_tiles(Args A, uint32_t ti, uint32_t lo, uint32_t hi) {
  const VM_K Task& t = task_of(A, ti);
  const uint32_t dt = (t.tile_op >> 8) & 0xFF;
  hi = min(hi, max(1u, (t.p[4] & 0xFFFF) * max(1u, t.p[4] >> 16)));
  if (dt == DT_BF16) decode_attn_run<DT_BF16>(A, ti, lo, hi);
  else if (dt == DT_F16) decode_attn_run<DT_F16>(A, ti, lo, hi);
  else decode_attn_run<DT_F32>(A, ti, lo, hi);
}

}  // namespace vm
