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
// Task: a q, b K^T cache [H, hd, C], p0 V cache [H, C, hd], p1 k, p2 v, p3 pos
// (i32 scalar, clamped to [0, C]), p4 H, p5 hd (multiple of 8, <= 256), p6 C
// (multiple of 8), p7 scale bits.  One dtype (bf16 / f16 / f32) for every
// operand and the output; f32 arithmetic.
#pragma once
#include "tile_gemv.h"

namespace vm {

constexpr uint32_t kDecKeys = 1024;                 // keys per chunk: 128 octets of 8
// LDS, in floats: q [256], reduction slots [16], chunk scores / probabilities
// [1024], then the two score halves [2][1024], reused for the P.V partials
constexpr uint32_t kDecQ = 0, kDecRed = 256, kDecS = 272, kDecPart = kDecS + kDecKeys;
constexpr uint32_t kDecLdsBytes = (kDecPart + 2 * kDecKeys) * 4;

VM_DEV float dec_block_max(float x, float* red) {
  x = wave_max(x);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

VM_DEV float dec_block_sum(float x, float* red) {
  x = wave_sum(x);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[4 + (threadIdx.x >> 6)] = x;
  __syncthreads();
  return (red[4] + red[5]) + (red[6] + red[7]);
}

template <uint32_t DT>
VM_TILE void decode_attn_head(Args A, uint32_t ti, uint32_t h) {
  A = uargs(A);
  const VM_K Task& t = task_of(A, ti);
  const uint32_t hd = t.p[5], C = t.p[6];
  const float scale = __uint_as_float(t.p[7]);
  h = uni(h);
  constexpr uint32_t esz = DT == DT_F32 ? 4 : 2;
  constexpr int kU = DT == DT_F32 ? 8 : 16;          // loads per batch and thread
  typedef typename GemvRaw<DT>::T Raw;
  const gbyte* q = resolve(A, t.a) + uint64_t(h) * hd * esz;
  const gbyte* kt = resolve(A, t.b) + uint64_t(h) * hd * C * esz;
  const gbyte* vc = resolve(A, t.p[0]) + uint64_t(h) * C * hd * esz;
  const gbyte* kn = resolve(A, t.p[1]) + uint64_t(h) * hd * esz;
  const gbyte* vn = resolve(A, t.p[2]) + uint64_t(h) * hd * esz;
  const int64_t praw = read_index(resolve(A, t.p[3]), false);
  const uint32_t pos = uni(uint32_t(praw < 0 ? 0 : praw > int64_t(C) ? int64_t(C) : praw));
  const uint32_t n = pos + 1;                        // keys, the step's own included

  float* lds = reinterpret_cast<float*>(vm_smem);
  float* qs = lds + kDecQ;
  float* red = lds + kDecRed;
  float* sc = lds + kDecS;
  float* part = lds + kDecPart;
  const uint32_t tid = threadIdx.x;

  __syncthreads();                                   // the previous user of the LDS is done
  float qn = 0.0f;
  if (tid < hd) {
    const float qv = load_f(q, DT, tid);
    qs[tid] = qv;
    qn = qv * load_f(kn, DT, tid);
  }
  const float s_new = dec_block_sum(qn, red) * scale;   // the step's own key (syncs: qs visible)

  // score pass: thread (octet o, half hh) owns keys [8o, 8o + 8) of the chunk
  // over channels [hh hd/2, (hh + 1) hd/2)
  const uint32_t o = tid & 127, hh = tid >> 7;
  const uint32_t dh = hd / 2, d0 = hh * dh, dend = d0 + dh;
  // P.V pass: gsz threads per V row (8 channels each), R rows at a time
  const uint32_t gsz = hd / 8, R = kBlock / gsz;
  const uint32_t cgi = tid % gsz, rgi = tid / gsz;

  float m = -INFINITY, l = 0.0f, oacc = 0.0f;
  for (uint32_t c0 = 0; c0 < n; c0 += kDecKeys) {
    const uint32_t cnt = min(kDecKeys, n - c0);
    const uint32_t kb = c0 + 8 * o;
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
    if (kb < pos) {                                  // kb + 8 <= C: C is a multiple of 8
      Raw ra[kU], rb[kU];
      auto issue = [&](Raw (&r)[kU], uint32_t d) {
#pragma unroll
        for (int u = 0; u < kU; ++u) r[u] = gemv_ld<DT>(kt, uint64_t(min(d + u, dend - 1)) * C + kb);
      };
      auto consume = [&](const Raw (&r)[kU], uint32_t d) {
#pragma unroll
        for (int u = 0; u < kU; ++u)
          if (d + u < dend) {
            float w[8];
            gemv_cvt<DT>(r[u], w);
            const float qd = qs[d + u];
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[j] = fmaf(qd, w[j], acc[j]);
          }
      };
      issue(ra, d0);
      for (uint32_t d = d0;; d += 2 * kU) {
        if (d + kU < dend) issue(rb, d + kU);
        consume(ra, d);
        if (d + kU >= dend) break;
        if (d + 2 * kU < dend) issue(ra, d + 2 * kU);
        consume(rb, d + kU);
        if (d + 2 * kU >= dend) break;
      }
    }
    *(v4f*)(part + hh * kDecKeys + 8 * o) = v4f{acc[0], acc[1], acc[2], acc[3]};
    *(v4f*)(part + hh * kDecKeys + 8 * o + 4) = v4f{acc[4], acc[5], acc[6], acc[7]};
    __syncthreads();

    float mx = -INFINITY;
    for (uint32_t j = tid; j < cnt; j += kBlock) {
      const float s = c0 + j == pos ? s_new : (part[j] + part[kDecKeys + j]) * scale;
      sc[j] = s;
      mx = fmaxf(mx, s);
    }
    const float mnew = fmaxf(m, dec_block_max(mx, red));
    const float alpha = expf(m - mnew);              // 0 on the first chunk
    float ps = 0.0f;
    for (uint32_t j = tid; j < cnt; j += kBlock) {
      const float p = expf(sc[j] - mnew);
      sc[j] = p;
      ps += p;
    }
    l = l * alpha + dec_block_sum(ps, red);          // syncs: sc and part free / visible
    m = mnew;

    // P.V over the chunk's rows; rows past cnt re-read the chunk's last row and
    // are not accumulated, so no load sits behind a branch
    float pacc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) pacc[j] = 0.0f;
    if (rgi < R) {
      auto vrow = [&](uint32_t r) -> const gbyte* {
        const uint32_t key = c0 + min(r, cnt - 1);
        return key == pos ? vn + cgi * 8 * esz : vc + (uint64_t(key) * hd + cgi * 8) * esz;
      };
      Raw va[kU], vb[kU];
      auto issue = [&](Raw (&r)[kU], uint32_t r0) {
#pragma unroll
        for (int u = 0; u < kU; ++u) r[u] = gemv_ld<DT>(vrow(r0 + u * R), 0);
      };
      auto consume = [&](const Raw (&r)[kU], uint32_t r0) {
#pragma unroll
        for (int u = 0; u < kU; ++u)
          if (r0 + u * R < cnt) {
            float w[8];
            gemv_cvt<DT>(r[u], w);
            const float p = sc[r0 + u * R];
#pragma unroll
            for (int j = 0; j < 8; ++j) pacc[j] = fmaf(p, w[j], pacc[j]);
          }
      };
      const uint32_t step = kU * R;
      issue(va, rgi);
      for (uint32_t r = rgi;; r += 2 * step) {
        if (r + step < cnt) issue(vb, r + step);
        consume(va, r);
        if (r + step >= cnt) break;
        if (r + 2 * step < cnt) issue(va, r + 2 * step);
        consume(vb, r + step);
        if (r + 2 * step >= cnt) break;
      }
      *(v4f*)(part + rgi * hd + cgi * 8) = v4f{pacc[0], pacc[1], pacc[2], pacc[3]};
      *(v4f*)(part + rgi * hd + cgi * 8 + 4) = v4f{pacc[4], pacc[5], pacc[6], pacc[7]};
    }
    __syncthreads();
    if (tid < hd) {
      float s = 0.0f;
      for (uint32_t g = 0; g < R; ++g) s += part[g * hd + tid];
      oacc = oacc * alpha + s;
    }
    __syncthreads();                                 // part / sc reused by the next chunk
  }
  if (tid < hd) store_f(resolve(A, t.dst) + uint64_t(h) * hd * esz, DT, tid, oacc / l);
}

VM_TILE void decode_attn_tiles(Args A, uint32_t ti, uint32_t lo, uint32_t hi) {
  A = uargs(A);
  const VM_K Task& t = task_of(A, ti);
  const uint32_t dt = (t.tile_op >> 8) & 0xFF;
  hi = min(hi, max(1u, t.p[4]));
  for (uint32_t h = lo; h < hi; ++h) {
    if (dt == DT_BF16) decode_attn_head<DT_BF16>(A, ti, h);
    else if (dt == DT_F16) decode_attn_head<DT_F16>(A, ti, h);
    else decode_attn_head<DT_F32>(A, ti, h);
  }
}

}  // namespace vm
