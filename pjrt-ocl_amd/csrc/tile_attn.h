// TOP_FLASH_ATTN: O = softmax(scale * Q K^T [causal]) V per head, online softmax
// with f32 statistics (reference semantics: ops/attention.cl:49-159,
// python/pjrt_ocl/ops/attention.py:53-64).  Task: a = Q, b = K, p0 = V,
// p1 = H, p2 = T, p3 = aux descriptor {H, T, C, hd, scale bits, causal, qv, kv, vv}.
// Tiles are query rows (H*T of them); causal masks key c > m + (C - T).
//
// Matrix-core path (bf16/f16, hd = 64 or 128, K read through the usual [H,hd,C]
// transpose view of a [H,C,hd] buffer): a lane takes 128 query rows, 32 per
// wave, and streams K/V in 32-key blocks staged through LDS.  Each wave computes
//   S^T (32 keys x 32 queries) = K_blk (32 x hd) . Q^T (hd x 32)
// so both MFMA operands are contiguous along hd, and the S^T accumulators are
// already the B operand of
//   O^T (hd x 32 queries) += V_blk^T (hd x 32 keys) . P^T (32 keys x 32 queries).
// Key rows of a block are permuted (kperm) so that the 8 keys a lane holds per
// 16-key MFMA step are consecutive.  Causal query blocks are visited in zig-zag
// order (block b, then nb-1-b) so contiguous tile chunks cost the same.
#pragma once
#include "tile_ew.h"
#include "tile_mma.h"
#include "tile_reduce.h"
#include "vm_math.h"

namespace vm {

constexpr int kAttnKeys = 32;            // keys per streamed block
constexpr int kAttnRows = 128;           // query rows per lane step (4 waves x 32)
constexpr int kAttnLdK = 128 + 8;        // K row stride (elements): 16-byte aligned rows
constexpr int kAttnLdV = 128 + 4;        // V row stride: odd multiple of 8 bytes
constexpr int kAttnBuf = kAttnKeys * (kAttnLdK + kAttnLdV);     // elements per buffer
constexpr int kAttnLdsBytes = 2 * kAttnBuf * 2;

// Row r of an S^T accumulator block holds key kperm(r) of the 32-key block:
// r = 8j + 4g + i (j = v/4 register group, g = lane/32, i = v%4) -> key
// 16*(j/2) + 8g + 4*(j%2) + i, so lane group g owns keys 16s + 8g + 0..7 in
// MFMA step s (registers 8s..8s+7).
VM_DEV uint32_t kperm(uint32_t r) {
  const uint32_t j = r >> 3, g = (r >> 2) & 1, i = r & 3;
  return 16 * (j >> 1) + 8 * g + 4 * (j & 1) + i;
}

VM_DEV float xor32(float x) { return __shfl_xor(x, 32); }

struct AttnDesc {
  uint32_t H, T, C, hd;
  float scale;
  bool causal;
  uint32_t qv, kv, vv;
};
VM_DEV AttnDesc attn_desc(Args A, const VM_K Task& t) {
  const VM_K int32_t* d = aux_of(A) + t.p[3];
  AttnDesc D;
  D.H = d[0];
  D.T = d[1];
  D.C = d[2];
  D.hd = d[3];
  D.scale = __int_as_float(d[4]);
  D.causal = d[5] != 0;
  D.qv = d[6];
  D.kv = d[7];
  D.vv = d[8];
  return D;
}

template <int HD, bool BF16>
VM_TILE void attn_block_mfma(Args A, uint32_t ti, uint32_t h, uint32_t row0, uint32_t vrow0, uint32_t vlo,
                             uint32_t vhi) {
  A = uargs(A);
  const VM_K Task& t = task_of(A, ti);
  const AttnDesc P = attn_desc(A, t);
  h = uni(h);
  row0 = uni(row0);
  vrow0 = uni(vrow0);
  vlo = uni(vlo);
  vhi = uni(vhi);
  const uint32_t T = P.T, C = P.C, dt = (t.tile_op >> 8) & 0xFF;
  uint16_t* lds = reinterpret_cast<uint16_t*>(vm_smem);
  constexpr int KS = HD / 16;            // MFMA steps over hd for S
  constexpr int DB = HD / 32;            // 32-row d blocks of O^T
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 5;
  const uint32_t qloc = wave * 32 + (lane & 31);           // 0..127 within the block
  const uint32_t q = row0 + qloc;                           // real query row
  const bool qvalid = q < T && vrow0 + qloc >= vlo && vrow0 + qloc < vhi;
  const VM_G uint16_t* Q = gcast<uint16_t>(resolve(A, t.a)) + uint64_t(h) * T * HD;
  const VM_G uint16_t* K = gcast<uint16_t>(resolve(A, t.b)) + uint64_t(h) * C * HD;
  const VM_G uint16_t* V = gcast<uint16_t>(resolve(A, t.p[0])) + uint64_t(h) * C * HD;
  gbyte* Ob = resolve(A, t.dst);

  // Q^T fragments (B operand): column = query, 8 consecutive hd values.
  u16x8 qf[KS];
  {
    const uint32_t qr = q < T ? q : T - 1;
#pragma unroll
    for (int s = 0; s < KS; ++s) qf[s] = *(const VM_G u16x8*)(Q + uint64_t(qr) * HD + s * 16 + 8 * g);
  }
  f32x16 o[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i) o[i] = f32x16{};
  float m_run = -INFINITY, l_run = 0.0f;
  const float sl2 = P.scale * 1.4426950408889634f;

  // keys this block needs: up to the last query's causal limit
  const uint32_t qmax = min(row0 + kAttnRows, T) - 1;
  uint32_t kend = C;
  if (P.causal) kend = min(C, uint32_t(max(0, int(qmax) + int(C) - int(T) + 1)));
  const uint32_t nblk = (kend + kAttnKeys - 1) / kAttnKeys;

  // staging: K and V blocks are 32 x HD = 4*HD chunks of 8 elements each
  constexpr int kChunks = kAttnKeys * HD / 8 / kBlock;      // per tensor per thread
  v4u rk[kChunks], rv[kChunks];
  auto gload = [&](uint32_t kb) {
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
      const uint32_t c = threadIdx.x + j * kBlock;
      const uint32_t r = c / (HD / 8), cc = (c % (HD / 8)) * 8;
      const uint32_t key = kb * kAttnKeys + r;
      if (key < C) {
        rk[j] = *(const VM_G v4u*)(K + uint64_t(key) * HD + cc);
        rv[j] = *(const VM_G v4u*)(V + uint64_t(key) * HD + cc);
      } else {
        rk[j] = v4u_make(0, 0, 0, 0);
        rv[j] = v4u_make(0, 0, 0, 0);
      }
    }
  };
  auto lstore = [&](uint16_t* buf) {
    uint16_t* lk = buf;
    uint16_t* lv = buf + kAttnKeys * kAttnLdK;
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
      const uint32_t c = threadIdx.x + j * kBlock;
      const uint32_t r = c / (HD / 8), cc = (c % (HD / 8)) * 8;
      *reinterpret_cast<v4u*>(lk + r * kAttnLdK + cc) = rk[j];
      v2u* pv = reinterpret_cast<v2u*>(lv + r * kAttnLdV + cc);
      pv[0] = v2u_make(rv[j].x, rv[j].y);
      pv[1] = v2u_make(rv[j].z, rv[j].w);
    }
  };

  __syncthreads();                      // LDS free from the previous user
  if (nblk) {
    gload(0);
    lstore(lds);
  }
  __syncthreads();
  const int32_t qlim = int32_t(q) + int32_t(C) - int32_t(T);     // last visible key
  const uint32_t krow = kperm(lane & 31);
  for (uint32_t kb = 0; kb < nblk; ++kb) {
    const uint16_t* buf = lds + (kb & 1) * kAttnBuf;
    const uint16_t* lk = buf;
    const uint16_t* lv = buf + kAttnKeys * kAttnLdK;
    if (kb + 1 < nblk) gload(kb + 1);
    // S^T = K_blk . Q^T
    f32x16 s = f32x16{};
#pragma unroll
    for (int st = 0; st < KS; ++st) {
      const u16x8 kf = *reinterpret_cast<const u16x8*>(lk + krow * kAttnLdK + st * 16 + 8 * g);
      s = mfma16<BF16>(kf, qf[st], s);
    }
    // scale, mask, online softmax (each query lives in lanes l and l^32)
    const uint32_t key0 = kb * kAttnKeys;
    float p[16];
    float mx = -INFINITY;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const uint32_t r = 8 * (v >> 2) + 4 * g + (v & 3);
      const int32_t key = int32_t(key0 + kperm(r));
      float x = s[v] * sl2;
      if (key >= int32_t(C) || (P.causal && key > qlim)) x = -INFINITY;
      p[v] = x;
      mx = fmaxf(mx, x);
    }
    mx = fmaxf(mx, xor32(mx));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    float rs = 0.0f;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      p[v] = __builtin_amdgcn_exp2f(p[v] - m_use);
      rs += p[v];
    }
    rs += xor32(rs);
    l_run = l_run * alpha + rs;
    m_run = m_new;
#pragma unroll
    for (int i = 0; i < DB; ++i) o[i] *= alpha;
    // P^T fragments: registers 8s..8s+7 = keys 16s + 8g + 0..7
    u16x8 pf[2];
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int e = 0; e < 8; ++e) pf[st][e] = uint16_t(BF16 ? f32_to_bf16(p[8 * st + e]) : f32_to_f16(p[8 * st + e]));
    // O^T += V^T . P^T
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const uint32_t d = db * 32 + (lane & 31);
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        u16x8 vf;
        const uint32_t kr = 16 * st + 8 * g;
#pragma unroll
        for (int e = 0; e < 8; ++e) vf[e] = lv[(kr + e) * kAttnLdV + d];
        o[db] = mfma16<BF16>(vf, pf[st], o[db]);
      }
    }
    if (kb + 1 < nblk) lstore(lds + ((kb + 1) & 1) * kAttnBuf);
    __syncthreads();
  }
  if (qvalid) {
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    const uint64_t obase = (uint64_t(h) * T + q) * HD;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t d = db * 32 + 8 * j + 4 * g;
        st4(Ob, dt, obase + d,
            v4f_make(o[db][4 * j] * inv, o[db][4 * j + 1] * inv, o[db][4 * j + 2] * inv, o[db][4 * j + 3] * inv));
      }
    }
  }
}

// Generic path: any head size, dtype or view.  One wave per query row; lanes split
// the keys of a 64-key chunk, then the hd outputs.
VM_TILE void attn_rows_generic(Args A, uint32_t ti, uint32_t lo, uint32_t hi) {
  A = uargs(A);
  const VM_K Task& t = task_of(A, ti);
  const AttnDesc P = attn_desc(A, t);
  const VM_K int32_t* aux = aux_of(A);
  const uint32_t H = P.H, T = P.T, C = P.C, hd = P.hd;
  const uint32_t dt = (t.tile_op >> 8) & 0xFF, adt = (t.tile_op >> 16) & 0xFF;
  const gbyte* Qb = resolve(A, t.a);
  const gbyte* Kb = resolve(A, t.b);
  const gbyte* Vb = resolve(A, t.p[0]);
  gbyte* Ob = resolve(A, t.dst);
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  hi = min(hi, H * T);
  constexpr int kMaxD = 4;               // hd <= 256
  for (uint32_t tile = lo + wave; tile < hi; tile += kWaves) {
    const uint32_t h = tile / T, m = tile % T;
    const int32_t qlim = int32_t(m) + int32_t(C) - int32_t(T);
    float mrun = -INFINITY, lrun = 0.0f;
    float o[kMaxD] = {0.f, 0.f, 0.f, 0.f};
    for (uint32_t c0 = 0; c0 < C; c0 += 64) {
      const uint32_t c = c0 + lane;
      float sc = -INFINITY;
      if (c < C && !(P.causal && int32_t(c) > qlim)) {
        float acc = 0.0f;
        for (uint32_t d = 0; d < hd; ++d) {
          const uint64_t qi = (uint64_t(h) * T + m) * hd + d;
          const uint64_t ki = (uint64_t(h) * hd + d) * C + c;      // K as [H, hd, C]
          const float qx = load_f(Qb, adt, P.qv ? uint64_t(view_index(aux, P.qv - 1, qi)) : qi);
          const float kx = load_f(Kb, adt, P.kv ? uint64_t(view_index(aux, P.kv - 1, ki)) : ki);
          acc = fmaf(qx, kx, acc);
        }
        sc = acc * P.scale;
      }
      const float mx = wave_max(sc);
      const float mnew = fmaxf(mrun, mx);
      const float muse = mnew == -INFINITY ? 0.0f : mnew;
      const float alpha = __expf(mrun - muse);
      const float pk = __expf(sc - muse);
      lrun = lrun * alpha + wave_sum(pk);
      mrun = mnew;
#pragma unroll
      for (int j = 0; j < kMaxD; ++j) o[j] *= alpha;
      const uint32_t cn = min(64u, C - c0);
      for (uint32_t k = 0; k < cn; ++k) {
        const float pb = lane_read(pk, k);
#pragma unroll
        for (int j = 0; j < kMaxD; ++j) {
          const uint32_t d = lane + 64 * j;
          if (d < hd) {
            const uint64_t vi = (uint64_t(h) * C + c0 + k) * hd + d;
            o[j] = fmaf(pb, load_f(Vb, adt, P.vv ? uint64_t(view_index(aux, P.vv - 1, vi)) : vi), o[j]);
          }
        }
      }
    }
    const float inv = lrun > 0.0f ? 1.0f / lrun : 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxD; ++j) {
      const uint32_t d = lane + 64 * j;
      if (d < hd) store_f(Ob, dt, (uint64_t(h) * T + m) * hd + d, o[j] * inv);
    }
  }
}

// Is view `kv` the plain transpose [H, hd, C] of a contiguous [H, C, hd] buffer?
VM_DEV bool is_kt_view(const VM_K int32_t* aux, uint32_t kv, uint32_t H, uint32_t C, uint32_t hd) {
  if (!kv) return false;
  const VM_K int32_t* x = aux + (kv - 1);
  return x[0] == 3 && uint32_t(x[1]) == H && uint32_t(x[2]) == hd && uint32_t(x[3]) == C &&
         uint32_t(x[4]) == C * hd && x[5] == 1 && uint32_t(x[6]) == hd && x[7] == 0;
}

VM_TILE void flash_attn_tiles(Args A, uint32_t ti, uint32_t lo, uint32_t hi) {
  A = uargs(A);
  const VM_K Task& t = task_of(A, ti);
  const AttnDesc P = attn_desc(A, t);
  const uint32_t adt = (t.tile_op >> 16) & 0xFF, dt = (t.tile_op >> 8) & 0xFF;
  const bool fast = (adt == DT_BF16 || adt == DT_F16) && (P.hd == 64 || P.hd == 128) && !P.qv && !P.vv &&
                    is_kt_view(aux_of(A), P.kv, P.H, P.C, P.hd) && (P.T % kAttnRows) == 0 &&
                    (dt == DT_F32 || dt == DT_BF16 || dt == DT_F16);
  if (!fast) return attn_rows_generic(A, ti, lo, hi);
  const uint32_t T = P.T;
  hi = min(hi, P.H * T);
  const uint32_t nb = T / kAttnRows;
  // virtual 128-row blocks intersecting [lo, hi)
  for (uint32_t vb0 = (lo / kAttnRows) * kAttnRows; vb0 < hi; vb0 += kAttnRows) {
    const uint32_t h = vb0 / T, vb = (vb0 % T) / kAttnRows;
    const uint32_t rb = P.causal ? ((vb & 1) ? nb - 1 - (vb >> 1) : (vb >> 1)) : vb;
    const uint32_t row0 = rb * kAttnRows, vrow0 = vb0 % T;
    const uint32_t vlo = (lo > vb0 ? lo - vb0 : 0u) + vrow0;      // valid virtual rows
    const uint32_t vhi = min(hi - vb0, uint32_t(kAttnRows)) + vrow0;
    if (adt == DT_BF16) {
      if (P.hd == 128) attn_block_mfma<128, true>(A, ti, h, row0, vrow0, vlo, vhi);
      else attn_block_mfma<64, true>(A, ti, h, row0, vrow0, vlo, vhi);
    } else {
      if (P.hd == 128) attn_block_mfma<128, false>(A, ti, h, row0, vrow0, vlo, vhi);
      else attn_block_mfma<64, false>(A, ti, h, row0, vrow0, vlo, vhi);
    }
  }
}

}  // namespace vm
