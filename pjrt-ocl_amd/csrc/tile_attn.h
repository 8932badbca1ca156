// TOP_FLASH_ATTN: O = softmax(scale * Q K^T [causal]) V per head, online softmax
// with f32 statistics (reference semantics: ops/attention.cl:49-159,
// python/pjrt_ocl/ops/attention.py:53-64).  Task: a = Q, b = K, p0 = V,
// p1 = H, p2 = T, p3 = aux descriptor {H, T, C, hd, scale bits, causal, qv, kv, vv}.
// Tiles are query rows, each head's padded to whole 256-row blocks (H * Tp tiles,
// Tp = T rounded up to 256; tiles past T are empty); causal masks key c > m + (C - T).
// Four paths, all in one leaf (flash_attn_tiles): the 16-bit matrix-core path
// below (attn_block_mfma), f32 operands (attn_block_f32), 16-bit rows wider than
// 128 (attn_block_h16w), and the general row kernel (attn_rows_generic).
//
// Matrix-core path (bf16/f16, hd = 64 or 128, or any other multiple of 8 up to
// 128 run as the next of the two on zero-padded rows, scale > 0, K read through
// the usual [H,hd,C] transpose view of a [H,C,hd] buffer): a lane takes 256 query rows, 64
// per wave as two 32-row sub-tiles, and streams K/V in 64-key blocks that go
// from global memory straight into LDS (global_load_lds_dwordx4; double-buffered,
// one barrier per block).  Per sub-tile each wave computes
//   S^T (keys x 32 queries) = K_blk (keys x hd) . Q^T (hd x 32)
// so both MFMA operands are contiguous along hd, and the S^T accumulators are
// already the B operand of
//   O^T (hd x 32 queries) += V_blk^T (hd x keys) . P^T (keys x 32 queries).
// K and V blocks keep their [key][hd] layout in LDS, rows dense, 16-byte hd
// chunks at swizzled slots (kswz, vswz).  A K fragment is one ds_read_b128; an A
// fragment of V^T (8 consecutive keys of one hd column per lane) is two
// ds_read_b64_tr_b16 (in each group of 16 lanes, lane 4e + q points at key row
// k0 + e, hd columns d0 + 4q .. +3, and receives column d0 + lane % 16 at rows
// k0 .. k0 + 3).  Key rows of a 32-key half are read permuted (kperm) so that
// the 8 keys a lane holds per 16-key MFMA step are consecutive.  K and V
// fragments are read once per wave and used by both sub-tiles.
//
// Softmax in base 2 against a per-row reference maximum fixed at the row's first
// block with a visible key (the same algebra as the online update, with the
// rescale factor folded into the reference): O and l accumulate exp2(scale' s -
// m_ref), so no accumulator is ever rescaled inside the key loop.  Should a later
// block's probabilities exceed 2^24 (2^14 for f16) the 256-row block is redone
// with exact row maxima (a max-only pass, then probabilities <= 1).  The row sum
// is kept per lane and the two lanes holding a row are added at the end.  Causal
// query blocks are visited in zig-zag order (block b, then nb-1-b) so contiguous
// tile chunks cost the same.
#pragma once
#include "tile_ew.h"
#include "tile_mma.h"
#include "tile_reduce.h"
#include "vm_math.h"

namespace vm {

constexpr int kAttnKeys = 64;            // keys per streamed block
constexpr int kAttnRows = 256;           // query rows per lane step (4 waves x 64)
template <int HD>
struct AttnLds {
  static constexpr uint32_t kRow = HD * 2;                    // bytes per key row
  static constexpr uint32_t kKBytes = kAttnKeys * kRow;       // K block; V block follows
  static constexpr uint32_t kStage = 2 * kKBytes;
  static constexpr uint32_t kRounds = kKBytes / 4096;         // block-wide 16-byte transfers per operand
  static constexpr int kBytes = 2 * int(kStage);
};
// f32 path (attn_block_f32): keys per streamed block, query rows per block, and
// its two LDS buffers of K and V rows padded to HD + 2 floats
constexpr int kAttnF32Keys = 32;
constexpr int kAttnF32Rows = 128;
template <int HD>
struct AttnF32Lds {
  static constexpr uint32_t kRS = HD + 2;                       // floats per LDS row
  static constexpr uint32_t kOp = kAttnF32Keys * kRS;           // floats per operand block
  static constexpr uint32_t kBuf = 2 * kOp;                     // K block, then V block
  static constexpr int kBytes = int(2 * kBuf * 4);              // two buffers
};
constexpr int kAttnF32LdsBytes = AttnF32Lds<128>::kBytes;
// wide 16-bit path (attn_block_h16w, hd up to 256): 32-key blocks of K rows padded
// to 528 bytes and V rows padded to 576 bytes, two buffers
constexpr uint32_t kAttnWKRow = 528, kAttnWVRow = 576;
constexpr uint32_t kAttnWBuf = kAttnF32Keys * (kAttnWKRow + kAttnWVRow);
constexpr int kAttnWLdsBytes = int(2 * kAttnWBuf);
constexpr int kAttnLdsBytes0 = AttnLds<128>::kBytes > kAttnF32LdsBytes ? AttnLds<128>::kBytes : kAttnF32LdsBytes;
constexpr int kAttnLdsBytes = kAttnLdsBytes0 > kAttnWLdsBytes ? kAttnLdsBytes0 : kAttnWLdsBytes;

// Slot swizzles of the 16-byte hd chunks of key row r (chunk c at slot c ^ swz).
// K (ds_read_b128 fragments, rows kperm-ordered): distinct bank groups for any 16
// consecutive lanes and for lanes 0-7 with 32-39.  V (transposed reads of four
// consecutive rows, 64 bytes each, per half wave): the four rows' pieces cover
// the 64 banks once.
template <int HD>
VM_DEV uint32_t kswz(uint32_t r) {
  if constexpr (HD == 128) return (((r & 3) | (((r >> 3) & 1) << 2)) << 1) | ((r >> 2) & 1);
  else return ((((r >> 1) & 1) | (((r >> 3) & 1) << 1)) << 1) | ((r >> 2) & 1);
}
template <int HD>
VM_DEV uint32_t vswz(uint32_t r) {
  if constexpr (HD == 128) return 4 * (r & 3);
  else return 4 * ((r >> 1) & 1);
}

// Row r of an S^T accumulator block holds key kperm(r) of the 32-key half:
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

// c + lo(x) + hi(x) for a packed bf16 / f16 pair (v_dot2_f32_{bf16,f16} with 1, 1)
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
template <bool BF16>
VM_DEV float dot2_ones(uint32_t x, float c) {
  if constexpr (BF16)
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, x), __builtin_bit_cast(bf16x2_t, 0x3F803F80u),
                                           c, false);
  else
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, x), __builtin_bit_cast(f16x2_t, 0x3C003C00u), c, false);
}

template <bool BF16>
VM_DEV uint32_t pack_h2(float a, float b) {
  if constexpr (BF16) return pack_bf16x2(a, b);
  else return uint32_t(f32_to_f16(a)) | (uint32_t(f32_to_f16(b)) << 16);
}

// One 256-row query block of head h against keys [0, kend).  Real rows row0 + i;
// the caller's span owns virtual rows [vlo, vhi) of the virtual block starting at
// vrow0 (the zig-zag order maps virtual block -> real block).  With PAD the
// operands' rows hold P.hd < HD elements (a multiple of 8) and the block computes
// as if each row were zero-padded to HD: Q's missing chunks are zeros in
// registers, the LDS slots of K and V chunks past P.hd are zeroed once per sweep
// by the lanes that own them (which skip those transfers), and O's columns past
// P.hd are not stored.
template <int HD, bool BF16, bool PAD>
VM_DEV void attn_block_mfma(Args A, uint32_t ti, uint32_t h, uint32_t row0, uint32_t vrow0, uint32_t vlo,
                            uint32_t vhi) {
  const VM_K Task& t = task_of(A, ti);
  const AttnDesc P = attn_desc(A, t);
  h = uni(h);
  row0 = uni(row0);
  vrow0 = uni(vrow0);
  vlo = uni(vlo);
  vhi = uni(vhi);
  typedef AttnLds<HD> L;
  const uint32_t T = P.T, C = P.C, dt = (t.tile_op >> 8) & 0xFF;
  const uint32_t hd = PAD ? uni(P.hd) : uint32_t(HD);     // elements per stored row
  constexpr int KS = HD / 16;            // MFMA steps over hd for S
  constexpr int DB = HD / 32;            // 32-row d blocks of O^T
  const uint32_t lane = threadIdx.x & 63, wave = uni(threadIdx.x >> 6), g = lane >> 5;
  const uint32_t qw0 = row0 + 64 * wave;                    // this wave's first row
  const VM_G uint16_t* Q = gcast<uint16_t>(resolve(A, t.a)) + uint64_t(h) * T * hd;
  const VM_G uint16_t* K = gcast<uint16_t>(resolve(A, t.b)) + uint64_t(h) * C * hd;
  const VM_G uint16_t* V = gcast<uint16_t>(resolve(A, t.p[0])) + uint64_t(h) * C * hd;
  gbyte* Ob = resolve(A, t.dst);

  // Q^T fragments (B operand) of both sub-tiles: column = query, 8 consecutive hd
  // values; rows past T re-read row T - 1 (results not stored)
  u16x8 qf[2][KS];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const uint32_t qr = min(qw0 + 32 * u + (lane & 31), T - 1);
#pragma unroll
    for (int s = 0; s < KS; ++s)
      qf[u][s] = (!PAD || 16 * s + 8 * g < hd) ? *(const VM_G u16x8*)(Q + uint64_t(qr) * hd + s * 16 + 8 * g)
                                                : u16x8{};
  }
  f32x16 o[2][DB];
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int i = 0; i < DB; ++i) o[u][i] = f32x16{};
  float m_run[2] = {-INFINITY, -INFINITY}, l_part[2] = {0.0f, 0.0f};
  const float sl2 = P.scale * 1.4426950408889634f;

  // keys this block needs: up to the last query's causal limit
  const int32_t shift = int32_t(C) - int32_t(T);
  const uint32_t qmax = min(row0 + kAttnRows, T) - 1;
  uint32_t kend = C;
  if (P.causal) kend = min(C, uint32_t(max(0, int32_t(qmax) + shift + 1)));
  const uint32_t nblk = (kend + kAttnKeys - 1) / kAttnKeys;
  // this wave: rows [qw0, qw0 + 64) (those below T); last visible key of its first
  // and last row
  const bool wave_rows = qw0 < T;
  const int32_t wq_lo = int32_t(qw0) + shift;
  const int32_t wq_hi = int32_t(min(qw0 + 63, T - 1)) + shift;

  // Staging: per block, kRounds transfers per operand and thread.  Round j of
  // wave w, lane l fills stage bytes 4096 j + 1024 w + 16 l of the operand: key
  // row r = (4096 j + 1024 w + 16 l) / kRow, slot (16 l % kRow) / 16, so the lane
  // fetches chunk slot ^ swz(r) of key min(kb 64 + r, C - 1).  Keys past C are
  // masked out of S; their V rows are zeroed by the lane that fetched them, once
  // its own transfers have landed, so 0-weight keys add 0.
  const uint32_t lds0 = uni(uint32_t(reinterpret_cast<uintptr_t>(lds_ptr<lds_u8>())));
  const lds_u8* LB = (const lds_u8*)uintptr_t(lds0);
  const uint32_t st0 = lds0, st1 = lds0 + L::kStage;
  const uint32_t wo = uni(1024 * wave);
  const uint32_t dr = (1024 * wave + 16 * lane) / L::kRow;            // row within a round
  const uint32_t dslot = (16 * lane) % L::kRow / 16;
  const uint32_t dk = (dslot ^ kswz<HD>(dr)) * 16, dv = (dslot ^ vswz<HD>(dr)) * 16;
  constexpr uint32_t kRowsPerRound = 4096 / L::kRow;
  const uint32_t grow = 2 * hd;                                      // global bytes per key row
  // the swizzles repeat every kRowsPerRound rows, so a lane fetches the same
  // chunk in every round: with PAD it lies inside the row always or never
  const bool kon = !PAD || dk < grow, von = !PAD || dv < grow;
  const gbyte* Kg = (const gbyte*)K;
  const gbyte* Vg = (const gbyte*)V;
  auto dma_block = [&](uint32_t st, uint32_t kb) {
#pragma unroll
    for (uint32_t j = 0; j < L::kRounds; ++j) {
      const uint32_t key = min(kb * kAttnKeys + j * kRowsPerRound + dr, C - 1);
      if (kon) dma16(Kg, key * grow + dk, st + 4096 * j + wo);
    }
#pragma unroll
    for (uint32_t j = 0; j < L::kRounds; ++j) {
      const uint32_t key = min(kb * kAttnKeys + j * kRowsPerRound + dr, C - 1);
      if (von) dma16(Vg, key * grow + dv, st + L::kKBytes + 4096 * j + wo);
    }
  };
  // PAD: zeros in the K and V slots of both stages that no transfer fills
  auto zero_pad = [&]() {
    if constexpr (PAD) {
#pragma unroll
      for (uint32_t j = 0; j < L::kRounds; ++j)
#pragma unroll
        for (uint32_t sg = 0; sg < 2; ++sg) {
          const uint32_t off = sg * L::kStage + 4096 * j + wo + 16 * lane;
          if (!kon) *(__attribute__((address_space(3))) v4u*)(LB + off) = v4u_make(0, 0, 0, 0);
          if (!von) *(__attribute__((address_space(3))) v4u*)(LB + off + L::kKBytes) = v4u_make(0, 0, 0, 0);
        }
    }
  };
  auto zero_tail = [&](uint32_t st, uint32_t kb) {
    if (kb * kAttnKeys + kAttnKeys > C) {
#pragma unroll
      for (uint32_t j = 0; j < L::kRounds; ++j)
        if (kb * kAttnKeys + j * kRowsPerRound + dr >= C)
          *(__attribute__((address_space(3))) v4u*)(LB + (st - lds0) + L::kKBytes + 4096 * j + wo + 16 * lane) =
              v4u_make(0, 0, 0, 0);
    }
  };
  // V^T fragment addresses (block db, second read at +4 rows): key row 16 ks +
  // 8 (gq >> 1) + e, hd chunk 4 db + 2 (gq & 1) + (q >> 1), half q & 1, where
  // gq = lane >> 4, e = (lane >> 2) & 3, q = lane & 3.
  uint32_t vfa[DB];
  {
    const uint32_t gq = lane >> 4, e = (lane >> 2) & 3, q = lane & 3;
    const uint32_t row = 8 * (gq >> 1) + e, sw = vswz<HD>(row);
#pragma unroll
    for (int db = 0; db < DB; ++db)
      vfa[db] = L::kKBytes + row * L::kRow + (((4 * uint32_t(db) + 2 * (gq & 1) + (q >> 1)) ^ sw) * 16) + (q & 1) * 8;
  }

  const uint32_t krow = kperm(lane & 31), ksw = kswz<HD>(krow);
  const int32_t qlim0 = int32_t(qw0 + (lane & 31)) + shift;   // last visible key, sub-tile 0
  // probabilities of a pass are exp2(scale' s - m_ref) with m_ref fixed per row; a
  // row sum partial above this bound flags the block for the exact pass (P must
  // stay finite in bf16 / f16)
  const float bound = BF16 ? 16777216.0f : 16384.0f;
  bool redo = false;

  // masked entries (keys past the row's causal limit or past C) -> -inf
  auto mask_s = [&](f32x16 (&s)[2], int u, uint32_t key0) {
    const int32_t lim = (P.causal ? min(qlim0 + 32 * u, int32_t(C) - 1) : int32_t(C) - 1) - int32_t(key0);
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int32_t kr = 32 * kh + 16 * (v >> 3) + 8 * int32_t(g) + (v & 7);
        if (kr > lim) s[kh][v] = -INFINITY;
      }
  };
  // scaled row maximum of a block, the same in both lanes of a row
  auto row_max = [&](const f32x16 (&s)[2]) -> float {
    float mx = -INFINITY;
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s[kh][v]);
    return fmaxf(mx, xor32(mx)) * sl2;
  };
  // P^T fragments (bf16/f16) and the row-sum partial of sub-tile u.  With MAXC (a
  // sweep's first block and the masked blocks) a row whose reference is still
  // unset (no visible key so far, so its O and l are 0) takes this block's
  // maximum; every other block of an unmasked run sees keys for all rows after
  // the first, so its rows all have a reference.
  auto probs = [&](auto maxc, const f32x16 (&s)[2], int u, u16x8 (&pf)[4]) {
    if constexpr (decltype(maxc)::value) {
      const float mx = row_max(s);
      m_run[u] = m_run[u] == -INFINITY ? mx : m_run[u];
    }
    const float mu = m_run[u] == -INFINITY ? 0.0f : m_run[u];
    float rs = 0.0f;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      float e[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) e[i] = __builtin_amdgcn_exp2f(fmaf(s[ks >> 1][8 * (ks & 1) + i], sl2, -mu));
      v4u w = v4u_make(pack_h2<BF16>(e[0], e[1]), pack_h2<BF16>(e[2], e[3]), pack_h2<BF16>(e[4], e[5]),
                       pack_h2<BF16>(e[6], e[7]));
      pf[ks] = __builtin_bit_cast(u16x8, w);
      // the row sum adds the rounded probabilities (the ones the MFMA multiplies),
      // two per dot instruction
      rs = dot2_ones<BF16>(w.x, rs);
      rs = dot2_ones<BF16>(w.y, rs);
      rs = dot2_ones<BF16>(w.z, rs);
      rs = dot2_ones<BF16>(w.w, rs);
    }
    redo = redo || !(rs <= bound);      // also catches inf (NaN rows propagate as in the reference)
    l_part[u] += rs;
  };
  auto s_tiles = [&](const lds_u8* S, f32x16 (&s0)[2], f32x16 (&s1)[2]) {
    // the two 32-key halves are independent accumulation chains: alternate them
    // so consecutive MFMAs never wait on each other's result
    u16x8 kf[2][KS];
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int st = 0; st < KS; ++st)
        kf[kh][st] = *(const lds_u16x8*)(S + (kh * 32 + krow) * L::kRow + (((2 * uint32_t(st) + g) ^ ksw) * 16));
    s0[0] = s0[1] = s1[0] = s1[1] = f32x16{};
#pragma unroll
    for (int st = 0; st < KS; ++st)
#pragma unroll
      for (int kh = 0; kh < 2; ++kh) s0[kh] = mfma16<BF16>(kf[kh][st], qf[0][st], s0[kh]);
#pragma unroll
    for (int st = 0; st < KS; ++st)
#pragma unroll
      for (int kh = 0; kh < 2; ++kh) s1[kh] = mfma16<BF16>(kf[kh][st], qf[1][st], s1[kh]);
  };
  // One 64-key block: S^T of both sub-tiles (K fragments read once, used twice),
  // sub-tile 0's softmax while sub-tile 1's S^T is on the matrix cores, then
  // P^T . V of sub-tile 0 while sub-tile 1's softmax runs (V^T fragments read
  // once, used twice).
  auto body = [&](auto maskc, auto maxc, const lds_u8* S, uint32_t key0) {
    f32x16 s0[2], s1[2];
    s_tiles(S, s0, s1);
    u16x8 p0[4], p1[4];
    if constexpr (decltype(maskc)::value) mask_s(s0, 0, key0);
    probs(maxc, s0, 0, p0);
    if constexpr (decltype(maskc)::value) mask_s(s1, 1, key0);
    u16x8 vf[DB][4];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(S + vfa[db] + ks * 16 * L::kRow));
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(S + vfa[db] + (ks * 16 + 4) * L::kRow));
        vf[db][ks] = __builtin_bit_cast(u16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int db = 0; db < DB; ++db) o[0][db] = mfma16<BF16>(vf[db][ks], p0[ks], o[0][db]);
    probs(maxc, s1, 1, p1);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int db = 0; db < DB; ++db) o[1][db] = mfma16<BF16>(vf[db][ks], p1[ks], o[1][db]);
  };
  // Exact pass 1: the true scaled row maxima over all visible keys.
  auto max_body = [&](auto maskc, auto, const lds_u8* S, uint32_t key0) {
    f32x16 s0[2], s1[2];
    s_tiles(S, s0, s1);
    if constexpr (decltype(maskc)::value) {
      mask_s(s0, 0, key0);
      mask_s(s1, 1, key0);
    }
    m_run[0] = fmaxf(m_run[0], row_max(s0));
    m_run[1] = fmaxf(m_run[1], row_max(s1));
  };

  // One sweep over the key blocks: per block, start the next block's transfers
  // into the other LDS stage (its last reader passed the previous barrier),
  // compute on this one, wait for this lane's transfers, then the block barrier
  // publishes the next stage.  Blocks wholly
  // below this wave's diagonal (and inside the keys) run unmasked; the rest are
  // masked, and those past the wave's last row's causal limit are skipped.  The
  // two kinds run in two loops (not one loop with a branch) so the body is laid
  // out once per loop.
  uint32_t nfull = wave_rows ? min(nblk, C / kAttnKeys) : 0u;
  if (P.causal) nfull = min(nfull, wq_lo >= kAttnKeys - 1 ? uint32_t(wq_lo - (kAttnKeys - 1)) / kAttnKeys + 1 : 0u);
  auto sweep = [&](auto fn) {
    __syncthreads();                    // LDS free from the previous user
    zero_pad();
    if (nblk) dma_block(st0, 0);
    // every global load so far (the Q fragments too) has landed: said explicitly
    // so the compiler's wait counting does not carry the Q loads into the loop
    wait_vm0();
    if (nblk) zero_tail(st0, 0);
    __syncthreads();
    auto step = [&](auto maskc, auto maxc, uint32_t kb) {
      const uint32_t cur = (kb & 1) ? st1 : st0, nxt = (kb & 1) ? st0 : st1;
      if (kb + 1 < nblk) dma_block(nxt, kb + 1);
      const uint32_t key0 = kb * kAttnKeys;
      const lds_u8* S = LB + (cur - lds0);
      if constexpr (decltype(maskc)::value) {
        if (wave_rows && (!P.causal || int32_t(key0) <= wq_hi)) fn(maskc, maxc, S, key0);
      } else {
        fn(maskc, maxc, S, key0);
      }
      wait_vm0();
      if (kb + 1 < nblk) zero_tail(nxt, kb + 1);
      __syncthreads();
    };
    uint32_t kb = 0;
    if (nfull) step(std::false_type{}, std::true_type{}, kb++);
    for (; kb < nfull; ++kb) step(std::false_type{}, std::false_type{}, kb);
    for (; kb < nblk; ++kb) step(std::true_type{}, std::true_type{}, kb);
  };
  sweep(body);
  if (__syncthreads_or(redo)) {
    // some row's scores rose too far above its first block's maximum: redo the
    // block with exact maxima (pass 1), then probabilities <= 1 (pass 2)
    m_run[0] = m_run[1] = -INFINITY;
    sweep(max_body);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      l_part[u] = 0.0f;
#pragma unroll
      for (int i = 0; i < DB; ++i) o[u][i] = f32x16{};
    }
    sweep(body);
  }
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const uint32_t ql = 64 * wave + 32 * u + (lane & 31);   // 0..255 within the block
    const uint32_t q = row0 + ql;
    const float l = l_part[u] + xor32(l_part[u]);
    if (q < T && vrow0 + ql >= vlo && vrow0 + ql < vhi) {
      // a row with no visible key (causal, T > C) has l = 0 and O = 0 and stores NaN,
      // as the reference's kernel does (attention.cl:155) and softmax of a -inf row
      const float inv = 1.0f / l;
      const uint64_t obase = (uint64_t(h) * T + q) * hd;
#pragma unroll
      for (int db = 0; db < DB; ++db) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t d = db * 32 + 8 * j + 4 * g;
          if (!PAD || d < hd)
            st4(Ob, dt, obase + d,
              v4f_make(o[u][db][4 * j] * inv, o[u][db][4 * j + 1] * inv, o[u][db][4 * j + 2] * inv,
                       o[u][db][4 * j + 3] * inv));
        }
      }
    }
  }
}

// Generic path: any head size, dtype or view.  One wave per query row; lanes split
// the keys of a 64-key chunk, then the hd outputs.
VM_DEV void attn_rows_generic(Args A, uint32_t ti, uint32_t lo, uint32_t hi) {
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
  // tile = head * Tp + row, each head's rows padded to whole 256-row blocks
  const uint32_t Tp = (T + kAttnRows - 1) / kAttnRows * kAttnRows;
  hi = min(hi, H * Tp);
  constexpr int kMaxD = 4;               // hd <= 256
  for (uint32_t tile = lo + wave; tile < hi; tile += kWaves) {
    const uint32_t h = tile / Tp, m = tile % Tp;
    if (m >= T) continue;                // padding past the head's rows
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
    // a row with no visible key (causal, T > C) has l = 0 and O = 0 and stores NaN,
    // as the reference's kernel does (attention.cl:155) and softmax of a -inf row
    const float inv = 1.0f / lrun;
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

// The lane's query blocks: per head, the virtual 256-row blocks intersecting
// [lo, hi), each mapped to its real block (zig-zag when causal, so that chunks of
// equally many blocks cost about the same).  A head's tiles are its rows padded
// to whole blocks (Tp rows): the scheduler cuts chunks on block boundaries, so no
// block is split between lanes, and the rows of the last real block past T are
// computed and not stored.
template <int HD, bool BF16, bool PAD>
VM_DEV void attn_fast(Args A, uint32_t ti, uint32_t lo, uint32_t hi) {
  A = uargs(A);
  const VM_K Task& t = task_of(A, ti);
  const AttnDesc P = attn_desc(A, t);
  const uint32_t T = P.T;
  const uint32_t nb = (T + kAttnRows - 1) / kAttnRows, Tp = nb * kAttnRows;
  hi = min(hi, P.H * Tp);
  const bool zig = P.causal;
  for (uint32_t h = lo / Tp; h * Tp < hi; ++h) {
    const uint32_t a = max(lo, h * Tp) - h * Tp, b = min(hi - h * Tp, Tp);     // virtual rows [a, b)
    for (uint32_t vb = a / kAttnRows; vb * kAttnRows < b; ++vb) {
      const uint32_t rb = zig ? ((vb & 1) ? nb - 1 - (vb >> 1) : (vb >> 1)) : vb;
      const uint32_t vrow0 = vb * kAttnRows;
      attn_block_mfma<HD, BF16, PAD>(A, ti, h, rb * kAttnRows, vrow0, max(a, vrow0), min(b, vrow0 + kAttnRows));
    }
  }
}

// ---- f32 operands -------------------------------------------------------------------
// Matrix-core path for f32 Q/K/V (hd a multiple of 4 up to 128, run as 64 or 128 on
// zero-padded rows; scale > 0; K read through the usual [H,hd,C] transpose view of
// a [H,C,hd] buffer): v_mfma_f32_32x32x2f32, so products and sums stay f32.  A lane
// takes 128 query rows at a time, 32 per wave (one 32x32 S^T tile per 32-key block),
// and streams K and V in 32-key blocks through registers into two LDS buffers whose
// rows are padded to HD + 2 floats: the 32 keys a half wave reads for S^T, and the
// 32 channels it reads for V^T, then lie in distinct banks.
//   S^T (32 keys x 32 queries) = sum over hd of K Q^T.  MFMA step 2c + e takes hd
//   4c + 2g + e in lane group g = lane / 32, so a lane reads one 8-byte pair of its
//   key row per two steps (two accumulation chains, c even / odd, added at the end).
//   O^T (HD x 32 queries) += V^T P^T.  Step s takes key 8 (s / 4) + 4 g + s % 4 in
//   lane group g, the key that register s of the S^T accumulator holds, so P^T is
//   the S^T registers themselves.
// Online softmax in base 2 with the usual per-block rescale of O and l.  Keys past C
// are masked; their V rows are staged as zeros, so 0-weight keys add 0.

// One 128-row query block of head h (real rows row0 .., virtual rows vrow0 .., the
// caller's span owns virtual rows [vlo, vhi)) against keys [0, kend).
template <int HD>
VM_DEV void attn_block_f32(Args A, uint32_t ti, uint32_t h, uint32_t row0, uint32_t vrow0, uint32_t vlo,
                           uint32_t vhi) {
  const VM_K Task& t = task_of(A, ti);
  const AttnDesc P = attn_desc(A, t);
  h = uni(h);
  row0 = uni(row0);
  vrow0 = uni(vrow0);
  vlo = uni(vlo);
  vhi = uni(vhi);
  typedef AttnF32Lds<HD> L;
  typedef __attribute__((address_space(3))) float lds_f;
  typedef __attribute__((address_space(3))) f32x2_t lds_f2;
  constexpr uint32_t NC = HD / 4;                              // 4-float chunks per row
  constexpr int DB = HD / 32;                                  // 32-channel blocks of O^T
  constexpr uint32_t NR = kAttnF32Keys * NC / kBlock;         // staged chunks per thread and operand
  static_assert(NR * kBlock == kAttnF32Keys * NC, "whole staging rounds");
  const uint32_t T = P.T, C = P.C, hd = uni(P.hd), dt = (t.tile_op >> 8) & 0xFF;
  const uint32_t hc = hd / 4;                                  // chunks inside the row
  const uint32_t lane = threadIdx.x & 63, wave = uni(threadIdx.x >> 6), g = lane >> 5, j = lane & 31;
  const uint32_t qw0 = row0 + 32 * wave;                       // this wave's first row
  const VM_G float* Q = gcast<float>(resolve(A, t.a)) + uint64_t(h) * T * hd;
  const VM_G float* K = gcast<float>(resolve(A, t.b)) + uint64_t(h) * C * hd;
  const VM_G float* V = gcast<float>(resolve(A, t.p[0])) + uint64_t(h) * C * hd;
  gbyte* Ob = resolve(A, t.dst);

  // Q^T fragments: step 2c + e <- Q[q][4c + 2g + e]; rows past T re-read row T - 1
  // (not stored); chunks past hd are zero (4c < hd is uniform: hd % 4 == 0)
  float qf[2 * NC];
  {
    const uint32_t qr = min(qw0 + j, T - 1);
#pragma unroll
    for (uint32_t c = 0; c < NC; ++c) {
      f32x2_t x = {0.0f, 0.0f};
      if (4 * c < hd) x = *(const VM_G f32x2_t*)(Q + uint64_t(qr) * hd + 4 * c + 2 * g);
      qf[2 * c] = x.x;
      qf[2 * c + 1] = x.y;
    }
  }
  f32x16 o[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i) o[i] = f32x16{};
  float m_run = -INFINITY, l_part = 0.0f;
  const float sl2 = P.scale * 1.4426950408889634f;

  // keys this block needs: up to its last row's causal limit
  const int32_t shift = int32_t(C) - int32_t(T);
  const uint32_t qmax = min(row0 + kAttnF32Rows, T) - 1;
  uint32_t kend = C;
  if (P.causal) kend = min(C, uint32_t(max(0, int32_t(qmax) + shift + 1)));
  const uint32_t nblk = (kend + kAttnF32Keys - 1) / kAttnF32Keys;
  const bool wave_rows = qw0 < T;
  const int32_t wq_hi = int32_t(min(qw0 + 31, T - 1)) + shift;   // last visible key of the wave's last row
  const int32_t qlim = int32_t(qw0 + j) + shift;                  // this lane's row's last visible key

  // Staging: chunk f = r kBlock + threadIdx.x of a block is key f / NC, chunk f % NC.
  // Keys past C re-read key C - 1 and chunks past hd re-read the row's last chunk
  // (no load behind a lane-dependent branch); both are replaced by zeros in the
  // LDS copy where they would matter (V rows past C, chunks past hd).
  const uint32_t lds0 = uni(uint32_t(reinterpret_cast<uintptr_t>(lds_ptr<lds_u8>())));
  v4f ks[NR], vs[NR];
  auto load = [&](uint32_t kb) {
#pragma unroll
    for (uint32_t r = 0; r < NR; ++r) {
      const uint32_t f = r * kBlock + threadIdx.x, key = f / NC, c = min(f % NC, hc - 1);
      const uint64_t e = uint64_t(min(kb * kAttnF32Keys + key, C - 1)) * hd + 4 * c;
      ks[r] = *(const VM_G v4f*)(K + e);
      vs[r] = *(const VM_G v4f*)(V + e);
    }
  };
  auto store = [&](uint32_t buf, uint32_t kb) {
#pragma unroll
    for (uint32_t r = 0; r < NR; ++r) {
      const uint32_t f = r * kBlock + threadIdx.x, key = f / NC, c = f % NC;
      const bool in = c < hc;
      const v4f z = v4f{0.0f, 0.0f, 0.0f, 0.0f};
      const v4f kx = in ? ks[r] : z;
      const v4f vx = in && kb * kAttnF32Keys + key < C ? vs[r] : z;
      lds_f* kd = (lds_f*)uintptr_t(lds0 + 4 * (buf * L::kBuf + key * L::kRS + 4 * c));
      *(lds_f2*)kd = f32x2_t{kx.x, kx.y};
      *(lds_f2*)(kd + 2) = f32x2_t{kx.z, kx.w};
      *(lds_f2*)(kd + L::kOp) = f32x2_t{vx.x, vx.y};
      *(lds_f2*)(kd + L::kOp + 2) = f32x2_t{vx.z, vx.w};
    }
  };

  auto body = [&](uint32_t buf, uint32_t key0) {
    const lds_f* Kr = (const lds_f*)uintptr_t(lds0 + 4 * (buf * L::kBuf + j * L::kRS + 2 * g));
    const lds_f* Vb = (const lds_f*)uintptr_t(lds0 + 4 * (buf * L::kBuf + L::kOp + j));
    f32x16 s0 = f32x16{}, s1 = f32x16{};
#pragma unroll
    for (uint32_t c = 0; c < NC; c += 2) {
      const f32x2_t k0 = *(const lds_f2*)(Kr + 4 * c);
      const f32x2_t k1 = *(const lds_f2*)(Kr + 4 * c + 4);
      s0 = __builtin_amdgcn_mfma_f32_32x32x2f32(k0.x, qf[2 * c], s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_32x32x2f32(k1.x, qf[2 * c + 2], s1, 0, 0, 0);
      s0 = __builtin_amdgcn_mfma_f32_32x32x2f32(k0.y, qf[2 * c + 1], s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_32x32x2f32(k1.y, qf[2 * c + 3], s1, 0, 0, 0);
    }
    f32x16 s = s0 + s1;
    // masked entries (keys past the row's causal limit or past C) -> -inf
    const int32_t lim = (P.causal ? min(qlim, int32_t(C) - 1) : int32_t(C) - 1) - int32_t(key0);
#pragma unroll
    for (int v = 0; v < 16; ++v)
      if (int32_t(8 * (v >> 2) + 4 * g + (v & 3)) > lim) s[v] = -INFINITY;
    float mx = -INFINITY;
#pragma unroll
    for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s[v]);
    mx = fmaxf(mx, xor32(mx));
    const float m_new = fmaxf(m_run, mx * sl2);
    const float mu = m_new == -INFINITY ? 0.0f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - mu);     // 0 while nothing is accumulated
    m_run = m_new;
    float rs = 0.0f;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      s[v] = __builtin_amdgcn_exp2f(fmaf(s[v], sl2, -mu));
      rs += s[v];
    }
    l_part = fmaf(l_part, alpha, rs);
#pragma unroll
    for (int i = 0; i < DB; ++i) o[i] *= alpha;
#pragma unroll
    for (int st = 0; st < 16; ++st) {
      const uint32_t key = 8 * (st >> 2) + 4 * g + (st & 3);
#pragma unroll
      for (int i = 0; i < DB; ++i)
        o[i] = __builtin_amdgcn_mfma_f32_32x32x2f32(Vb[key * L::kRS + 32 * i], s[st], o[i], 0, 0, 0);
    }
  };

  // Per block: the next block's loads go out, this block is computed, then the
  // next block is written to the other buffer (its last reader passed the
  // previous barrier) and a barrier publishes it.  Blocks past the wave's last
  // row's causal limit are skipped (the wave still stages and syncs).
  __syncthreads();                      // LDS free from the previous user
  if (nblk) {
    load(0);
    store(0, 0);
  }
  __syncthreads();
  for (uint32_t kb = 0; kb < nblk; ++kb) {
    if (kb + 1 < nblk) load(kb + 1);
    if (wave_rows && (!P.causal || int32_t(kb * kAttnF32Keys) <= wq_hi)) body(kb & 1, kb * kAttnF32Keys);
    if (kb + 1 < nblk) store((kb + 1) & 1, kb + 1);
    __syncthreads();
  }

  const float l = l_part + xor32(l_part);
  const uint32_t q = qw0 + j, vq = vrow0 + 32 * wave + j;
  if (q < T && vq >= vlo && vq < vhi) {
    // a row with no visible key (causal, T > C) has l = 0 and O = 0 and stores NaN,
    // as the reference's kernel does (attention.cl:155) and softmax of a -inf row
    const float inv = 1.0f / l;
    const uint64_t obase = (uint64_t(h) * T + q) * hd;
#pragma unroll
    for (int i = 0; i < DB; ++i)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const uint32_t d = 32 * i + 8 * jj + 4 * g;
        if (d < hd)
          st4(Ob, dt, obase + d,
              v4f_make(o[i][4 * jj] * inv, o[i][4 * jj + 1] * inv, o[i][4 * jj + 2] * inv, o[i][4 * jj + 3] * inv));
      }
  }
}

// The lane's query blocks in the order attn_fast takes them (virtual 256-row
// blocks, zig-zag when causal), each as two 128-row halves: blk(h, real first
// row, virtual first row, virtual rows [vlo, vhi) the span owns).
template <class Blk>
VM_DEV void attn_lane128(Args A, uint32_t ti, uint32_t lo, uint32_t hi, Blk blk) {
  const VM_K Task& t = task_of(A, ti);
  const AttnDesc P = attn_desc(A, t);
  const uint32_t T = P.T;
  const uint32_t nb = (T + kAttnRows - 1) / kAttnRows, Tp = nb * kAttnRows;
  hi = min(hi, P.H * Tp);
  const bool zig = P.causal;
  for (uint32_t h = lo / Tp; h * Tp < hi; ++h) {
    const uint32_t a = max(lo, h * Tp) - h * Tp, b = min(hi - h * Tp, Tp);     // virtual rows [a, b)
    for (uint32_t vb = a / kAttnRows; vb * kAttnRows < b; ++vb) {
      const uint32_t rb = zig ? ((vb & 1) ? nb - 1 - (vb >> 1) : (vb >> 1)) : vb;
      const uint32_t vrow0 = vb * kAttnRows;
      for (uint32_t hf = 0; hf < 2; ++hf) {
        const uint32_t r0 = rb * kAttnRows + hf * kAttnF32Rows;
        if (r0 < T) blk(h, r0, vrow0 + hf * kAttnF32Rows, max(a, vrow0), min(b, vrow0 + kAttnRows));
      }
    }
  }
}

VM_DEV void attn_f32_run(Args A, uint32_t ti, uint32_t lo, uint32_t hi) {
  A = uargs(A);
  const AttnDesc P = attn_desc(A, task_of(A, ti));
  if (P.hd > 64)
    attn_lane128(A, ti, lo, hi, [&](uint32_t h, uint32_t r0, uint32_t v0, uint32_t vl, uint32_t vh) {
      attn_block_f32<128>(A, ti, h, r0, v0, vl, vh);
    });
  else
    attn_lane128(A, ti, lo, hi, [&](uint32_t h, uint32_t r0, uint32_t v0, uint32_t vl, uint32_t vh) {
      attn_block_f32<64>(A, ti, h, r0, v0, vl, vh);
    });
}

// ---- wide 16-bit rows (hd up to 256) ---------------------------------------------------
// bf16 / f16 Q/K/V with hd a multiple of 8 in (128, 256], run as 256 on zero-padded
// rows (scale > 0, K through the usual transpose view): the f32 path's structure
// (128 query rows per lane, 32 per wave, 32-key blocks staged through registers
// into two LDS buffers) with v_mfma_f32_32x32x16_{bf16,f16}.
//   S^T (32 keys x 32 queries): MFMA step s takes hd [16 s + 8 g, +8) in lane
//   group g, one 16-byte read of the lane's key row (rows padded to 528 bytes, so
//   the 16 lanes of a read pass hit distinct banks).
//   O^T (256 x 32 queries) += V^T P^T in two 16-key steps: element i of lane group
//   g in step ps is S^T register 8 ps + i, key 16 ps + 8 (i / 4) + 4 g + i % 4, so
//   P^T is the packed S^T registers.  The matching V^T operand is two
//   ds_read_b64_tr_b16 (in each group of 16 lanes, lane 4e + q points at key row
//   k0 + e, channels d0 + 4q .. +3, and receives channel d0 + lane % 16 at rows
//   k0 .. k0 + 3), at rows 16 ps + 4 g and 16 ps + 8 + 4 g; V rows padded to 576
//   bytes, so a 32-lane pass covers the 64 banks once.
// Online softmax in base 2 with the per-block rescale of O and l; the row sum adds
// the rounded probabilities (the ones the MFMA multiplies).
template <bool BF16>
VM_DEV void attn_block_h16w(Args A, uint32_t ti, uint32_t h, uint32_t row0, uint32_t vrow0, uint32_t vlo,
                            uint32_t vhi) {
  const VM_K Task& t = task_of(A, ti);
  const AttnDesc P = attn_desc(A, t);
  h = uni(h);
  row0 = uni(row0);
  vrow0 = uni(vrow0);
  vlo = uni(vlo);
  vhi = uni(vhi);
  constexpr int HD = 256;
  constexpr uint32_t NC = HD / 8;                              // 16-byte chunks per row
  constexpr int KS = HD / 16;                                  // MFMA steps of S^T
  constexpr int DB = HD / 32;                                  // 32-channel blocks of O^T
  constexpr uint32_t NR = kAttnF32Keys * NC / kBlock;         // staged chunks per thread and operand
  static_assert(NR * kBlock == kAttnF32Keys * NC, "whole staging rounds");
  const uint32_t T = P.T, C = P.C, hd = uni(P.hd), dt = (t.tile_op >> 8) & 0xFF;
  const uint32_t hc = hd / 8;                                  // chunks inside the row
  const uint32_t lane = threadIdx.x & 63, wave = uni(threadIdx.x >> 6), g = lane >> 5, j = lane & 31;
  const uint32_t qw0 = row0 + 32 * wave;
  const VM_G uint16_t* Q = gcast<uint16_t>(resolve(A, t.a)) + uint64_t(h) * T * hd;
  const VM_G uint16_t* K = gcast<uint16_t>(resolve(A, t.b)) + uint64_t(h) * C * hd;
  const VM_G uint16_t* V = gcast<uint16_t>(resolve(A, t.p[0])) + uint64_t(h) * C * hd;
  gbyte* Ob = resolve(A, t.dst);

  // Q^T fragments: step s <- Q[q][16 s + 8 g, +8); rows past T re-read row T - 1
  // (not stored); chunks past hd re-read the row's last chunk and are zeroed
  u16x8 qf[KS];
  {
    const uint32_t qr = min(qw0 + j, T - 1);
#pragma unroll
    for (int st = 0; st < KS; ++st) {
      const uint32_t c = 2 * st + g;
      const u16x8 x = *(const VM_G u16x8*)(Q + uint64_t(qr) * hd + 8 * min(c, hc - 1));
      qf[st] = c < hc ? x : u16x8{};
    }
  }
  f32x16 o[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i) o[i] = f32x16{};
  float m_run = -INFINITY, l_part = 0.0f;
  const float sl2 = P.scale * 1.4426950408889634f;

  const int32_t shift = int32_t(C) - int32_t(T);
  const uint32_t qmax = min(row0 + kAttnF32Rows, T) - 1;
  uint32_t kend = C;
  if (P.causal) kend = min(C, uint32_t(max(0, int32_t(qmax) + shift + 1)));
  const uint32_t nblk = (kend + kAttnF32Keys - 1) / kAttnF32Keys;
  const bool wave_rows = qw0 < T;
  const int32_t wq_hi = int32_t(min(qw0 + 31, T - 1)) + shift;
  const int32_t qlim = int32_t(qw0 + j) + shift;

  // Staging as in the f32 path: chunk f = r kBlock + threadIdx.x of a block is key
  // f / NC, chunk f % NC; keys past C re-read key C - 1 (their V rows are staged as
  // zeros), chunks past hd re-read the last chunk (staged as zeros).
  const uint32_t lds0 = uni(uint32_t(reinterpret_cast<uintptr_t>(lds_ptr<lds_u8>())));
  typedef __attribute__((address_space(3))) v4u lds_v4u;
  v4u ks[NR], vs[NR];
  auto load = [&](uint32_t kb) {
#pragma unroll
    for (uint32_t r = 0; r < NR; ++r) {
      const uint32_t f = r * kBlock + threadIdx.x, key = f / NC, c = min(f % NC, hc - 1);
      const uint64_t e = uint64_t(min(kb * kAttnF32Keys + key, C - 1)) * hd + 8 * c;
      ks[r] = *(const VM_G v4u*)(K + e);
      vs[r] = *(const VM_G v4u*)(V + e);
    }
  };
  auto store = [&](uint32_t buf, uint32_t kb) {
    const uint32_t kbase = lds0 + buf * kAttnWBuf, vbase = kbase + kAttnF32Keys * kAttnWKRow;
#pragma unroll
    for (uint32_t r = 0; r < NR; ++r) {
      const uint32_t f = r * kBlock + threadIdx.x, key = f / NC, c = f % NC;
      const bool in = c < hc;
      const v4u z = v4u_make(0, 0, 0, 0);
      *(lds_v4u*)uintptr_t(kbase + key * kAttnWKRow + 16 * c) = in ? ks[r] : z;
      *(lds_v4u*)uintptr_t(vbase + key * kAttnWVRow + 16 * c) = in && kb * kAttnF32Keys + key < C ? vs[r] : z;
    }
  };
  // V^T read addresses (block db, step ps, first read; the second is 8 rows on)
  const uint32_t e4 = (lane >> 2) & 3, q4 = lane & 3, hcol = (lane >> 4) & 1;
  const uint32_t vcol = 2 * (16 * hcol + 4 * q4);             // bytes within a 32-channel block

  auto body = [&](uint32_t buf, uint32_t key0) {
    const uint32_t kbase = lds0 + buf * kAttnWBuf, vbase = kbase + kAttnF32Keys * kAttnWKRow;
    const uint32_t kr = kbase + j * kAttnWKRow + 16 * g;
    f32x16 s0 = f32x16{}, s1 = f32x16{};
#pragma unroll
    for (int st = 0; st < KS; st += 2) {
      const u16x8 k0 = *(const lds_u16x8*)uintptr_t(kr + 32 * st);
      const u16x8 k1 = *(const lds_u16x8*)uintptr_t(kr + 32 * st + 32);
      s0 = mfma16<BF16>(k0, qf[st], s0);
      s1 = mfma16<BF16>(k1, qf[st + 1], s1);
    }
    f32x16 s = s0 + s1;
    const int32_t lim = (P.causal ? min(qlim, int32_t(C) - 1) : int32_t(C) - 1) - int32_t(key0);
#pragma unroll
    for (int v = 0; v < 16; ++v)
      if (int32_t(8 * (v >> 2) + 4 * g + (v & 3)) > lim) s[v] = -INFINITY;
    float mx = -INFINITY;
#pragma unroll
    for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s[v]);
    mx = fmaxf(mx, xor32(mx));
    const float m_new = fmaxf(m_run, mx * sl2);
    const float mu = m_new == -INFINITY ? 0.0f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - mu);
    m_run = m_new;
    u16x8 pf[2];
    float rs = 0.0f;
#pragma unroll
    for (int ps = 0; ps < 2; ++ps) {
      float e[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) e[i] = __builtin_amdgcn_exp2f(fmaf(s[8 * ps + i], sl2, -mu));
      const v4u w = v4u_make(pack_h2<BF16>(e[0], e[1]), pack_h2<BF16>(e[2], e[3]), pack_h2<BF16>(e[4], e[5]),
                             pack_h2<BF16>(e[6], e[7]));
      pf[ps] = __builtin_bit_cast(u16x8, w);
      rs = dot2_ones<BF16>(w.x, rs);
      rs = dot2_ones<BF16>(w.y, rs);
      rs = dot2_ones<BF16>(w.z, rs);
      rs = dot2_ones<BF16>(w.w, rs);
    }
    l_part = fmaf(l_part, alpha, rs);
#pragma unroll
    for (int i = 0; i < DB; ++i) o[i] *= alpha;
#pragma unroll
    for (int ps = 0; ps < 2; ++ps) {
      const uint32_t r0 = vbase + (16 * ps + 4 * g + e4) * kAttnWVRow + vcol;
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)uintptr_t(r0 + 64 * db));
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)uintptr_t(r0 + 8 * kAttnWVRow + 64 * db));
        const u16x8 vf = __builtin_bit_cast(u16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        o[db] = mfma16<BF16>(vf, pf[ps], o[db]);
      }
    }
  };

  __syncthreads();                      // LDS free from the previous user
  if (nblk) {
    load(0);
    store(0, 0);
  }
  __syncthreads();
  for (uint32_t kb = 0; kb < nblk; ++kb) {
    if (kb + 1 < nblk) load(kb + 1);
    if (wave_rows && (!P.causal || int32_t(kb * kAttnF32Keys) <= wq_hi)) body(kb & 1, kb * kAttnF32Keys);
    if (kb + 1 < nblk) store((kb + 1) & 1, kb + 1);
    __syncthreads();
  }

  const float l = l_part + xor32(l_part);
  const uint32_t q = qw0 + j, vq = vrow0 + 32 * wave + j;
  if (q < T && vq >= vlo && vq < vhi) {
    // a row with no visible key (causal, T > C) has l = 0 and O = 0 and stores NaN,
    // as the reference's kernel does (attention.cl:155) and softmax of a -inf row
    const float inv = 1.0f / l;
    const uint64_t obase = (uint64_t(h) * T + q) * hd;
#pragma unroll
    for (int i = 0; i < DB; ++i)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const uint32_t d = 32 * i + 8 * jj + 4 * g;
        if (d < hd)
          st4(Ob, dt, obase + d,
              v4f_make(o[i][4 * jj] * inv, o[i][4 * jj + 1] * inv, o[i][4 * jj + 2] * inv, o[i][4 * jj + 3] * inv));
      }
  }
}

template <bool BF16>
VM_DEV void attn_h16w_run(Args A, uint32_t ti, uint32_t lo, uint32_t hi) {
  A = uargs(A);
  attn_lane128(A, ti, lo, hi, [&](uint32_t h, uint32_t r0, uint32_t v0, uint32_t vl, uint32_t vh) {
    attn_block_h16w<BF16>(A, ti, h, r0, v0, vl, vh);
  });
}

// One leaf holds every attention variant inlined, so the kernel's dispatch switch
// has a single call site for the op.  Each call site costs the kernel code and
// register moves around it: with the ten variants as leaves of their own, the
// kernel's decode loop (C5) ran 3 % slower.
VM_LEAF void flash_attn_tiles(Args A, uint32_t ti, uint32_t lo, uint32_t hi) {
  A = uargs(A);
  const VM_K Task& t = task_of(A, ti);
  const AttnDesc P = attn_desc(A, t);
  const uint32_t adt = (t.tile_op >> 16) & 0xFF, dt = (t.tile_op >> 8) & 0xFF;
  // head sizes other than 64 and 128 (multiples of 8 up to 128) run the next
  // larger kernel on zero-padded rows
  const bool fast = (adt == DT_BF16 || adt == DT_F16) && P.hd % 8 == 0 && P.hd >= 8 && P.hd <= 128 && !P.qv &&
                    !P.vv && is_kt_view(aux_of(A), P.kv, P.H, P.C, P.hd) && P.scale > 0.0f &&
                    (dt == DT_F32 || dt == DT_BF16 || dt == DT_F16);
  const bool fast32 = adt == DT_F32 && P.hd % 4 == 0 && P.hd >= 4 && P.hd <= 128 && !P.qv && !P.vv &&
                      is_kt_view(aux_of(A), P.kv, P.H, P.C, P.hd) && P.scale > 0.0f &&
                      (dt == DT_F32 || dt == DT_BF16 || dt == DT_F16);
  if (fast32) return attn_f32_run(A, ti, lo, hi);
  const bool wide = (adt == DT_BF16 || adt == DT_F16) && P.hd % 8 == 0 && P.hd > 128 && P.hd <= 256 && !P.qv &&
                    !P.vv && is_kt_view(aux_of(A), P.kv, P.H, P.C, P.hd) && P.scale > 0.0f &&
                    (dt == DT_F32 || dt == DT_BF16 || dt == DT_F16);
  if (wide) return adt == DT_BF16 ? attn_h16w_run<true>(A, ti, lo, hi) : attn_h16w_run<false>(A, ti, lo, hi);
  if (!fast) return attn_rows_generic(A, ti, lo, hi);
  if (adt == DT_BF16) {
    if (P.hd == 128) attn_fast<128, true, false>(A, ti, lo, hi);
    else if (P.hd == 64) attn_fast<64, true, false>(A, ti, lo, hi);
    else if (P.hd > 64) attn_fast<128, true, true>(A, ti, lo, hi);
    else attn_fast<64, true, true>(A, ti, lo, hi);
  } else {
    if (P.hd == 128) attn_fast<128, false, false>(A, ti, lo, hi);
    else if (P.hd == 64) attn_fast<64, false, false>(A, ti, lo, hi);
    else if (P.hd > 64) attn_fast<128, false, true>(A, ti, lo, hi);
    else attn_fast<64, false, true>(A, ti, lo, hi);
  }
}

}  // namespace vm
