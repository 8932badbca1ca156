// Reductions and fused row ops (ops/reduce.cl semantics):
//   TOP_RED_PART / TOP_RED_COMB  two-phase flat reduce (reduce.cl:90-153, 529-549)
//   TOP_RED_SEG                  per-row reduce, GEMV dot mode (reduce.cl:165-281)
//   TOP_RED_STRIDED              reduce over an interior axis (reduce.cl:488-527)
//   TOP_SOFTMAX_SEG              row softmax (reduce.cl:304-392)
//   TOP_LAYERNORM_SEG            row layernorm (reduce.cl:399-479) + the affine /
//                                tanh-GELU / output-convert extension flags
//   TOP_ARGMAX_SEG               (value, first index) of the row maximum
// Float reductions accumulate in f32 through DPP wave reductions; integer ones are
// exact.  Kinds: 0 sum, 1 max, 2 min, 3 prod, 4 and, 5 or, 6 xor.
#pragma once
#include "vm_math.h"

namespace vm {

// LDS-only block barrier: orders LDS traffic between the waves of the block
// without waiting for outstanding global loads (prefetches stay in flight).
VM_DEV void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

VM_DEV float* lds_f32() { return lds_ptr<float>(); }

template <class Op>
VM_DEV float block_reduce(float x, Op op, float* red) {
  const float w = wave_reduce(x, op);
  lds_barrier();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = w;
  lds_barrier();
  float r = red[0];
#pragma unroll
  for (int k = 1; k < kWaves; ++k) r = op(r, red[k]);
  return r;
}

VM_DEV float fred_ident(uint32_t kind) {
  return kind == 0 ? 0.0f : kind == 1 ? -INFINITY : kind == 2 ? INFINITY : 1.0f;
}
VM_DEV float fred(uint32_t kind, float a, float b) {
  return kind == 0 ? a + b : kind == 1 ? fmaxf(a, b) : kind == 2 ? fminf(a, b) : a * b;
}
VM_DEV float block_reduce_kind(float x, uint32_t kind, float* red) {
  switch (kind) {
    case 0: return block_reduce(x, OpSum(), red);
    case 1: return block_reduce(x, OpMax(), red);
    case 2: return block_reduce(x, OpMin(), red);
    default: return block_reduce(x, OpProd(), red);
  }
}

// ---- integer kinds (reduce.cl:16-40; u32 compares unsigned) -----------------------------
template <typename T>
VM_DEV T ired_ident(uint32_t kind, bool uns) {
  constexpr bool k64 = sizeof(T) == 8;
  switch (kind) {
    case 0: return 0;
    case 1: return uns ? T(0) : (k64 ? T(INT64_MIN) : T(INT32_MIN));
    case 2: return uns ? T(~T(0)) : (k64 ? T(INT64_MAX) : T(INT32_MAX));
    case 3: return 1;
    case 4: return T(~T(0));
    default: return 0;
  }
}
template <typename T, typename U>
VM_DEV T ired(uint32_t kind, bool uns, T a, T b) {
  switch (kind) {
    case 0: return T(U(a) + U(b));
    case 1: return uns ? (U(a) > U(b) ? a : b) : (a > b ? a : b);
    case 2: return uns ? (U(a) < U(b) ? a : b) : (a < b ? a : b);
    case 3: return T(U(a) * U(b));
    case 4: return a & b;
    case 5: return a | b;
    default: return a ^ b;
  }
}

// Block reduction of an integer value through an LDS tree (exact).
template <typename T, typename U>
VM_DEV T block_ireduce(T v, uint32_t kind, bool uns) {
  T* tree = lds_ptr<T>();
  lds_barrier();
  tree[threadIdx.x] = v;
  lds_barrier();
  for (int s = kBlock / 2; s > 0; s >>= 1) {
    if (int(threadIdx.x) < s) tree[threadIdx.x] = ired<T, U>(kind, uns, tree[threadIdx.x], tree[threadIdx.x + s]);
    lds_barrier();
  }
  return tree[0];
}

VM_DEV int64_t load_i(const gbyte* p, uint32_t dt, uint64_t i) {
  switch (dt) {
    case DT_I64: return gcast<int64_t>(p)[i];
    case DT_U32: return int64_t(gcast<uint32_t>(p)[i]);
    case DT_BOOL: return p[i] != 0;
    default: return gcast<int32_t>(p)[i];
  }
}
VM_DEV void store_i(gbyte* p, uint32_t dt, uint64_t i, int64_t v) {
  switch (dt) {
    case DT_I64: gcast<int64_t>(p)[i] = v; break;
    case DT_BOOL: p[i] = uint8_t(v & 1); break;
    default: gcast<uint32_t>(p)[i] = uint32_t(uint64_t(v)); break;
  }
}
VM_DEV bool is_int_dt(uint32_t dt) { return dt == DT_I32 || dt == DT_U32 || dt == DT_I64 || dt == DT_BOOL; }

// Integer reduction of src[i0, i1) by the whole block.
VM_DEV int64_t block_int_range(const gbyte* src, uint32_t dt, uint32_t kind, uint64_t i0, uint64_t i1) {
  if (dt == DT_I64) {
    int64_t acc = ired_ident<int64_t>(kind, false);
    for (uint64_t i = i0 + threadIdx.x; i < i1; i += kBlock)
      acc = ired<int64_t, uint64_t>(kind, false, acc, load_i(src, dt, i));
    return block_ireduce<int64_t, uint64_t>(acc, kind, false);
  }
  const bool uns = dt == DT_U32;
  int32_t acc = ired_ident<int32_t>(kind, uns);
  if (dt == DT_BOOL && kind == 1) acc = 0;       // bool max identity is false
  if (dt == DT_BOOL && kind == 2) acc = 1;       // bool min identity is true
  for (uint64_t i = i0 + threadIdx.x; i < i1; i += kBlock)
    acc = ired<int32_t, uint32_t>(kind, uns, acc, int32_t(load_i(src, dt, i)));
  return int64_t(uint32_t(block_ireduce<int32_t, uint32_t>(acc, kind, uns)));
}

// ---- TOP_RED_PART / TOP_RED_COMB -----------------------------------------------------
// RED_PART: p0 n, p1 chunk, p2 kind; tile k reduces [k*chunk, (k+1)*chunk) into dst[k].
// RED_COMB: p0 n_parts, p1 kind; one tile reduces the partials into dst[0].
VM_TILE void red_flat_tiles(Args A, uint32_t ti, uint32_t lo, uint32_t hi, bool comb) {
  A = uargs(A);
  const VM_K Task& t = task_of(A, ti);
  const uint32_t n = t.p[0], chunk = comb ? t.p[0] : t.p[1], kind = comb ? t.p[1] : t.p[2];
  const uint32_t dt = (t.tile_op >> 8) & 0xFF;
  const gbyte* a = resolve(A, t.a);
  gbyte* d = resolve(A, t.dst);
  if (comb) hi = min(hi, 1u);
  for (uint32_t tile = lo; tile < hi; ++tile) {
    const uint64_t s0 = uint64_t(tile) * chunk, s1 = min(s0 + chunk, uint64_t(n));
    if (is_int_dt(dt)) {
      const int64_t r = block_int_range(a, dt, kind, s0, s1);
      if (threadIdx.x == 0) store_i(d, dt, tile, r);
    } else {
      float acc = fred_ident(kind);
      for (uint64_t i = s0 + threadIdx.x; i < s1; i += kBlock) acc = fred(kind, acc, load_f(a, dt, i));
      const float r = block_reduce_kind(acc, kind, lds_f32());
      if (threadIdx.x == 0) store_f(d, dt, tile, r);
    }
  }
}

// ---- TOP_RED_SEG -----------------------------------------------------------------------
// p0 n_out, p1 seg, p2 kind, p3 dot mode (row . vector at b, GEMV routing).
VM_TILE void red_seg_tiles(Args A, uint32_t ti, uint32_t lo, uint32_t hi) {
  A = uargs(A);
  const VM_K Task& t = task_of(A, ti);
  const uint32_t n_out = t.p[0], seg = t.p[1], kind = t.p[2], dot = t.p[3];
  const uint32_t dt = (t.tile_op >> 8) & 0xFF, adt = (t.tile_op >> 16) & 0xFF;
  const gbyte* a = resolve(A, t.a);
  const gbyte* bv = resolve(A, t.b);
  gbyte* d = resolve(A, t.dst);
  hi = min(hi, n_out);
  if (is_int_dt(dt) && !dot) {
    for (uint32_t o = lo; o < hi; ++o) {
      const int64_t r = block_int_range(a, dt, kind, uint64_t(o) * seg, uint64_t(o + 1) * seg);
      if (threadIdx.x == 0) store_i(d, dt, o, r);
    }
    return;
  }
  if (seg <= 32 && !dot) {             // short rows: one thread per row
    for (uint32_t o = lo + threadIdx.x; o < hi; o += kBlock) {
      float acc = fred_ident(kind);
      for (uint32_t j = 0; j < seg; ++j) acc = fred(kind, acc, load_f(a, adt, uint64_t(o) * seg + j));
      store_f(d, dt, o, acc);
    }
    return;
  }
  float* red = lds_f32();
  const bool vec = adt == DT_F32 && (seg & 3) == 0 && ((uintptr_t(a) | uintptr_t(bv)) & 15) == 0;
  for (uint32_t o = lo; o < hi; ++o) {
    const uint64_t base = uint64_t(o) * seg;
    float acc = dot ? 0.0f : fred_ident(kind);
    if (vec) {
      const VM_G v4f* r4 = (const VM_G v4f*)(gcast<float>(a) + base);
      const VM_G v4f* v4 = (const VM_G v4f*)gcast<float>(bv);
      for (uint32_t j = threadIdx.x; j < (seg >> 2); j += kBlock) {
        const v4f x = r4[j];
        if (dot) {
          const v4f y = v4[j];
          acc = fmaf(x.x, y.x, fmaf(x.y, y.y, fmaf(x.z, y.z, fmaf(x.w, y.w, acc))));
        } else {
          acc = fred(kind, acc, fred(kind, fred(kind, x.x, x.y), fred(kind, x.z, x.w)));
        }
      }
    } else {
      for (uint32_t j = threadIdx.x; j < seg; j += kBlock) {
        const float x = load_f(a, adt, base + j);
        acc = dot ? fmaf(x, load_f(bv, adt, j), acc) : fred(kind, acc, x);
      }
    }
    const float r = block_reduce_kind(acc, dot ? 0u : kind, red);
    if (threadIdx.x == 0) store_f(d, dt, o, r);
  }
}

// ---- TOP_RED_STRIDED ----------------------------------------------------------------------
// out[o*inner + i] = reduce_r in[(o*red + r)*inner + i]; p0 n_out, p1 red, p2 inner,
// p3 kind; tiles of ew_ts outputs, one thread per output.
VM_TILE void red_strided_tiles(Args A, uint32_t ti, uint32_t lo, uint32_t hi) {
  A = uargs(A);
  const VM_K Task& t = task_of(A, ti);
  const uint32_t n_out = t.p[0], red = t.p[1], inner = t.p[2], kind = t.p[3];
  const uint32_t dt = (t.tile_op >> 8) & 0xFF, adt = (t.tile_op >> 16) & 0xFF;
  const gbyte* a = resolve(A, t.a);
  gbyte* d = resolve(A, t.dst);
  const uint64_t e0 = uint64_t(lo) * A->ew_ts, e1 = min(uint64_t(hi) * A->ew_ts, uint64_t(n_out));
  for (uint64_t q = e0 + threadIdx.x; q < e1; q += kBlock) {
    const uint64_t o = q / inner, i = q % inner;
    const uint64_t base = o * uint64_t(red) * inner + i;
    if (is_int_dt(dt)) {
      if (dt == DT_I64) {
        int64_t acc = ired_ident<int64_t>(kind, false);
        for (uint32_t r = 0; r < red; ++r)
          acc = ired<int64_t, uint64_t>(kind, false, acc, load_i(a, dt, base + uint64_t(r) * inner));
        store_i(d, dt, q, acc);
      } else {
        const bool uns = dt == DT_U32;
        int32_t acc = ired_ident<int32_t>(kind, uns);
        if (dt == DT_BOOL && kind == 1) acc = 0;
        if (dt == DT_BOOL && kind == 2) acc = 1;
        for (uint32_t r = 0; r < red; ++r)
          acc = ired<int32_t, uint32_t>(kind, uns, acc, int32_t(load_i(a, dt, base + uint64_t(r) * inner)));
        store_i(d, dt, q, int64_t(uint32_t(acc)));
      }
    } else {
      float acc = fred_ident(kind);
      for (uint32_t r = 0; r < red; ++r) acc = fred(kind, acc, load_f(a, adt, base + uint64_t(r) * inner));
      store_f(d, dt, q, acc);
    }
  }
}

// ---- row-resident fused ops -------------------------------------------------------------
// A row of `seg` elements is held in registers as NV v4f per thread (thread t
// owns v4f slots t, t+256, ...), so a row costs one HBM read and one write.
// The next row's loads are issued before the current row's reductions.

template <int NV>
struct Row { v4f v[NV]; };

template <int NV>
VM_DEV void row_load(Row<NV>& r, const gbyte* p, uint32_t dt, uint64_t base, uint32_t nv4) {
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const uint32_t q = threadIdx.x + k * kBlock;
    if (q < nv4) r.v[k] = ld4(p, dt, base + 4ull * q);
  }
}

// LAYERNORM_SEG over rows [r0, r1): p0 n_out, p1 seg, p2 eps bits, p3 flags,
// b = gamma, p4 = beta (LN_AFFINE).
template <int NV>
VM_DEV void ln_rows_vec(Args A, uint32_t ti, uint32_t r0, uint32_t r1) {
  A = uargs(A);
  const VM_K Task& t = task_of(A, ti);
  float* red = lds_f32();
  const uint32_t seg = t.p[1], flags = t.p[3];
  const float eps = __uint_as_float(t.p[2]);
  const uint32_t dt = (t.tile_op >> 8) & 0xFF, adt = (t.tile_op >> 16) & 0xFF;
  const gbyte* a = resolve(A, t.a);
  gbyte* d = resolve(A, t.dst);
  const bool affine = flags & LN_AFFINE, do_gelu = flags & LN_GELU, two_pass = flags & LN_TWO_PASS;
  const gbyte* gp = resolve(A, affine ? t.b : t.a);
  const gbyte* bp = resolve(A, affine ? t.p[4] : t.a);
  const uint32_t nv4 = seg >> 2;
  const float inv_n = 1.0f / float(seg);
  // gamma / beta slots of this thread stay in registers for every row
  Row<NV> g, be;
  if (affine) {
    row_load(g, gp, DT_F32, 0, nv4);
    row_load(be, bp, DT_F32, 0, nv4);
  }
  Row<NV> x, xn;
  row_load(x, a, adt, uint64_t(r0) * seg, nv4);
  for (uint32_t r = r0; r < r1; ++r) {
    if (r + 1 < r1) row_load(xn, a, adt, uint64_t(r + 1) * seg, nv4);
    float s = 0.0f, s2 = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      if (threadIdx.x + k * kBlock < nv4) {
        const v4f v = x.v[k];
        s += (v.x + v.y) + (v.z + v.w);
        if (!two_pass) s2 = fmaf(v.x, v.x, fmaf(v.y, v.y, fmaf(v.z, v.z, fmaf(v.w, v.w, s2))));
      }
    }
    const float mean = block_reduce(s, OpSum(), red) * inv_n;
    float var;
    if (two_pass) {
      float q = 0.0f;
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        if (threadIdx.x + k * kBlock < nv4) {
          const v4f v = x.v[k];
          const float dx = v.x - mean, dy = v.y - mean, dz = v.z - mean, dw = v.w - mean;
          q = fmaf(dx, dx, fmaf(dy, dy, fmaf(dz, dz, fmaf(dw, dw, q))));
        }
      }
      var = block_reduce(q, OpSum(), red + kWaves) * inv_n;
    } else {
      var = block_reduce(s2, OpSum(), red + kWaves) * inv_n - mean * mean;
    }
    const float rstd = rsqrtf(var + eps);
    const float shift = -mean * rstd;
    const uint64_t base = uint64_t(r) * seg;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const uint32_t q = threadIdx.x + k * kBlock;
      if (q < nv4) {
        float y[4] = {x.v[k].x, x.v[k].y, x.v[k].z, x.v[k].w};
        const float gg[4] = {g.v[k].x, g.v[k].y, g.v[k].z, g.v[k].w};
        const float bb[4] = {be.v[k].x, be.v[k].y, be.v[k].z, be.v[k].w};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          float z = fmaf(y[c], rstd, shift);
          if (affine) z = fmaf(z, gg[c], bb[c]);
          if (do_gelu) z = gelu(z);
          y[c] = z;
        }
        st4(d, dt, base + 4ull * q, v4f_make(y[0], y[1], y[2], y[3]));
      }
    }
    if (r + 1 < r1) x = xn;
  }
}

// Wave-per-row layernorm, specialised on the input / output formats.  Each wave64
// owns every fourth row of the lane's range and holds a row as NV groups of 4
// elements per thread (thread t: groups t, t+64, ...; f32 rows as float4, bf16 rows
// packed two per register).  Rows stream through three rotating register buffers,
// so two rows are in flight while the third is reduced (DPP only, no block
// barriers) and written.  gamma / beta (1 / 0 when the op has no affine) are staged
// once into LDS.
template <bool BF16>
struct RowFmt {
  typedef v4f Raw;                       // f32: 4 elements in a float4
  static VM_DEV v4f unpack(Raw r) { return r; }
};
template <>
struct RowFmt<true> {
  typedef v2u Raw;                       // bf16: 4 elements in two registers
  static VM_DEV v4f unpack(Raw r) {
    return v4f_make(__uint_as_float(r.x << 16), __uint_as_float(r.x & 0xFFFF0000u), __uint_as_float(r.y << 16),
                    __uint_as_float(r.y & 0xFFFF0000u));
  }
};

struct LnRow {                 // per-row constants of one layernorm task
  const gbyte* a;
  gbyte* d;
  const v4f* lg;
  const v4f* lb;
  uint32_t seg, nv4, lane;
  uint32_t ichunk, istride;      // row interleave: row i -> (i % ichunk) * istride + i / ichunk
  float eps, inv_n;
  bool two_pass;
};

// Loads are never predicated: a load inside an exec-masked block makes the
// compiler drain every outstanding load (s_waitcnt vmcnt(0)) at the block
// boundary, which would serialise the row prefetch.  Groups past the row end
// re-read the row's last group and are masked out of the sums and stores.
// The rows are read once, so the loads are non-temporal (streaming): C2 with
// every step reading HBM (three rotating sets), alternating runs on one
// MI355X: 42.3 against 45.7-46.3 us; one set left in the memory-side cache
// then runs at about the same 41 us instead of 39.
template <int NV, bool IN_BF16, bool FULL>
VM_DEV void ln_load(typename RowFmt<IN_BF16>::Raw (&buf)[NV], const LnRow& L, uint32_t r) {
  typedef typename RowFmt<IN_BF16>::Raw Raw;
  r = (r % L.ichunk) * L.istride + r / L.ichunk;
  const VM_G Raw* rp = (const VM_G Raw*)(L.a + uint64_t(r) * L.seg * (IN_BF16 ? 2 : 4));
#pragma unroll
  for (int k = 0; k < NV; ++k)
    buf[k] = __builtin_nontemporal_load(&rp[FULL ? L.lane + 64 * k : min(L.lane + 64 * k, L.nv4 - 1)]);
}

template <int NV, bool IN_BF16, bool OUT_BF16, bool GELU, bool FULL>
VM_DEV void ln_process(const typename RowFmt<IN_BF16>::Raw (&buf)[NV], const LnRow& L, uint32_t r) {
  float s = 0.0f, s2 = 0.0f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const bool valid = FULL || L.lane + 64 * k < L.nv4;
    const v4f x = RowFmt<IN_BF16>::unpack(buf[k]);
    const float ps = (x.x + x.y) + (x.z + x.w);
    s += valid ? ps : 0.0f;
    if (!L.two_pass) {
      const float p2 = fmaf(x.x, x.x, fmaf(x.y, x.y, fmaf(x.z, x.z, x.w * x.w)));
      s2 += valid ? p2 : 0.0f;
    }
  }
  const float mean = wave_sum(s) * L.inv_n;
  float var;
  if (L.two_pass) {
    float q2 = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const bool valid = FULL || L.lane + 64 * k < L.nv4;
      const v4f dv = RowFmt<IN_BF16>::unpack(buf[k]) - mean;
      const float p2 = fmaf(dv.x, dv.x, fmaf(dv.y, dv.y, fmaf(dv.z, dv.z, dv.w * dv.w)));
      q2 += valid ? p2 : 0.0f;
    }
    var = wave_sum(q2) * L.inv_n;
  } else {
    var = wave_sum(s2) * L.inv_n - mean * mean;
  }
  const float rstd = rsqrtf(var + L.eps);
  const float shift = -mean * rstd;
  r = (r % L.ichunk) * L.istride + r / L.ichunk;
  gbyte* rowd = L.d + uint64_t(r) * L.seg * (OUT_BF16 ? 2 : 4);
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    // one group at a time: keeps the GELU temporaries of 4 elements live, not 64
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t q = FULL ? L.lane + 64 * k : min(L.lane + 64 * k, L.nv4 - 1);
    {
      const v4f x = RowFmt<IN_BF16>::unpack(buf[k]);
      const v4f gg = L.lg[q], bb = L.lb[q];
      v4f z;
      z.x = fmaf(fmaf(x.x, rstd, shift), gg.x, bb.x);
      z.y = fmaf(fmaf(x.y, rstd, shift), gg.y, bb.y);
      z.z = fmaf(fmaf(x.z, rstd, shift), gg.z, bb.z);
      z.w = fmaf(fmaf(x.w, rstd, shift), gg.w, bb.w);
      if constexpr (GELU) {
        z.x = gelu(z.x);
        z.y = gelu(z.y);
        z.z = gelu(z.z);
        z.w = gelu(z.w);
      }
      if (FULL || L.lane + 64 * k < L.nv4) {
        // streaming stores: the rows are not read again by this launch (C2,
        // alternating runs: 38.2 against 38.7 us; streaming loads were slower)
        if constexpr (OUT_BF16)
          __builtin_nontemporal_store(v2u_make(pack_bf16x2(z.x, z.y), pack_bf16x2(z.z, z.w)), &((VM_G v2u*)rowd)[q]);
        else
          __builtin_nontemporal_store(z, &((VM_G v4f*)rowd)[q]);
      }
    }
  }
}

// Rows i = 0..mine-1 of this wave (row rbase + 4i) through rotating register
// buffers: while one row is reduced and written, the next one or two are in
// flight.  The prefetch is unconditional (past the last row it re-reads the last
// row) so no load sits behind a branch; `mine` is wave-uniform, so the loop exits
// are scalar branches.
template <int NV, bool IN_BF16, bool OUT_BF16, bool GELU, bool FULL>
VM_DEV void ln_stream(const LnRow& L, uint32_t rbase, uint32_t mine) {
  typedef typename RowFmt<IN_BF16>::Raw Raw;
  if (mine == 0) return;
  const uint32_t lastr = rbase + kWaves * (mine - 1);
  if constexpr (NV * sizeof(Raw) / 4 > 32) {
    // a row larger than 32 registers: two buffers (one row in flight)
    Raw b0[NV], b1[NV];
    ln_load<NV, IN_BF16, FULL>(b0, L, rbase);
    for (uint32_t i = 0; i < mine; i += 2) {
      const uint32_t r = rbase + kWaves * i;
      ln_load<NV, IN_BF16, FULL>(b1, L, min(r + kWaves, lastr));
      ln_process<NV, IN_BF16, OUT_BF16, GELU, FULL>(b0, L, r);
      if (i + 1 >= mine) break;
      ln_load<NV, IN_BF16, FULL>(b0, L, min(r + 2 * kWaves, lastr));
      ln_process<NV, IN_BF16, OUT_BF16, GELU, FULL>(b1, L, r + kWaves);
    }
    return;
  }
  Raw b0[NV], b1[NV], b2[NV];
  ln_load<NV, IN_BF16, FULL>(b0, L, rbase);
  ln_load<NV, IN_BF16, FULL>(b1, L, min(rbase + kWaves, lastr));
  for (uint32_t i = 0; i < mine; i += 3) {
    const uint32_t r = rbase + kWaves * i;
    ln_load<NV, IN_BF16, FULL>(b2, L, min(r + 2 * kWaves, lastr));
    ln_process<NV, IN_BF16, OUT_BF16, GELU, FULL>(b0, L, r);
    if (i + 1 >= mine) break;
    ln_load<NV, IN_BF16, FULL>(b0, L, min(r + 3 * kWaves, lastr));
    ln_process<NV, IN_BF16, OUT_BF16, GELU, FULL>(b1, L, r + kWaves);
    if (i + 2 >= mine) break;
    ln_load<NV, IN_BF16, FULL>(b1, L, min(r + 4 * kWaves, lastr));
    ln_process<NV, IN_BF16, OUT_BF16, GELU, FULL>(b2, L, r + 2 * kWaves);
  }
}

template <int NV, bool IN_BF16, bool OUT_BF16, bool FULL>
VM_DEV void ln_rows_fast(Args A, uint32_t ti, uint32_t r0, uint32_t r1) {
  A = uargs(A);
  const VM_K Task& t = task_of(A, ti);
  r0 = uni(r0);
  r1 = uni(r1);
  const uint32_t flags = t.p[3];
  const bool affine = flags & LN_AFFINE;
  LnRow L;
  L.seg = t.p[1];
  L.nv4 = L.seg >> 2;
  L.eps = __uint_as_float(t.p[2]);
  L.inv_n = 1.0f / float(L.seg);
  L.two_pass = flags & LN_TWO_PASS;
  L.a = resolve(A, t.a);
  L.d = resolve(A, t.dst);
  L.lane = threadIdx.x & 63;
  // p5: row interleave (0: none; the loader checks that it divides n_out)
  L.ichunk = t.p[5] ? t.p[5] : 0xFFFFFFFFu;
  L.istride = t.p[5] ? t.p[0] / t.p[5] : 1u;
  const uint32_t wave = uni(threadIdx.x >> 6);       // wave-uniform: scalar loop control
  v4f* lg = lds_ptr<v4f>();
  v4f* lb = lg + L.nv4;
  {
    const VM_G v4f* g4 = (const VM_G v4f*)gcast<float>(resolve(A, affine ? t.b : t.a));
    const VM_G v4f* b4 = (const VM_G v4f*)gcast<float>(resolve(A, affine ? t.p[4] : t.a));
    for (uint32_t q = threadIdx.x; q < L.nv4; q += kBlock) {
      lg[q] = affine ? g4[q] : v4f{1.0f, 1.0f, 1.0f, 1.0f};
      lb[q] = affine ? b4[q] : v4f{0.0f, 0.0f, 0.0f, 0.0f};
    }
  }
  L.lg = lg;
  L.lb = lb;
  __syncthreads();
  const uint32_t mine = r1 > r0 + wave ? (r1 - r0 - wave + kWaves - 1) / kWaves : 0;
  if (flags & LN_GELU) ln_stream<NV, IN_BF16, OUT_BF16, true, FULL>(L, r0 + wave, mine);
  else ln_stream<NV, IN_BF16, OUT_BF16, false, FULL>(L, r0 + wave, mine);
}

// Wave-per-row layernorm for rows up to 4096 elements: each wave64 owns every
// fourth row of the lane's range, holds it as NV float4 per thread (thread t:
// float4 slots t, t+64, ...), prefetches its next row before reducing the current
// one, and reduces with DPP only -- no block barriers, four rows in flight per CU.
// gamma / beta are staged once into LDS and read back per row.
template <int NV>
VM_DEV void ln_rows_wave(Args A, uint32_t ti, uint32_t r0, uint32_t r1) {
  A = uargs(A);
  const VM_K Task& t = task_of(A, ti);
  const uint32_t seg = t.p[1], flags = t.p[3];
  const float eps = __uint_as_float(t.p[2]);
  const uint32_t dt = (t.tile_op >> 8) & 0xFF, adt = (t.tile_op >> 16) & 0xFF;
  const gbyte* a = resolve(A, t.a);
  gbyte* d = resolve(A, t.dst);
  const bool affine = flags & LN_AFFINE, do_gelu = flags & LN_GELU, two_pass = flags & LN_TWO_PASS;
  const uint32_t nv4 = seg >> 2;
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v4f* lg = lds_ptr<v4f>();
  v4f* lb = lg + nv4;
  if (affine) {
    const VM_G v4f* g4 = (const VM_G v4f*)gcast<float>(resolve(A, t.b));
    const VM_G v4f* b4 = (const VM_G v4f*)gcast<float>(resolve(A, t.p[4]));
    for (uint32_t q = threadIdx.x; q < nv4; q += kBlock) {
      lg[q] = g4[q];
      lb[q] = b4[q];
    }
  }
  __syncthreads();
  const float inv_n = 1.0f / float(seg);
  v4f x[NV], xn[NV];
  auto load_row = [&](v4f (&dst)[NV], uint32_t r) {
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const uint32_t q = lane + 64 * k;
      if (q < nv4) dst[k] = ld4(a, adt, uint64_t(r) * seg + 4ull * q);
    }
  };
  uint32_t r = r0 + wave;
  if (r < r1) load_row(x, r);
  for (; r < r1; r += kWaves) {
    if (r + kWaves < r1) load_row(xn, r + kWaves);
    float s = 0.0f, s2 = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      if (lane + 64 * k < nv4) {
        s += (x[k].x + x[k].y) + (x[k].z + x[k].w);
        if (!two_pass) s2 = fmaf(x[k].x, x[k].x, fmaf(x[k].y, x[k].y, fmaf(x[k].z, x[k].z, fmaf(x[k].w, x[k].w, s2))));
      }
    }
    const float mean = wave_sum(s) * inv_n;
    float var;
    if (two_pass) {
      float q2 = 0.0f;
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        if (lane + 64 * k < nv4) {
          const v4f dv = x[k] - mean;
          q2 = fmaf(dv.x, dv.x, fmaf(dv.y, dv.y, fmaf(dv.z, dv.z, fmaf(dv.w, dv.w, q2))));
        }
      }
      var = wave_sum(q2) * inv_n;
    } else {
      var = wave_sum(s2) * inv_n - mean * mean;
    }
    const float rstd = rsqrtf(var + eps);
    const float shift = -mean * rstd;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const uint32_t q = lane + 64 * k;
      if (q < nv4) {
        v4f z;
        z.x = fmaf(x[k].x, rstd, shift);
        z.y = fmaf(x[k].y, rstd, shift);
        z.z = fmaf(x[k].z, rstd, shift);
        z.w = fmaf(x[k].w, rstd, shift);
        if (affine) {
          const v4f gg = lg[q], bb = lb[q];
          z.x = fmaf(z.x, gg.x, bb.x);
          z.y = fmaf(z.y, gg.y, bb.y);
          z.z = fmaf(z.z, gg.z, bb.z);
          z.w = fmaf(z.w, gg.w, bb.w);
        }
        if (do_gelu) {
          z.x = gelu(z.x);
          z.y = gelu(z.y);
          z.z = gelu(z.z);
          z.w = gelu(z.w);
        }
        st4(d, dt, uint64_t(r) * seg + 4ull * q, z);
      }
    }
#pragma unroll
    for (int k = 0; k < NV; ++k) x[k] = xn[k];
  }
}

// Any seg / alignment: three passes over the row in global memory.
VM_DEV void ln_rows_generic(Args A, uint32_t ti, uint32_t r0, uint32_t r1) {
  A = uargs(A);
  const VM_K Task& t = task_of(A, ti);
  float* red = lds_f32();
  const uint32_t seg = t.p[1], flags = t.p[3];
  const float eps = __uint_as_float(t.p[2]);
  const uint32_t dt = (t.tile_op >> 8) & 0xFF, adt = (t.tile_op >> 16) & 0xFF;
  const gbyte* a = resolve(A, t.a);
  gbyte* d = resolve(A, t.dst);
  const bool affine = flags & LN_AFFINE, do_gelu = flags & LN_GELU, two_pass = flags & LN_TWO_PASS;
  const gbyte* gp = resolve(A, affine ? t.b : t.a);
  const gbyte* bp = resolve(A, affine ? t.p[4] : t.a);
  const float inv_n = 1.0f / float(seg);
  for (uint32_t r = r0; r < r1; ++r) {
    const uint64_t base = uint64_t(r) * seg;
    float s = 0.0f, s2 = 0.0f;
    for (uint32_t j = threadIdx.x; j < seg; j += kBlock) {
      const float v = load_f(a, adt, base + j);
      s += v;
      s2 = fmaf(v, v, s2);
    }
    const float mean = block_reduce(s, OpSum(), red) * inv_n;
    float var;
    if (two_pass) {
      float q = 0.0f;
      for (uint32_t j = threadIdx.x; j < seg; j += kBlock) {
        const float dv = load_f(a, adt, base + j) - mean;
        q = fmaf(dv, dv, q);
      }
      var = block_reduce(q, OpSum(), red + kWaves) * inv_n;
    } else {
      var = block_reduce(s2, OpSum(), red + kWaves) * inv_n - mean * mean;
    }
    const float rstd = rsqrtf(var + eps);
    const float shift = -mean * rstd;
    for (uint32_t j = threadIdx.x; j < seg; j += kBlock) {
      float z = fmaf(load_f(a, adt, base + j), rstd, shift);
      if (affine) z = fmaf(z, load_f(gp, DT_F32, j), load_f(bp, DT_F32, j));
      if (do_gelu) z = gelu(z);
      store_f(d, dt, base + j, z);
    }
  }
}

VM_DEV bool row_vec_ok(uint32_t seg, const gbyte* a, const gbyte* d, uint32_t adt, uint32_t dt) {
  const bool fmt = (adt == DT_F32 || adt == DT_BF16 || adt == DT_F16) &&
                   (dt == DT_F32 || dt == DT_BF16 || dt == DT_F16);
  return fmt && (seg & 3) == 0 && seg <= 8 * 4 * kBlock && ((uintptr_t(a) | uintptr_t(d)) & 15) == 0;
}

VM_DEV void layernorm_rows(Args A, uint32_t ti, uint32_t lo, uint32_t hi);

// LAYERNORM_SEG tiles [lo, hi).  Task p5 (scheduler, extension): the lanes'
// rows interleaved -- logical row i is row (i % p5) * (n_out / p5) + i / p5, so
// that at any moment the lanes stream neighbouring rows of the input (C2,
// alternating runs on one MI355X: 38.7 against 39.6 us).  The streaming row
// kernel applies it per row;
// the other row kernels take the rows one by one.
// A leaf with its row kernels inlined, for the reason ew_tile gives: as a
// function calling them it saved and reloaded 14 registers in scratch around
// every entry (C2, alternating runs: 41.6-41.8 against 42.2 us).
VM_LEAF void layernorm_tiles(Args A, uint32_t ti, uint32_t lo, uint32_t hi) {
  A = uargs(A);
  const VM_K Task& t = task_of(A, ti);
  const uint32_t n_out = t.p[0], seg = t.p[1];
  const uint32_t dt = (t.tile_op >> 8) & 0xFF, adt = (t.tile_op >> 16) & 0xFF;
  hi = min(hi, n_out);
  if (lo >= hi) return;
  bool ok = row_vec_ok(seg, resolve(A, t.a), resolve(A, t.dst), adt, dt);
  if (ok && (t.p[3] & LN_AFFINE)) ok = ((uintptr_t(resolve(A, t.b)) | uintptr_t(resolve(A, t.p[4]))) & 15) == 0;
  const uint32_t nv4 = seg >> 2;
  const bool fast = ok && (adt == DT_F32 || adt == DT_BF16) && (dt == DT_F32 || dt == DT_BF16) && nv4 <= 16 * 64;
  if (t.p[5] && !fast) {
    const uint32_t c = t.p[5], stride = n_out / c;
    for (uint32_t i = lo; i < hi; ++i) {
      const uint32_t r = (i % c) * stride + i / c;
      layernorm_rows(A, ti, r, r + 1);
    }
    return;
  }
  layernorm_rows(A, ti, lo, hi);
}

// Rows [lo, hi) of a LAYERNORM_SEG task through the fitting row kernel (rows
// taken as they are, except the streaming kernel, which applies p5 itself).
VM_DEV void layernorm_rows(Args A, uint32_t ti, uint32_t lo, uint32_t hi) {
  const VM_K Task& t = task_of(A, ti);
  const uint32_t seg = t.p[1];
  const uint32_t dt = (t.tile_op >> 8) & 0xFF, adt = (t.tile_op >> 16) & 0xFF;
  bool ok = row_vec_ok(seg, resolve(A, t.a), resolve(A, t.dst), adt, dt);
  if (ok && (t.p[3] & LN_AFFINE)) ok = ((uintptr_t(resolve(A, t.b)) | uintptr_t(resolve(A, t.p[4]))) & 15) == 0;
  if (!ok) return ln_rows_generic(A, ti, lo, hi);
  const uint32_t nv4 = seg >> 2;
  if ((adt == DT_F32 || adt == DT_BF16) && (dt == DT_F32 || dt == DT_BF16) && nv4 <= 16 * 64) {
    const bool ib = adt == DT_BF16, ob = dt == DT_BF16;
#define VM_LN_FAST(NVV, FULLV)                                                               \
    {                                                                                         \
      if (ib) return ob ? ln_rows_fast<NVV, true, true, FULLV>(A, ti, lo, hi)                  \
                        : ln_rows_fast<NVV, true, false, FULLV>(A, ti, lo, hi);                \
      return ob ? ln_rows_fast<NVV, false, true, FULLV>(A, ti, lo, hi)                         \
                : ln_rows_fast<NVV, false, false, FULLV>(A, ti, lo, hi);                       \
    }
    if (nv4 == 4 * 64) VM_LN_FAST(4, true)
    if (nv4 < 4 * 64) VM_LN_FAST(4, false)
    if (nv4 == 16 * 64) VM_LN_FAST(16, true)
    VM_LN_FAST(16, false)
#undef VM_LN_FAST
  }
  if (nv4 <= 2 * 64) return ln_rows_wave<2>(A, ti, lo, hi);
  if (nv4 <= 4 * 64) return ln_rows_wave<4>(A, ti, lo, hi);
  if (nv4 <= 8 * 64) return ln_rows_wave<8>(A, ti, lo, hi);
  if (nv4 <= 16 * 64) return ln_rows_wave<16>(A, ti, lo, hi);
  if (nv4 <= 1 * kBlock) return ln_rows_vec<1>(A, ti, lo, hi);
  if (nv4 <= 2 * kBlock) return ln_rows_vec<2>(A, ti, lo, hi);
  if (nv4 <= 4 * kBlock) return ln_rows_vec<4>(A, ti, lo, hi);
  return ln_rows_vec<8>(A, ti, lo, hi);
}

// SOFTMAX_SEG rows: exp(x - max) / sum.
template <int NV>
VM_TILE void softmax_rows_vec(Args A, uint32_t ti, uint32_t r0, uint32_t r1) {
  A = uargs(A);
  const VM_K Task& t = task_of(A, ti);
  float* red = lds_f32();
  const uint32_t seg = t.p[1];
  const uint32_t dt = (t.tile_op >> 8) & 0xFF, adt = (t.tile_op >> 16) & 0xFF;
  const gbyte* a = resolve(A, t.a);
  gbyte* d = resolve(A, t.dst);
  const uint32_t nv4 = seg >> 2;
  Row<NV> x, xn;
  row_load(x, a, adt, uint64_t(r0) * seg, nv4);
  for (uint32_t r = r0; r < r1; ++r) {
    if (r + 1 < r1) row_load(xn, a, adt, uint64_t(r + 1) * seg, nv4);
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < NV; ++k)
      if (threadIdx.x + k * kBlock < nv4) m = fmaxf(m, fmaxf(fmaxf(x.v[k].x, x.v[k].y), fmaxf(x.v[k].z, x.v[k].w)));
    m = block_reduce(m, OpMax(), red);
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      if (threadIdx.x + k * kBlock < nv4) {
        x.v[k].x = __expf(x.v[k].x - m);
        x.v[k].y = __expf(x.v[k].y - m);
        x.v[k].z = __expf(x.v[k].z - m);
        x.v[k].w = __expf(x.v[k].w - m);
        s += (x.v[k].x + x.v[k].y) + (x.v[k].z + x.v[k].w);
      }
    }
    s = block_reduce(s, OpSum(), red + kWaves);
    const float inv = 1.0f / s;
    const uint64_t base = uint64_t(r) * seg;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const uint32_t q = threadIdx.x + k * kBlock;
      if (q < nv4) st4(d, dt, base + 4ull * q, v4f_make(x.v[k].x * inv, x.v[k].y * inv, x.v[k].z * inv, x.v[k].w * inv));
    }
    if (r + 1 < r1) x = xn;
  }
}

VM_TILE void softmax_tiles(Args A, uint32_t ti, uint32_t lo, uint32_t hi) {
  A = uargs(A);
  const VM_K Task& t = task_of(A, ti);
  float* red = lds_f32();
  const uint32_t n_out = t.p[0], seg = t.p[1];
  const uint32_t dt = (t.tile_op >> 8) & 0xFF, adt = (t.tile_op >> 16) & 0xFF;
  hi = min(hi, n_out);
  if (lo >= hi) return;
  const gbyte* a = resolve(A, t.a);
  gbyte* d = resolve(A, t.dst);
  if (row_vec_ok(seg, a, d, adt, dt)) {
    const uint32_t nv4 = seg >> 2;
    if (nv4 <= 1 * kBlock) return softmax_rows_vec<1>(A, ti, lo, hi);
    if (nv4 <= 2 * kBlock) return softmax_rows_vec<2>(A, ti, lo, hi);
    if (nv4 <= 4 * kBlock) return softmax_rows_vec<4>(A, ti, lo, hi);
    return softmax_rows_vec<8>(A, ti, lo, hi);
  }
  for (uint32_t r = lo; r < hi; ++r) {
    const uint64_t base = uint64_t(r) * seg;
    float m = -INFINITY;
    for (uint32_t j = threadIdx.x; j < seg; j += kBlock) m = fmaxf(m, load_f(a, adt, base + j));
    m = block_reduce(m, OpMax(), red);
    float s = 0.0f;
    for (uint32_t j = threadIdx.x; j < seg; j += kBlock) s += __expf(load_f(a, adt, base + j) - m);
    s = block_reduce(s, OpSum(), red + kWaves);
    const float inv = 1.0f / s;
    for (uint32_t j = threadIdx.x; j < seg; j += kBlock) store_f(d, dt, base + j, __expf(load_f(a, adt, base + j) - m) * inv);
  }
}

// ARGMAX_SEG: dst = first index of the row maximum (a NaN wins: its first index),
// b = that value (a's dtype).  p0 n_out, p1 seg, p3 S: a row's elements split S
// ways (tile = row * S + split; S <= 1: one tile per row).  Each split finds its
// best (value, index); the split that arrives last at the row's counter in the
// task's scratch combines the S candidates (the order is total, so the result
// does not depend on which split is last) and resets the counter.  Candidates
// and counters are agent-scope atomics, which go to memory past the XCD's L2.
// Scratch (S > 1): [n_out * S] {value bits, index}, then n_out counters.
VM_DEV bool amax_better(float v, uint32_t i, float bv, uint32_t bi) {
  const bool vn = v != v, bn = bv != bv;
  if (vn != bn) return vn;
  if (vn) return i < bi;
  if (v != bv) return v > bv;
  return i < bi;
}

// Best (value, index) of elements [j0, j1) of a row over the block; the result
// is in sv[0] / si[0] (index 0xFFFFFFFF: no element).
VM_DEV void amax_block(const gbyte* a, uint32_t adt, uint64_t base, uint32_t j0, uint32_t j1, float* sv,
                       uint32_t* si) {
  float bv = -INFINITY;
  uint32_t bi = 0xFFFFFFFFu;
  auto take = [&](float v, uint32_t j) {
    if (bi == 0xFFFFFFFFu || amax_better(v, j, bv, bi)) {
      bv = v;
      bi = j;
    }
  };
  if (adt == DT_F32 && ((j0 | j1) & 3) == 0 && (((uintptr_t(a) + base * 4) & 15) == 0)) {
    // f32 rows (logits): 16-byte loads, 16 of them in flight per thread; each
    // thread still visits its elements in increasing index order
    const VM_G v4f* row = (const VM_G v4f*)(a + base * 4);
    const uint32_t q0b = j0 >> 2, n4 = j1 >> 2;
    constexpr int U = 16;
    for (uint32_t q0 = q0b + threadIdx.x; q0 < n4; q0 += U * kBlock) {
      v4f v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) v[u] = row[min(q0 + u * kBlock, n4 - 1)];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint32_t q = q0 + u * kBlock;
        if (q < n4) {
          take(v[u].x, 4 * q);
          take(v[u].y, 4 * q + 1);
          take(v[u].z, 4 * q + 2);
          take(v[u].w, 4 * q + 3);
        }
      }
    }
  } else {
    for (uint32_t j = j0 + threadIdx.x; j < j1; j += kBlock) take(load_f(a, adt, base + j), j);
  }
  lds_barrier();
  sv[threadIdx.x] = bv;
  si[threadIdx.x] = bi;
  lds_barrier();
  for (int s = kBlock / 2; s > 0; s >>= 1) {
    if (int(threadIdx.x) < s) {
      const float v2 = sv[threadIdx.x + s];
      const uint32_t i2 = si[threadIdx.x + s];
      if (i2 != 0xFFFFFFFFu && (si[threadIdx.x] == 0xFFFFFFFFu || amax_better(v2, i2, sv[threadIdx.x], si[threadIdx.x]))) {
        sv[threadIdx.x] = v2;
        si[threadIdx.x] = i2;
      }
    }
    lds_barrier();
  }
}

VM_DEV void amax_store(gbyte* di, gbyte* dv, uint32_t dt, uint32_t adt, uint32_t o, float v, uint32_t i) {
  const uint32_t idx = i == 0xFFFFFFFFu ? 0u : i;
  if (dt == DT_I64) gcast<int64_t>(di)[o] = idx;
  else gcast<uint32_t>(di)[o] = idx;
  store_f(dv, adt, o, i == 0xFFFFFFFFu ? -INFINITY : v);
}

VM_TILE void argmax_tiles(Args A, uint32_t ti, uint32_t lo, uint32_t hi) {
  A = uargs(A);
  const VM_K Task& t = task_of(A, ti);
  const uint32_t n_out = t.p[0], seg = t.p[1], S = max(1u, t.p[3]);
  const uint32_t dt = (t.tile_op >> 8) & 0xFF, adt = (t.tile_op >> 16) & 0xFF;
  const gbyte* a = resolve(A, t.a);
  gbyte* di = resolve(A, t.dst);
  gbyte* dv = resolve(A, t.b);
  float* sv = lds_f32();
  uint32_t* si = reinterpret_cast<uint32_t*>(sv + kBlock);
  uint32_t* flag = si + kBlock;
  // split length: whole 16-byte runs
  const uint32_t per = ((seg + S - 1) / S + 3) & ~3u;
  hi = min(hi, n_out * S);
  for (uint32_t tile = lo; tile < hi; ++tile) {
    const uint32_t o = tile / S, split = tile % S;
    const uint32_t j0 = min(split * per, seg), j1 = min(seg, j0 + per);
    amax_block(a, adt, uint64_t(o) * seg, j0, j1, sv, si);
    if (S == 1) {
      if (threadIdx.x == 0) amax_store(di, dv, dt, adt, o, sv[0], si[0]);
      continue;
    }
    uint32_t* sp = reinterpret_cast<uint32_t*>(A->scratch + A->task_scratch[ti]);
    uint32_t* arrivals = sp + 2ull * n_out * S;
    if (threadIdx.x == 0) {
      uint32_t* mine = sp + 2ull * (uint64_t(o) * S + split);
      __hip_atomic_store(mine, __float_as_uint(sv[0]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(mine + 1, si[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __builtin_amdgcn_s_waitcnt(0x0F70);             // vmcnt(0): the candidate is in memory
      // acquire-release at agent scope: publishes this split's candidate, and the
      // last arriver sees every other split's before it combines
      const uint32_t before = __hip_atomic_fetch_add(arrivals + o, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
      const bool last = before == S - 1;
      if (last) __hip_atomic_store(arrivals + o, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *flag = last;
    }
    lds_barrier();
    if (*flag) {
      // candidate k by thread k, then the same tree as above
      float bv = -INFINITY;
      uint32_t bi = 0xFFFFFFFFu;
      for (uint32_t k = threadIdx.x; k < S; k += kBlock) {
        const uint32_t* c = sp + 2ull * (uint64_t(o) * S + k);
        const float v = __uint_as_float(__hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        const uint32_t i = __hip_atomic_load(c + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (i != 0xFFFFFFFFu && (bi == 0xFFFFFFFFu || amax_better(v, i, bv, bi))) {
          bv = v;
          bi = i;
        }
      }
      sv[threadIdx.x] = bv;
      si[threadIdx.x] = bi;
      lds_barrier();
      for (int s = kBlock / 2; s > 0; s >>= 1) {
        if (int(threadIdx.x) < s) {
          const float v2 = sv[threadIdx.x + s];
          const uint32_t i2 = si[threadIdx.x + s];
          if (i2 != 0xFFFFFFFFu &&
              (si[threadIdx.x] == 0xFFFFFFFFu || amax_better(v2, i2, sv[threadIdx.x], si[threadIdx.x]))) {
            sv[threadIdx.x] = v2;
            si[threadIdx.x] = i2;
          }
        }
        lds_barrier();
      }
      if (threadIdx.x == 0) amax_store(di, dv, dt, adt, o, sv[0], si[0]);
    }
    lds_barrier();                                    // flag / sv reused by the next tile
  }
}

}  // namespace vm
