// Index-driven tile ops (ops/gather.cl, scatter.cl, iota.cl, dynslice.cl, region.cl):
//   TOP_GATHER        dst[i] = a[view(i)]                (strided view copy)
//   TOP_SCATTER       dst[view(i)] = a[i]                (concat / pad pieces)
//   TOP_IOTA_DIM      dst[i] = coordinate of i along one dimension
//   TOP_DYN_GATHER    dynamic_slice with runtime start scalars (clamped)
//   TOP_DYN_SCATTER   dynamic_update_slice (in place)
//   TOP_GATHER_INDEX  stablehlo.gather with a runtime index buffer
//   TOP_MAP_REGION    fused straight-line map chain
// All are EW-tiled: tile k covers elements [k*ew_ts, (k+1)*ew_ts).  Element moves
// are raw copies of the element width; index math is exact integer arithmetic.
#pragma once
#include "tile_ew.h"

namespace vm {

// Affine map {rank, dims[rank], strides[rank], off} evaluated incrementally: the
// division chain runs once per thread, then each grid-stride step of kBlock
// elements advances the coordinates with carries.
struct AffineWalk {
  int rank;
  int32_t dims[8];
  int32_t strides[8];
  int32_t coord[8];
  int64_t off;
  VM_DEV void init(const VM_K int32_t* aux, uint32_t x, uint64_t i) {
    rank = aux[x];
    int64_t rem = int64_t(i);
    off = aux[x + 1 + 2 * rank];
    for (int e = rank - 1; e >= 0; --e) {
      dims[e] = aux[x + 1 + e];
      strides[e] = aux[x + 1 + rank + e];
      const int32_t c = int32_t(rem % dims[e]);
      rem /= dims[e];
      coord[e] = c;
      off += int64_t(c) * strides[e];
    }
  }
  // advance by `step` elements (the new position stays inside the map)
  VM_DEV void advance(uint32_t step) {
    uint32_t carry = step;
    for (int e = rank - 1; e >= 0 && carry; --e) {
      const uint32_t dim = uint32_t(dims[e]);
      const uint32_t c = uint32_t(coord[e]) + carry;
      const uint32_t nc = c % dim;
      carry = c / dim;
      off += (int64_t(nc) - coord[e]) * strides[e];
      coord[e] = int32_t(nc);
    }
  }
};

// A view whose innermost axis is contiguous, with the innermost extent, every
// other stride and the offset whole multiples of 16 bytes, moves 16-byte runs:
// the same map over 16-byte units (innermost extent and strides divided by the
// elements per unit).  Four runs are loaded per thread before any is stored, so
// a thread keeps four loads in flight instead of one; a view that is one
// contiguous run (a slice of whole rows) skips the index walk altogether.
// Returns false when the view does not qualify (the element path runs).
VM_DEV bool gather_wide(const VM_K int32_t* aux, uint32_t x, gbyte* d, const gbyte* a, uint64_t e0,
                        uint64_t e1, uint32_t es, bool scatter) {
  const int rank = aux[x];
  if (rank < 1 || rank > 8 || es > 16 || 16 % es || ((uintptr_t(a) | uintptr_t(d)) & 15)) return false;
  const int64_t per = 16 / es;
  const int64_t off = aux[x + 1 + 2 * rank];
  if (aux[x + 2 * rank] != 1 || aux[x + rank] % per || off % per || off < 0) return false;
  bool linear = true;
  int64_t want = 1;
  for (int e = rank - 1; e >= 0; --e) {
    const int32_t dim = aux[x + 1 + e], st = aux[x + 1 + rank + e];
    if (e < rank - 1 && st % per) return false;
    if (dim != 1 && st != want) linear = false;
    want *= dim;
  }
  const uint64_t c0 = e0 / uint64_t(per), c1 = e1 / uint64_t(per);    // e0, e1: whole units (see caller)
  constexpr int U = 4;
  const uint32_t tid = threadIdx.x;
  if (linear) {
    const VM_G v4u* src = (const VM_G v4u*)(scatter ? a : a + off * es);
    VM_G v4u* dst = (VM_G v4u*)(scatter ? d + off * es : d);
    for (uint64_t c = c0 + tid; c < c1; c += U * kBlock) {
      v4u v[U];
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (c + u * kBlock < c1) v[u] = src[c + u * kBlock];
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (c + u * kBlock < c1) dst[c + u * kBlock] = v[u];
    }
    return true;
  }
  if (c0 + tid >= c1) return true;
  AffineWalk w;
  w.rank = rank;
  w.off = off / per;
  int64_t rem = int64_t(c0 + tid);
  for (int e = rank - 1; e >= 0; --e) {
    w.dims[e] = e == rank - 1 ? int32_t(aux[x + 1 + e] / per) : aux[x + 1 + e];
    w.strides[e] = e == rank - 1 ? 1 : int32_t(aux[x + 1 + rank + e] / per);
    const int32_t cc = int32_t(rem % w.dims[e]);
    rem /= w.dims[e];
    w.coord[e] = cc;
    w.off += int64_t(cc) * w.strides[e];
  }
  const VM_G v4u* src = (const VM_G v4u*)a;
  VM_G v4u* dst = (VM_G v4u*)d;
  for (uint64_t c = c0 + tid; c < c1; c += U * kBlock) {
    v4u v[U];
    int64_t o[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      o[u] = w.off;
      if (c + (u + 1) * kBlock < c1) w.advance(kBlock);
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (c + u * kBlock < c1) v[u] = scatter ? src[c + u * kBlock] : src[o[u]];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (c + u * kBlock < c1) {
        if (scatter) dst[o[u]] = v[u];
        else dst[c + u * kBlock] = v[u];
      }
  }
  return true;
}

// A view whose every stride is 0 (or whose dim is 1): one source element
// broadcast, as the lowering emits for a constant broadcast into a buffer (the
// decoder's zero-filled K/V caches).  One load, then 16-byte stores of the
// replicated bits; the element path took 126 us for a 960 KB cache.  Returns
// false when the view does not qualify.
VM_DEV bool gather_splat(const VM_K int32_t* aux, uint32_t x, gbyte* d, const gbyte* a, uint64_t e0, uint64_t e1,
                         uint32_t es) {
  const int rank = aux[x];
  if (rank < 0 || rank > 8 || 16 % es || (uintptr_t(d) & 15)) return false;
  for (int e = 0; e < rank; ++e)
    if (aux[x + 1 + rank + e] != 0 && aux[x + 1 + e] != 1) return false;
  const uint64_t per = 16 / es;
  if (e0 % per) return false;
  const int64_t off = aux[x + 1 + 2 * rank];
  uint32_t lo, hi;
  if (es == 8) {
    const uint64_t v = gcast<uint64_t>(a)[off];
    lo = uint32_t(v);
    hi = uint32_t(v >> 32);
  } else {
    lo = hi = es == 4 ? gcast<uint32_t>(a)[off] : es == 2 ? uint32_t(gcast<uint16_t>(a)[off]) * 0x00010001u
                                                         : uint32_t(a[off]) * 0x01010101u;
  }
  const v4u pat = v4u_make(lo, hi, lo, hi);
  const uint64_t c1 = e1 / per;
  VM_G v4u* dv = (VM_G v4u*)d;
  for (uint64_t c = e0 / per + threadIdx.x; c < c1; c += kBlock) dv[c] = pat;
  for (uint64_t i = c1 * per + threadIdx.x; i < e1; i += kBlock) copy_elem(d, i, a, uint64_t(off), es);
  return true;
}

VM_TILE void gather_tiles(Args A, uint32_t ti, uint32_t lo, uint32_t hi, bool scatter) {
  A = uargs(A);
  const VM_K Task& t = task_of(A, ti);
  const VM_K int32_t* aux = aux_of(A);
  const uint32_t n = t.p[1];
  const uint32_t dt = (t.tile_op >> 8) & 0xFF;
  const uint32_t es = dt_size(dt);
  const uint64_t e0 = uint64_t(lo) * A->ew_ts, e1 = min(uint64_t(hi) * A->ew_ts, uint64_t(n));
  if (e0 >= e1) return;
  gbyte* d = resolve(A, t.dst);
  const gbyte* a = resolve(A, t.a);
  const int rank = aux[t.p[0]];
  // e0 is a multiple of ew_ts (a multiple of 16), e1 too or the element count,
  // which a qualifying view makes a multiple of the elements per 16 bytes
  if (!scatter && gather_splat(aux, t.p[0], d, a, e0, e1, es)) return;
  if (gather_wide(aux, t.p[0], d, a, e0, e1, es, scatter)) return;
  if (rank > 8) {        // wide maps: direct evaluation per element
    for (uint64_t i = e0 + threadIdx.x; i < e1; i += kBlock) {
      const int64_t j = view_index(aux, t.p[0], i);
      if (scatter) copy_elem(d, uint64_t(j), a, i, es);
      else copy_elem(d, i, a, uint64_t(j), es);
    }
    return;
  }
  if (e0 + threadIdx.x >= e1) return;
  AffineWalk w;
  w.init(aux, t.p[0], e0 + threadIdx.x);
  for (uint64_t i = e0 + threadIdx.x; i < e1; i += kBlock) {
    if (scatter) copy_elem(d, uint64_t(w.off), a, i, es);
    else copy_elem(d, i, a, uint64_t(w.off), es);
    if (i + kBlock < e1) w.advance(kBlock);
  }
}

// aux at p0: {rank, dims[rank], dim}
VM_TILE void iota_tiles(Args A, uint32_t ti, uint32_t lo, uint32_t hi) {
  A = uargs(A);
  const VM_K Task& t = task_of(A, ti);
  const uint32_t n = t.p[1];
  const uint32_t dt = (t.tile_op >> 8) & 0xFF;
  const uint64_t e0 = uint64_t(lo) * A->ew_ts, e1 = min(uint64_t(hi) * A->ew_ts, uint64_t(n));
  const VM_K int32_t* x = aux_of(A) + t.p[0];
  const int rank = x[0];
  const int dim = x[1 + rank];
  uint64_t inner = 1;
  for (int e = dim + 1; e < rank; ++e) inner *= uint64_t(x[1 + e]);
  const uint64_t extent = uint64_t(x[1 + dim]);
  gbyte* d = resolve(A, t.dst);
  for (uint64_t i = e0 + threadIdx.x; i < e1; i += kBlock) {
    const uint64_t c = (i / inner) % extent;
    switch (dt) {
      case DT_I32: case DT_U32: gcast<uint32_t>(d)[i] = uint32_t(c); break;
      case DT_I64: gcast<int64_t>(d)[i] = int64_t(c); break;
      default: store_f(d, dt, i, float(c)); break;
    }
  }
}

// Runtime start offset of a dynamic slice: sum_d clamp(start_d, 0, cmax_d) * stride_d
// (dynslice.cl:1-56).  aux at p0: {rank, sizes, strides, cmax, start handles,
// start buffer ids, is64}; the start handles were patched at load.
VM_DEV int64_t dyn_base(Args A, uint32_t x) {
  const VM_K int32_t* w = aux_of(A) + x;
  const int rank = w[0];
  const bool is64 = w[1 + 5 * rank] != 0;
  int64_t base = 0;
  for (int e = 0; e < rank; ++e) {
    int64_t s = read_index(resolve(A, uint32_t(w[1 + 3 * rank + e])), is64);
    const int64_t cmax = w[1 + 2 * rank + e];
    s = s < 0 ? 0 : (s > cmax ? cmax : s);
    base += s * int64_t(w[1 + rank + e]);
  }
  return base;
}

VM_TILE void dyn_tiles(Args A, uint32_t ti, uint32_t lo, uint32_t hi, bool scatter) {
  A = uargs(A);
  const VM_K Task& t = task_of(A, ti);
  const uint32_t n = t.p[1];
  const uint32_t dt = (t.tile_op >> 8) & 0xFF;
  const uint32_t es = dt_size(dt);
  const uint64_t e0 = uint64_t(lo) * A->ew_ts, e1 = min(uint64_t(hi) * A->ew_ts, uint64_t(n));
  if (e0 >= e1) return;
  const int64_t base = dyn_base(A, t.p[0]);
  const VM_K int32_t* w = aux_of(A) + t.p[0];
  const int rank = w[0];
  gbyte* d = resolve(A, t.dst);
  const gbyte* a = resolve(A, t.a);
  // Row runs: the last dim has stride 1 in the large tensor, so a run of 16 bytes
  // of the small (contiguous) tensor is 16 contiguous bytes of the large one.
  // With whole 16-byte runs, aligned bases, strides and start, each thread copies
  // 16-byte chunks with the index math once per chunk in 32 bits (C5's prefill
  // K/V cache writes, [12, 512, 64] bf16: 50-65 us per task element by element).
  const int last = rank - 1;
  const uint32_t vec = es >= 2 && es <= 8 ? 16 / es : 0;
  bool runs = vec && rank >= 1 && w[1 + rank + last] == 1 && uint32_t(w[1 + last]) % vec == 0 && n < (1u << 31) &&
              base >= 0 && (base * es) % 16 == 0 && ((uintptr_t(a) | uintptr_t(d)) & 15) == 0;
  for (int e = 0; e < last; ++e) runs = runs && (int64_t(w[1 + rank + e]) * es) % 16 == 0;
  if (runs) {
    const uint32_t q1 = uint32_t(e1) / vec;               // e0, e1: whole runs (ew_ts % 64 == 0, n % w[last] == 0)
#pragma unroll 2
    for (uint32_t q = uint32_t(e0) / vec + threadIdx.x; q < q1; q += kBlock) {
      uint32_t rem = q * vec;
      int64_t off = base;
      for (int e = last; e >= 0; --e) {
        const uint32_t dim = uint32_t(w[1 + e]);
        off += int64_t(rem % dim) * int64_t(w[1 + rank + e]);
        rem /= dim;
      }
      if (scatter) *(VM_G v4u*)(d + uint64_t(off) * es) = *(const VM_G v4u*)(a + uint64_t(q) * 16);
      else *(VM_G v4u*)(d + uint64_t(q) * 16) = *(const VM_G v4u*)(a + uint64_t(off) * es);
    }
    return;
  }
  for (uint64_t i = e0 + threadIdx.x; i < e1; i += kBlock) {
    int64_t rem = int64_t(i), off = base;
    for (int e = rank - 1; e >= 0; --e) {
      const int64_t dim = w[1 + e];
      off += (rem % dim) * int64_t(w[1 + rank + e]);
      rem /= dim;
    }
    if (scatter) copy_elem(d, uint64_t(off), a, i, es);
    else copy_elem(d, i, a, uint64_t(off), es);
  }
}

// stablehlo.gather (gather.cl:108+): aux at p0 = {out_rank, nidx, si_vec_stride,
// is64, idx handle (patched), idx buffer id, out_dims[out_rank],
// operand_strides[out_rank], start_index_strides[out_rank],
// index_operand_strides[nidx], clamp_max[nidx]}.
VM_TILE void gather_index_tiles(Args A, uint32_t ti, uint32_t lo, uint32_t hi) {
  A = uargs(A);
  const VM_K Task& t = task_of(A, ti);
  const uint32_t n = t.p[1];
  const uint32_t dt = (t.tile_op >> 8) & 0xFF;
  const uint32_t es = dt_size(dt);
  const uint64_t e0 = uint64_t(lo) * A->ew_ts, e1 = min(uint64_t(hi) * A->ew_ts, uint64_t(n));
  if (e0 >= e1) return;
  const VM_K int32_t* w = aux_of(A) + t.p[0];
  const int out_rank = w[0], nidx = w[1];
  const int64_t vstride = w[2];
  const bool is64 = w[3] != 0;
  const gbyte* ib = resolve(A, uint32_t(w[4]));
  const VM_K int32_t* od = w + 6;
  const VM_K int32_t* ops = od + out_rank;
  const VM_K int32_t* sis = ops + out_rank;
  const VM_K int32_t* ios = sis + out_rank;
  const VM_K int32_t* cm = ios + nidx;
  gbyte* d = resolve(A, t.dst);
  const gbyte* a = resolve(A, t.a);
  // Row runs (take_rows, embedding lookups): along the last output dim the
  // operand offset steps by 1 and no index varies (ops[last] == 1, sis[last] ==
  // 0).  With whole 16-byte runs and 16-byte aligned bases and strides, each
  // thread copies 16-byte chunks, the index math once per chunk in 32 bits (C5's
  // prefill embedding, 512 rows of 768 bf16: 591 us element by element on the 3
  // lanes its phase gave it).
  const int last = out_rank - 1;
  const uint32_t vec = es >= 2 && es <= 8 ? 16 / es : 0;
  bool runs = vec && out_rank >= 1 && ops[last] == 1 && sis[last] == 0 && uint32_t(od[last]) % vec == 0 &&
              n < (1u << 31) && ((uintptr_t(a) | uintptr_t(d)) & 15) == 0;
  for (int e = 0; e < last; ++e) runs = runs && (int64_t(ops[e]) * es) % 16 == 0;
  for (int k = 0; k < nidx; ++k) runs = runs && (int64_t(ios[k]) * es) % 16 == 0;
  if (runs) {
    const uint32_t q1 = uint32_t(e1) / vec;               // e0, e1: whole runs (ew_ts % 64 == 0, n % od[last] == 0)
#pragma unroll 2
    for (uint32_t q = uint32_t(e0) / vec + threadIdx.x; q < q1; q += kBlock) {
      uint32_t rem = q * vec;
      int64_t off = 0, si = 0;
      for (int e = last; e >= 0; --e) {
        const uint32_t c = rem % uint32_t(od[e]);
        rem /= uint32_t(od[e]);
        off += int64_t(c) * ops[e];
        si += int64_t(c) * sis[e];
      }
      for (int k = 0; k < nidx; ++k) {
        const uint64_t qi = uint64_t(si + k * vstride);
        int64_t sx = is64 ? gcast<int64_t>(ib)[qi] : int64_t(gcast<int32_t>(ib)[qi]);
        sx = sx < 0 ? 0 : (sx > cm[k] ? int64_t(cm[k]) : sx);
        off += sx * ios[k];
      }
      *(VM_G v4u*)(d + uint64_t(q) * 16) = *(const VM_G v4u*)(a + uint64_t(off) * es);
    }
    return;
  }
  for (uint64_t i = e0 + threadIdx.x; i < e1; i += kBlock) {
    int64_t rem = int64_t(i), off = 0, si = 0;
    for (int e = out_rank - 1; e >= 0; --e) {
      const int64_t c = rem % od[e];
      rem /= od[e];
      off += c * ops[e];
      si += c * sis[e];
    }
    for (int k = 0; k < nidx; ++k) {
      const uint64_t q = uint64_t(si + k * vstride);
      int64_t s = is64 ? gcast<int64_t>(ib)[q] : int64_t(gcast<int32_t>(ib)[q]);
      s = s < 0 ? 0 : (s > cm[k] ? int64_t(cm[k]) : s);
      off += s * ios[k];
    }
    copy_elem(d, i, a, uint64_t(off), es);
  }
}

// TOP_MAP_REGION (region.cl:43-98): straight-line micro-program over per-element
// slots.  aux at p0 = {n_in, out_slot, n_micro, in_slot[n_in],
// n_micro x {kind, dst, a, b, s_bits, t_bits}}; inputs in a, b, p2..p7.
VM_TILE void map_region_tiles(Args A, uint32_t ti, uint32_t lo, uint32_t hi) {
  A = uargs(A);
  const VM_K Task& t = task_of(A, ti);
  const uint32_t n = t.p[1];
  const uint32_t dt = (t.tile_op >> 8) & 0xFF;
  const uint64_t e0 = uint64_t(lo) * A->ew_ts, e1 = min(uint64_t(hi) * A->ew_ts, uint64_t(n));
  if (e0 >= e1) return;
  const VM_K int32_t* w = aux_of(A) + t.p[0];
  const int n_in = w[0], out_slot = w[1], n_micro = w[2];
  const uint32_t handles[8] = {t.a, t.b, t.p[2], t.p[3], t.p[4], t.p[5], t.p[6], t.p[7]};
  gbyte* d = resolve(A, t.dst);
  const VM_K int32_t* prog = w + 3 + n_in;
  for (uint64_t i = e0 + threadIdx.x; i < e1; i += kBlock) {
    float R[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) R[k] = 0.0f;
    for (int k = 0; k < n_in; ++k) R[w[3 + k] & 15] = load_f(resolve(A, handles[k]), dt, i);
    for (int m = 0; m < n_micro; ++m) {
      const VM_K int32_t* u = prog + 6 * m;
      const float x = R[u[2] & 15], y = R[u[3] & 15];
      R[u[1] & 15] = micro(uint32_t(u[0]), x, y, __int_as_float(u[4]), __int_as_float(u[5]));
    }
    store_f(d, dt, i, R[out_slot & 15]);
  }
}

}  // namespace vm
