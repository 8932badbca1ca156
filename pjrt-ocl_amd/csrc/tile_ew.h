// TOP_EW: elementwise tile op over an entry's tile range (ops/ew.cl semantics).
// Task fields: p0 subop, p1 n, p2 cmp pred / fill bits / affine s / a-view+1,
// p3 affine t / b-view+1 / select predicate handle.
//
// An entry's tiles [lo, hi) are one contiguous element range, so the op streams
// the whole range with 128-bit loads (v4f for f32, 8 x 16-bit for bf16/f16),
// several loads in flight per thread, instead of tile by tile.
#pragma once
#include "vm_divu32.h"
#include "vm_math.h"

namespace vm {

constexpr int kEwUnroll = 4;

// Compile-time operation of the vector paths.
template <uint32_t SUB>
struct EwOp {
  static constexpr bool kBin = (SUB <= SUB_POW) || (SUB >= SUB_ATAN2 && SUB <= SUB_REMAINDER);
  float s, t;
  VM_DEV float operator()(float x, float y) const {
    if constexpr (SUB == SUB_AFFINE) return fmaf(x, s, t);
    else if constexpr (SUB == SUB_FILL) return s;
    else if constexpr (kBin) return ew_bin(SUB, x, y);
    else return ew_un(SUB, x);
  }
};

// f32 contiguous range [e0, e1): v4f body, scalar tail.
template <uint32_t SUB>
VM_DEV void ew_f32_range(gbyte* dp, const gbyte* ap, const gbyte* bp, uint64_t e0, uint64_t e1, float s,
                          float t) {
  dp = uni_ptr(dp);
  ap = uni_ptr(ap);
  bp = uni_ptr(bp);
  const EwOp<SUB> op{s, t};
  VM_G float* d = gcast<float>(dp);
  const VM_G float* a = gcast<float>(ap);
  const VM_G float* b = gcast<float>(bp);
  const uint64_t nv = (e1 - e0) >> 2;
  const VM_G v4f* a4 = (const VM_G v4f*)(a + e0);
  const VM_G v4f* b4 = (const VM_G v4f*)(b + e0);
  VM_G v4f* d4 = (VM_G v4f*)(d + e0);
  for (uint64_t j = threadIdx.x; j < nv; j += uint64_t(kBlock) * kEwUnroll) {
    v4f x[kEwUnroll], y[kEwUnroll];
#pragma unroll
    for (int k = 0; k < kEwUnroll; ++k) {
      const uint64_t q = j + uint64_t(k) * kBlock;
      if (q < nv) {
        if constexpr (SUB != SUB_FILL) x[k] = a4[q];
        if constexpr (EwOp<SUB>::kBin) y[k] = b4[q];
      }
    }
#pragma unroll
    for (int k = 0; k < kEwUnroll; ++k) {
      const uint64_t q = j + uint64_t(k) * kBlock;
      if (q < nv) {
        v4f r;
        r.x = op(x[k].x, y[k].x);
        r.y = op(x[k].y, y[k].y);
        r.z = op(x[k].z, y[k].z);
        r.w = op(x[k].w, y[k].w);
        d4[q] = r;
      }
    }
  }
  for (uint64_t i = e0 + (nv << 2) + threadIdx.x; i < e1; i += kBlock) {
    const float x = SUB == SUB_FILL ? 0.0f : a[i];
    const float y = EwOp<SUB>::kBin ? b[i] : 0.0f;
    d[i] = op(x, y);
  }
}

// 16-bit float formats: 8 elements per 128-bit access, f32 arithmetic.
template <bool BF16>
VM_DEV float h2f(uint32_t h) { return BF16 ? bf16_to_f32(uint16_t(h)) : f16_to_f32(uint16_t(h)); }
template <bool BF16>
VM_DEV uint32_t f2h(float f) { return BF16 ? f32_to_bf16(f) : f32_to_f16(f); }

template <uint32_t SUB, bool BF16>
VM_DEV void ew_h16_range(gbyte* dp, const gbyte* ap, const gbyte* bp, uint64_t e0, uint64_t e1, float s,
                          float t) {
  dp = uni_ptr(dp);
  ap = uni_ptr(ap);
  bp = uni_ptr(bp);
  const EwOp<SUB> op{s, t};
  VM_G uint16_t* d = gcast<uint16_t>(dp);
  const VM_G uint16_t* a = gcast<uint16_t>(ap);
  const VM_G uint16_t* b = gcast<uint16_t>(bp);
  const uint64_t nv = (e1 - e0) >> 3;
  const VM_G v4u* a8 = (const VM_G v4u*)(a + e0);
  const VM_G v4u* b8 = (const VM_G v4u*)(b + e0);
  VM_G v4u* d8 = (VM_G v4u*)(d + e0);
  for (uint64_t j = threadIdx.x; j < nv; j += uint64_t(kBlock) * 2) {
    v4u x[2], y[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const uint64_t q = j + uint64_t(k) * kBlock;
      if (q < nv) {
        if constexpr (SUB != SUB_FILL) x[k] = a8[q];
        if constexpr (EwOp<SUB>::kBin) y[k] = b8[q];
      }
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const uint64_t q = j + uint64_t(k) * kBlock;
      if (q < nv) {
        const uint32_t xs[4] = {x[k].x, x[k].y, x[k].z, x[k].w};
        const uint32_t ys[4] = {y[k].x, y[k].y, y[k].z, y[k].w};
        uint32_t rs[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const float lo = op(h2f<BF16>(xs[w] & 0xFFFF), h2f<BF16>(ys[w] & 0xFFFF));
          const float hi = op(h2f<BF16>(xs[w] >> 16), h2f<BF16>(ys[w] >> 16));
          rs[w] = f2h<BF16>(lo) | (f2h<BF16>(hi) << 16);
        }
        d8[q] = v4u_make(rs[0], rs[1], rs[2], rs[3]);
      }
    }
  }
  for (uint64_t i = e0 + (nv << 3) + threadIdx.x; i < e1; i += kBlock) {
    const float x = SUB == SUB_FILL ? 0.0f : h2f<BF16>(a[i]);
    const float y = EwOp<SUB>::kBin ? h2f<BF16>(b[i]) : 0.0f;
    d[i] = uint16_t(f2h<BF16>(op(x, y)));
  }
}

// Subops with a 128-bit streaming specialisation; the rest (pow, atan2, fmod and
// the libm-heavy unaries) take the scalar path.
#define VM_EW_FAST_SUBS(X)                                                                      \
  X(SUB_ADD) X(SUB_MUL) X(SUB_SUB) X(SUB_DIV) X(SUB_MAX) X(SUB_MIN) X(SUB_COPY) X(SUB_NEG)      \
  X(SUB_EXP) X(SUB_LOG) X(SUB_SQRT) X(SUB_RSQRT) X(SUB_TANH) X(SUB_ABS) X(SUB_GELU)             \
  X(SUB_AFFINE) X(SUB_FILL)

// Strided view index (the reference's vmo_view_idx, ew.cl:174-185): element i of
// a view {rank, dims[rank], strides[rank], src_off} -> flat source index.
// Below 2^32 (every element index a tensor of this runtime holds) the
// quotients and remainders are taken in 32 bits: a 64-bit division is a long
// software sequence, and with two viewed operands of rank 3 it made an
// elementwise tile of 4096 elements cost 20-45 us (C5 prefill's broadcast bias
// adds and the attention output's transposed read).
VM_DEV int64_t view_index(const VM_K int32_t* aux, uint32_t off, uint64_t i) {
  const VM_K int32_t* x = aux + off;
  const int rank = x[0];
  int64_t o = x[1 + 2 * rank];
  if (i <= 0xFFFFFFFFull) {
    uint32_t rem = uint32_t(i);
    for (int e = rank - 1; e >= 0; --e) {
      const uint32_t dim = uint32_t(x[1 + e]);              // dims are positive
      o += int64_t(rem % dim) * int64_t(x[1 + rank + e]);
      rem /= dim;
    }
    return o;
  }
  int64_t rem = int64_t(i);
  for (int e = rank - 1; e >= 0; --e) {
    const int64_t dim = x[1 + e];
    o += (rem % dim) * int64_t(x[1 + rank + e]);
    rem /= dim;
  }
  return o;
}

// The view map decoded once per tile for views of rank <= kViewRank: dims
// innermost first, each with its invariant divisor, so the descriptor is not
// re-read from memory per element.  rank < 0: no view.
constexpr int kViewRank = 4;
struct ViewMap {
  int rank;
  int64_t off;
  DivU32 dim[kViewRank];
  int32_t stride[kViewRank];
};
VM_DEV ViewMap view_map(const VM_K int32_t* aux, uint32_t vo) {   // vo: view operand (aux offset + 1, 0 = none)
  ViewMap v;
  v.rank = -1;
  v.off = 0;
  if (vo == 0) return v;
  const VM_K int32_t* x = aux + (vo - 1);
  v.rank = int(uni(x[0]));
  if (v.rank > kViewRank) return v;
  v.off = x[1 + 2 * v.rank];
#pragma unroll
  for (int k = 0; k < kViewRank; ++k) {
    const int e = v.rank - 1 - k;
    v.dim[k] = k < v.rank ? div_u32(uint32_t(x[1 + e])) : DivU32{1u, 1u, 0u, 0u};   // dims are positive
    v.stride[k] = k < v.rank ? x[1 + v.rank + e] : 0;
  }
  return v;
}
// Source index of element i (< 2^32) through a decoded map.
VM_DEV uint64_t view_at(const ViewMap& v, const VM_K int32_t* aux, uint32_t vo, uint32_t i) {
  if (v.rank < 0) return i;
  if (v.rank > kViewRank) return uint64_t(view_index(aux, vo - 1, i));
  int64_t o = v.off;
  uint32_t rem = i;
#pragma unroll
  for (int k = 0; k < kViewRank; ++k) {
    if (k < v.rank) {
      const uint32_t q = v.dim[k].quo(rem);
      o += int64_t(rem - q * v.dim[k].d) * v.stride[k];
      rem = q;
    }
  }
  return uint64_t(o);
}

// A view that reads src[off + i % P]: leading dims broadcast (stride 0), the
// trailing ones contiguous row-major -- a bias row added to every row of a
// matrix and the like.  ok: no view (index i) or such a view with P and off
// multiples of 4, so four consecutive elements are one 16-byte access.  p.d = 0
// where no index of the range [0, e1) wraps (no view, or P >= e1).
struct PeriodicView {
  bool ok;
  uint32_t off;
  DivU32 p;
  VM_DEV uint32_t at(uint32_t i) const { return off + (p.d ? i - p.quo(i) * p.d : i); }
};
VM_DEV PeriodicView periodic_view(const VM_K int32_t* aux, uint32_t vo, uint64_t e1) {
  PeriodicView v{vo == 0, 0u, DivU32{0u, 0u, 0u, 0u}};
  if (vo == 0) return v;
  const VM_K int32_t* x = aux + (vo - 1);
  const int rank = int(uni(x[0]));
  uint64_t p = 1;
  int k = rank - 1;
  for (; k >= 0 && (x[1 + k] == 1 || int64_t(x[1 + rank + k]) == int64_t(p)); --k) p *= uint64_t(x[1 + k]);
  for (; k >= 0; --k)
    if (x[1 + k] != 1 && x[1 + rank + k] != 0) return v;
  const int64_t off = x[1 + 2 * rank];
  if (p % 4 != 0 || p > 0xFFFFFFFFull || off < 0 || off % 4 != 0 || off > 0xFFFFFFFFll) return v;
  v.ok = true;
  v.off = uint32_t(off);
  if (p < e1) v.p = div_u32(uint32_t(p));
  return v;
}

// f32 binary op over [e0, e1) with each operand contiguous or a periodic view:
// v4f body (P and off multiples of 4, e0 too), scalar tail.
template <uint32_t SUB>
VM_DEV void ew_f32_periodic(gbyte* dp, const gbyte* ap, const gbyte* bp, uint32_t e0, uint32_t e1,
                            const PeriodicView& va, const PeriodicView& vb) {
  const EwOp<SUB> op{0.0f, 0.0f};
  VM_G float* d = gcast<float>(uni_ptr(dp));
  const VM_G float* a = gcast<float>(uni_ptr(ap));
  const VM_G float* b = gcast<float>(uni_ptr(bp));
  const uint32_t nv = (e1 - e0) >> 2;
  for (uint32_t j = threadIdx.x; j < nv; j += kBlock * kEwUnroll) {
    v4f x[kEwUnroll], y[kEwUnroll];
#pragma unroll
    for (int k = 0; k < kEwUnroll; ++k) {
      const uint32_t q = j + k * kBlock, i = e0 + 4 * q;
      if (q < nv) {
        x[k] = *(const VM_G v4f*)(a + va.at(i));
        y[k] = *(const VM_G v4f*)(b + vb.at(i));
      }
    }
#pragma unroll
    for (int k = 0; k < kEwUnroll; ++k) {
      const uint32_t q = j + k * kBlock;
      if (q < nv)
        *(VM_G v4f*)(d + e0 + 4 * q) = v4f_make(op(x[k].x, y[k].x), op(x[k].y, y[k].y), op(x[k].z, y[k].z),
                                                op(x[k].w, y[k].w));
    }
  }
  for (uint32_t i = e0 + (nv << 2) + threadIdx.x; i < e1; i += kBlock) d[i] = op(a[va.at(i)], b[vb.at(i)]);
}

// ---- integer / bool / f64 scalar paths ------------------------------------------------
template <typename T, typename U>
VM_DEV T int_op(uint32_t sub, T x, T y, bool is_unsigned) {
  constexpr int kBits = sizeof(T) * 8;
  switch (sub) {
    case SUB_ADD: return T(U(x) + U(y));
    case SUB_MUL: return T(U(x) * U(y));
    case SUB_SUB: return T(U(x) - U(y));
    case SUB_DIV:
      if (y == 0) return 0;
      if (is_unsigned) return T(U(x) / U(y));
      if (y == T(-1)) return T(U(0) - U(x));   // INT_MIN / -1 wraps
      return x / y;
    case SUB_MAX: return is_unsigned ? (U(x) > U(y) ? x : y) : (x > y ? x : y);
    case SUB_MIN: return is_unsigned ? (U(x) < U(y) ? x : y) : (x < y ? x : y);
    case SUB_COPY: return x;
    case SUB_NEG: return T(U(0) - U(x));
    case SUB_ABS: return is_unsigned ? x : (x < 0 ? T(U(0) - U(x)) : x);
    case SUB_SIGN: return is_unsigned ? T(x != 0) : T((x > 0) - (x < 0));
    case SUB_AND: return x & y;
    case SUB_OR: return x | y;
    case SUB_XOR: return x ^ y;
    case SUB_NOT: return ~x;
    case SUB_SHL: return T(U(x) << (U(y) & U(kBits - 1)));
    case SUB_SHR_L: return T(U(x) >> (U(y) & U(kBits - 1)));
    case SUB_SHR_A: return x >> (U(y) & U(kBits - 1));
    default: return x;
  }
}

VM_DEV double f64_op(uint32_t sub, double x, double y) {
  switch (sub) {
    case SUB_ADD: return x + y;
    case SUB_MUL: return x * y;
    case SUB_SUB: return x - y;
    case SUB_DIV: return x / y;
    case SUB_MAX: return fmax(x, y);
    case SUB_MIN: return fmin(x, y);
    case SUB_POW: return pow(x, y);
    case SUB_ATAN2: return atan2(x, y);
    case SUB_REMAINDER: return fmod(x, y);
    case SUB_COPY: return x;
    case SUB_NEG: return -x;
    case SUB_EXP: return exp(x);
    case SUB_LOG: return log(x);
    case SUB_SQRT: return sqrt(x);
    case SUB_RSQRT: return 1.0 / sqrt(x);
    case SUB_TANH: return tanh(x);
    case SUB_ABS: return fabs(x);
    case SUB_FLOOR: return floor(x);
    case SUB_CEIL: return ceil(x);
    case SUB_SIGN: return x > 0.0 ? 1.0 : (x < 0.0 ? -1.0 : x);
    case SUB_LOG1P: return log1p(x);
    case SUB_EXPM1: return expm1(x);
    case SUB_CBRT: return cbrt(x);
    case SUB_SIN: return sin(x);
    case SUB_COS: return cos(x);
    case SUB_TAN: return tan(x);
    case SUB_RINT: return rint(x);
    case SUB_ROUND: return round(x);
    case SUB_GELU: return 0.5 * x * (1.0 + tanh(0.7978845608 * (x + 0.044715 * x * x * x)));
    default: return x;
  }
}

template <typename T>
VM_DEV bool cmp_pred(uint32_t p, T x, T y) {
  switch (p) {
    case 0: return x == y;
    case 1: return x != y;
    case 2: return x < y;
    case 3: return x <= y;
    case 4: return x > y;
    default: return x >= y;
  }
}

// Numeric conversion (ew.cl:532-588): integer <-> integer through 64 bits keeping
// the low bits; otherwise through double, with float -> int saturating and NaN -> 0
// (XLA's convert semantics), bool = (v != 0).
VM_DEV float quiet_nan(float v) { return v != v ? __uint_as_float(__float_as_uint(v) | 0x400000u) : v; }

VM_DEV void convert_elem(const gbyte* a, uint32_t adt, gbyte* d, uint32_t dt, uint64_t i) {
  const bool a_int = adt == DT_I32 || adt == DT_U32 || adt == DT_I64 || adt == DT_BOOL;
  const bool d_int = dt == DT_I32 || dt == DT_U32 || dt == DT_I64;
  if (a_int && d_int) {
    const int64_t v = adt == DT_I64 ? gcast<int64_t>(a)[i]
                    : adt == DT_U32 ? int64_t(gcast<uint32_t>(a)[i])
                    : adt == DT_BOOL ? int64_t(a[i])
                    : int64_t(gcast<int32_t>(a)[i]);
    if (dt == DT_I64) gcast<int64_t>(d)[i] = v;
    else gcast<uint32_t>(d)[i] = uint32_t(uint64_t(v));
    return;
  }
  double v;
  switch (adt) {
    case DT_I32: v = double(gcast<int32_t>(a)[i]); break;
    case DT_U32: v = double(gcast<uint32_t>(a)[i]); break;
    case DT_BOOL: v = double(a[i]); break;
    case DT_I64: v = double(gcast<int64_t>(a)[i]); break;
    case DT_F64: v = gcast<double>(a)[i]; break;
    case DT_F16: v = double(f16_to_f32(gcast<uint16_t>(a)[i])); break;
    case DT_BF16: v = double(bf16_to_f32(gcast<uint16_t>(a)[i])); break;
    default: v = double(gcast<float>(a)[i]); break;
  }
  const double tv = trunc(v);
  switch (dt) {
    case DT_I32:
      gcast<int32_t>(d)[i] = (v != v) ? 0 : tv >= 2147483648.0 ? 2147483647
                           : tv < -2147483648.0 ? int32_t(-2147483647 - 1) : int32_t(tv);
      break;
    case DT_U32:
      gcast<uint32_t>(d)[i] = (v != v || tv <= 0.0) ? 0u : tv >= 4294967296.0 ? 0xFFFFFFFFu : uint32_t(tv);
      break;
    case DT_I64:
      gcast<int64_t>(d)[i] = (v != v) ? 0 : tv >= 9223372036854775808.0 ? INT64_MAX
                           : tv < -9223372036854775808.0 ? INT64_MIN : int64_t(tv);
      break;
    case DT_BOOL: d[i] = v != 0.0; break;
    case DT_F64: gcast<double>(d)[i] = v; break;
    case DT_F16: gcast<uint16_t>(d)[i] = f32_to_f16(float(v)); break;
    case DT_BF16: gcast<uint16_t>(d)[i] = f32_to_bf16(float(v)); break;
    default: gcast<float>(d)[i] = float(v); break;
  }
}

VM_DEV void copy_elem(gbyte* d, uint64_t di, const gbyte* s, uint64_t si, uint32_t es) {
  switch (es) {
    case 1: d[di] = s[si]; break;
    case 2: gcast<uint16_t>(d)[di] = gcast<uint16_t>(s)[si]; break;
    case 8: gcast<uint64_t>(d)[di] = gcast<uint64_t>(s)[si]; break;
    default: gcast<uint32_t>(d)[di] = gcast<uint32_t>(s)[si]; break;
  }
}

// Compare, select, convert, bitcast, is_finite, LTS: mixed-dtype subops.
VM_DEV void ew_special(Args A, uint32_t ti, uint64_t e0, uint64_t e1) {
  A = uargs(A);
  const VM_K Task& t = task_of(A, ti);
  const uint32_t sub = uni(t.p[0]);
  const uint32_t dt = uni((t.tile_op >> 8) & 0xFF), adt = uni((t.tile_op >> 16) & 0xFF);
  gbyte* d = resolve(A, t.dst);
  const gbyte* a = resolve(A, t.a);
  const gbyte* b = resolve(A, t.b);
  const uint32_t tid = threadIdx.x;
  switch (sub) {
    case SUB_CMP: {
      const uint32_t p = uni(t.p[2]);
      for (uint64_t i = e0 + tid; i < e1; i += kBlock) {
        bool r;
        switch (adt) {
          case DT_I32: r = cmp_pred(p, gcast<int32_t>(a)[i], gcast<int32_t>(b)[i]); break;
          case DT_U32: r = cmp_pred(p, gcast<uint32_t>(a)[i], gcast<uint32_t>(b)[i]); break;
          case DT_I64: r = cmp_pred(p, gcast<int64_t>(a)[i], gcast<int64_t>(b)[i]); break;
          case DT_BOOL: r = cmp_pred(p, uint32_t(a[i]), uint32_t(b[i])); break;
          case DT_F64: r = cmp_pred(p, gcast<double>(a)[i], gcast<double>(b)[i]); break;
          default: r = cmp_pred(p, load_f(a, adt, i), load_f(b, adt, i)); break;
        }
        d[i] = r;
      }
      return;
    }
    case SUB_SELECT: {
      const gbyte* pr = resolve(A, t.p[3]);
      const uint32_t es = dt_size(dt);
      for (uint64_t i = e0 + tid; i < e1; i += kBlock) copy_elem(d, i, pr[i] ? a : b, i, es);
      return;
    }
    case SUB_CONVERT:
      // f32 / bf16 / f16 to one another: four elements a step through ld4 / st4,
      // four steps' loads issued before the first store (one element a step, each
      // waiting on its own load, a tile of 4096 cost 9-10 us).  The reference
      // converts through a double (ew.cl:556-576), which sets a signalling NaN's
      // quiet bit and keeps its payload; the widening here is exact, so the quiet
      // bit is set explicitly.
      if ((adt == DT_F32 || adt == DT_BF16 || adt == DT_F16) && (dt == DT_F32 || dt == DT_BF16 || dt == DT_F16) &&
          (e0 & 3) == 0 && ((uintptr_t(a) | uintptr_t(d)) & 15) == 0) {
        constexpr uint32_t U = 4;
        const uint64_t q1 = e1 >> 2;
        for (uint64_t q = (e0 >> 2) + tid; q < q1; q += U * kBlock) {
          v4f x[U];
#pragma unroll
          for (uint32_t k = 0; k < U; ++k)
            if (q + k * kBlock < q1) x[k] = ld4(a, adt, 4 * (q + k * kBlock));
#pragma unroll
          for (uint32_t k = 0; k < U; ++k)
            if (q + k * kBlock < q1)
              st4(d, dt, 4 * (q + k * kBlock), v4f_make(quiet_nan(x[k].x), quiet_nan(x[k].y),
                                                        quiet_nan(x[k].z), quiet_nan(x[k].w)));
        }
        for (uint64_t i = (q1 << 2) + tid; i < e1; i += kBlock) convert_elem(a, adt, d, dt, i);
        return;
      }
      for (uint64_t i = e0 + tid; i < e1; i += kBlock) convert_elem(a, adt, d, dt, i);
      return;
    case SUB_BITCAST: {
      const uint32_t es = dt_size(dt);
      for (uint64_t i = e0 + tid; i < e1; i += kBlock) copy_elem(d, i, a, i, es);
      return;
    }
    case SUB_ISFINITE:
      for (uint64_t i = e0 + tid; i < e1; i += kBlock)
        d[i] = adt == DT_F64 ? isfinite(gcast<double>(a)[i]) : isfinite(load_f(a, adt, i));
      return;
    case SUB_LTS:   // scalar a[0] < b[0] -> 1 / 0 (one element)
      if (e0 == 0 && tid == 0) store_f(d, dt, 0, load_f(a, adt, 0) < load_f(b, adt, 0) ? 1.0f : 0.0f);
      return;
    default: return;
  }
}

// Integer, bool and f64 elementwise.
VM_DEV void ew_intlike(Args A, uint32_t ti, uint64_t e0, uint64_t e1) {
  A = uargs(A);
  const VM_K Task& t = task_of(A, ti);
  const uint32_t sub = uni(t.p[0]), dt = uni((t.tile_op >> 8) & 0xFF);
  gbyte* d = resolve(A, t.dst);
  const gbyte* a = resolve(A, t.a);
  const gbyte* b = resolve(A, t.b);
  const uint32_t tid = threadIdx.x;
  if (dt == DT_I32 || dt == DT_U32) {
    const bool u = dt == DT_U32;
    for (uint64_t i = e0 + tid; i < e1; i += kBlock) {
      int32_t r;
      if (sub == SUB_FILL) r = int32_t(t.p[2]);
      else if (sub == SUB_IOTA_FLAT) r = int32_t(i);
      else r = int_op<int32_t, uint32_t>(sub, gcast<int32_t>(a)[i], gcast<int32_t>(b)[i], u);
      gcast<int32_t>(d)[i] = r;
    }
  } else if (dt == DT_I64) {
    for (uint64_t i = e0 + tid; i < e1; i += kBlock) {
      int64_t r;
      if (sub == SUB_FILL) r = int64_t(int32_t(t.p[2]));
      else if (sub == SUB_IOTA_FLAT) r = int64_t(i);
      else r = int_op<int64_t, uint64_t>(sub, gcast<int64_t>(a)[i], gcast<int64_t>(b)[i], false);
      gcast<int64_t>(d)[i] = r;
    }
  } else if (dt == DT_BOOL) {
    for (uint64_t i = e0 + tid; i < e1; i += kBlock) {
      const uint8_t x = a[i] != 0, y = b[i] != 0;
      uint8_t r;
      switch (sub) {
        case SUB_FILL: r = t.p[2] != 0; break;
        case SUB_NOT: r = !x; break;
        case SUB_AND: r = x & y; break;
        case SUB_OR: r = x | y; break;
        case SUB_XOR: r = x ^ y; break;
        default: r = a[i]; break;
      }
      d[i] = r;
    }
  } else {   // f64
    for (uint64_t i = e0 + tid; i < e1; i += kBlock) {
      double r;
      if (sub == SUB_FILL) r = double(__uint_as_float(t.p[2]));
      else if (sub == SUB_IOTA_FLAT) r = double(i);
      else r = f64_op(sub, gcast<double>(a)[i], is_bin(sub) ? gcast<double>(b)[i] : 0.0);
      gcast<double>(d)[i] = r;
    }
  }
}

// f32 / f16 / bf16 scalar path: folded views, misalignment, libm-heavy subops.
VM_DEV void ew_float_scalar(Args A, uint32_t ti, uint64_t e0, uint64_t e1) {
  A = uargs(A);
  const VM_K Task& t = task_of(A, ti);
  const uint32_t sub = uni(t.p[0]), dt = uni((t.tile_op >> 8) & 0xFF);
  gbyte* d = resolve(A, t.dst);
  const gbyte* a = resolve(A, t.a);
  const gbyte* b = resolve(A, t.b);
  const float s = __uint_as_float(t.p[2]), tt = __uint_as_float(t.p[3]);
  const bool viewable = is_bin(sub) || is_un(sub);
  const uint32_t av = viewable ? t.p[2] : 0u, bv = viewable ? t.p[3] : 0u;
  const VM_K int32_t* aux = aux_of(A);
  const bool ld_a = sub != SUB_IOTA_FLAT && sub != SUB_FILL, ld_b = is_bin(sub);
  const ViewMap va = view_map(aux, av), vb = view_map(aux, bv);   // e1 <= n < 2^32
  // four elements a step: their (viewed) loads are issued before the first result
  // is computed, the result code itself stays rolled (libm-heavy subops)
  constexpr uint32_t U = 4;
  for (uint64_t i0 = e0 + threadIdx.x; i0 < e1; i0 += U * kBlock) {
    float xa[U], xb[U];
#pragma unroll
    for (uint32_t k = 0; k < U; ++k) {
      const uint64_t i = i0 + k * kBlock;
      xa[k] = xb[k] = 0.0f;
      if (i < e1 && ld_a) {
        xa[k] = load_f(a, dt, view_at(va, aux, av, uint32_t(i)));
        if (ld_b) xb[k] = load_f(b, dt, view_at(vb, aux, bv, uint32_t(i)));
      }
    }
#pragma unroll 1
    for (uint32_t k = 0; k < U; ++k) {
      const uint64_t i = i0 + k * kBlock;
      if (i >= e1) break;
      const float x = k == 0 ? xa[0] : k == 1 ? xa[1] : k == 2 ? xa[2] : xa[3];
      float r;
      if (sub == SUB_IOTA_FLAT) {
        r = float(i);
      } else if (sub == SUB_FILL) {
        r = s;
      } else if (sub == SUB_AFFINE) {
        r = fmaf(x, s, tt);
      } else if (ld_b) {
        r = ew_bin(sub, x, k == 0 ? xb[0] : k == 1 ? xb[1] : k == 2 ? xb[2] : xb[3]);
      } else {
        r = ew_un(sub, x);
      }
      store_f(d, dt, i, r);
    }
  }
}

// A leaf with its loops inlined: as a function calling (or jumping to) separate
// loop functions it followed the calling convention, saving its callee-saved
// registers to scratch on entry and reloading them before each jump, a memory
// round trip per entry.  Called only from the kernel, a leaf leaves the saving
// to the kernel (interprocedural register allocation).
VM_LEAF void ew_tile(Args A, uint32_t ti, uint32_t lo, uint32_t hi) {
  A = uargs(A);
  const VM_K Task& t = task_of(A, ti);
  const uint32_t sub = uni(t.p[0]), n = uni(t.p[1]);
  const uint32_t dt = uni((t.tile_op >> 8) & 0xFF);
  const uint64_t e0 = uint64_t(uni(lo)) * A->ew_ts;
  const uint64_t e1 = min(uint64_t(uni(hi)) * A->ew_ts, uint64_t(n));
  if (e0 >= e1) return;
  if (sub == SUB_CMP || sub == SUB_SELECT || sub == SUB_CONVERT || sub == SUB_BITCAST || sub == SUB_ISFINITE ||
      sub == SUB_LTS)
    return ew_special(A, ti, e0, e1);
  if (dt == DT_I32 || dt == DT_U32 || dt == DT_I64 || dt == DT_BOOL || dt == DT_F64) return ew_intlike(A, ti, e0, e1);
  gbyte* d = resolve(A, t.dst);
  const gbyte* a = resolve(A, t.a);
  const gbyte* b = resolve(A, t.b);
  const bool viewable = is_bin(sub) || is_un(sub);
  const bool views = viewable && (t.p[2] || t.p[3]);
  const float s = __uint_as_float(t.p[2]), tt = __uint_as_float(t.p[3]);
  const bool aligned = ((uintptr_t(d) | uintptr_t(a) | uintptr_t(b)) & 15) == 0;
  if (!views && aligned && dt == DT_F32) {
    switch (sub) {
#define VM_EW_CASE(S) case S: return ew_f32_range<S>(d, a, b, e0, e1, s, tt);
      VM_EW_FAST_SUBS(VM_EW_CASE)
#undef VM_EW_CASE
      default: break;
    }
  }
  if (views && aligned && (e0 & 3) == 0 && dt == DT_F32 && is_bin(sub)) {
    // broadcast operands (bias rows): 16-byte accesses instead of the per-element
    // path, whose tile of 4096 cost 17-24 us against 3 us here
    const VM_K int32_t* aux = aux_of(A);
    const PeriodicView pa = periodic_view(aux, t.p[2], e1), pb = periodic_view(aux, t.p[3], e1);
    if (pa.ok && pb.ok) {
      const uint32_t u0 = uint32_t(e0), u1 = uint32_t(e1);
      switch (sub) {
        case SUB_ADD: return ew_f32_periodic<SUB_ADD>(d, a, b, u0, u1, pa, pb);
        case SUB_MUL: return ew_f32_periodic<SUB_MUL>(d, a, b, u0, u1, pa, pb);
        case SUB_SUB: return ew_f32_periodic<SUB_SUB>(d, a, b, u0, u1, pa, pb);
        case SUB_DIV: return ew_f32_periodic<SUB_DIV>(d, a, b, u0, u1, pa, pb);
        case SUB_MAX: return ew_f32_periodic<SUB_MAX>(d, a, b, u0, u1, pa, pb);
        case SUB_MIN: return ew_f32_periodic<SUB_MIN>(d, a, b, u0, u1, pa, pb);
        default: break;
      }
    }
  }
  if (!views && aligned && (e0 & 7) == 0 && (dt == DT_BF16 || dt == DT_F16)) {
    if (dt == DT_BF16) {
      switch (sub) {
#define VM_EW_CASE(S) case S: return ew_h16_range<S, true>(d, a, b, e0, e1, s, tt);
        VM_EW_FAST_SUBS(VM_EW_CASE)
#undef VM_EW_CASE
        default: break;
      }
    } else {
      switch (sub) {
#define VM_EW_CASE(S) case S: return ew_h16_range<S, false>(d, a, b, e0, e1, s, tt);
        VM_EW_FAST_SUBS(VM_EW_CASE)
#undef VM_EW_CASE
        default: break;
      }
    }
  }
  ew_float_scalar(A, ti, e0, e1);
}

}  // namespace vm
