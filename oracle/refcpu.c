/*
 * refcpu.c -- TEST INFRASTRUCTURE ONLY: C restatement of the reference plugin's
 * CPU (PoCL) execution path, timed as bench.py's CPU baseline.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 *
 * The reference cannot run here (no jax, no PoCL; see oracle/__init__.py), so this
 * file restates what its CPU engine executes for a configuration:
 *
 *   - config 2, layernorm + tanh-GELU + f32->bf16 on [rows, d]: for d > 1024 the
 *     reference's fused norm does not fire (python/pjrt_ocl/lowering.py:1553,
 *     1635), so the program is the decomposed chain of barrier phases the JAX
 *     layernorm lowers to (tools/bench_transformer.py:23-26):
 *       row sum -> mean, x - mean, square, row sum -> var, + eps, ^-0.5,
 *       * rstd, * gamma, + beta, GELU (OP_GELU, ew.cl:7-17), convert (RNE,
 *       vm_common.cl:66-70)
 *     each phase a full pass over memory, as the reference's host-dispatch engine
 *     runs them (runtime.cc:1483-2105), work split over the host cores like PoCL's
 *     one-work-item work-groups (runtime.cc:620-622);
 *   - f32 matmul: a cache-blocked SGEMM standing in for the packed mm2p kernel
 *     (vm_main.cl:419-518), row panels split over the cores;
 *   - config 1, the f32 MLP: two SGEMM phases with the bias adds and the relu
 *     as elementwise phases between them.
 *
 * Parity of these routines is checked by tests/test_refcpu.py against the numpy
 * oracle; they exist to be timed, not to define semantics.
 */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static uint16_t f32_to_bf16_rne(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

static float gelu_tanh(float x) {
  return 0.5f * x * (1.0f + tanhf(0.7978845608f * (x + 0.044715f * x * x * x)));
}

/* Decomposed layernorm + GELU + bf16 convert.  `scratch` holds 2*rows*d + 2*rows
 * floats (the phase intermediates).  Returns 0. */
int refcpu_ln_gelu_bf16(const float* x, const float* gamma, const float* beta, uint16_t* out, int64_t rows,
                        int64_t d, float eps, float* scratch, int threads) {
  float* t0 = scratch;                 /* [rows, d] */
  float* t1 = scratch + rows * d;      /* [rows, d] */
  float* rs = scratch + 2 * rows * d;  /* [rows] */
  float* rv = rs + rows;               /* [rows] */
  const float inv = 1.0f / (float)d;
  omp_set_num_threads(threads);
  /* phase: row sum -> mean */
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    float s = 0.0f;
    for (int64_t j = 0; j < d; ++j) s += x[r * d + j];
    rs[r] = s * inv;
  }
  /* phase: x - mean (broadcast view) */
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t j = 0; j < d; ++j) t0[r * d + j] = x[r * d + j] - rs[r];
  /* phase: square */
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < rows * d; ++i) t1[i] = t0[i] * t0[i];
  /* phase: row sum -> var, + eps, ^-0.5 */
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    float s = 0.0f;
    for (int64_t j = 0; j < d; ++j) s += t1[r * d + j];
    rv[r] = powf(s * inv + eps, -0.5f);
  }
  /* phase: * rstd (broadcast view) */
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t j = 0; j < d; ++j) t1[r * d + j] = t0[r * d + j] * rv[r];
  /* phase: * gamma (broadcast view) */
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t j = 0; j < d; ++j) t0[r * d + j] = t1[r * d + j] * gamma[j];
  /* phase: + beta (broadcast view) */
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t j = 0; j < d; ++j) t1[r * d + j] = t0[r * d + j] + beta[j];
  /* phase: GELU */
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < rows * d; ++i) t0[i] = gelu_tanh(t1[i]);
  /* phase: convert f32 -> bf16 */
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < rows * d; ++i) out[i] = f32_to_bf16_rne(t0[i]);
  return 0;
}

/* C[M,N] = A[M,K] . B[K,N], f32, row-major; blocked over K and N. */
int refcpu_sgemm(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K, int threads) {
  const int64_t KC = 256, NC = 512;
  omp_set_num_threads(threads);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < M; ++i)
    for (int64_t j = 0; j < N; ++j) C[i * N + j] = 0.0f;
  for (int64_t k0 = 0; k0 < K; k0 += KC) {
    const int64_t k1 = k0 + KC < K ? k0 + KC : K;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < M; ++i) {
      for (int64_t n0 = 0; n0 < N; n0 += NC) {
        const int64_t n1 = n0 + NC < N ? n0 + NC : N;
        float* c = C + i * N;
        for (int64_t k = k0; k < k1; ++k) {
          const float a = A[i * K + k];
          const float* b = B + k * N;
          for (int64_t j = n0; j < n1; ++j) c[j] += a * b[j];
        }
      }
    }
  }
  return 0;
}

/* Config 1, the f32 MLP y = relu(x W1 + b1) W2 + b2, as the reference's CPU engine
 * runs it: each matmul phase peeled to the packed SGEMM (runtime.cc:1698-1800),
 * the bias adds and the relu as elementwise phases over the result.  `h` holds
 * M * H floats. */
int refcpu_mlp_f32(const float* x, const float* w1, const float* b1, const float* w2, const float* b2, float* y,
                   float* h, int64_t M, int64_t D, int64_t H, int64_t O, int threads) {
  refcpu_sgemm(x, w1, h, M, H, D, threads);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < M * H; ++i) h[i] += b1[i % H];
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < M * H; ++i) h[i] = h[i] > 0.0f ? h[i] : 0.0f;
  refcpu_sgemm(h, w2, y, M, O, H, threads);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < M * O; ++i) y[i] += b2[i % O];
  return 0;
}

int refcpu_max_threads(void) { return omp_get_max_threads(); }

/* Pins the f32 -> bf16 bit formula (u + 0x7fff + ((u >> 16) & 1)) >> 16
 * (vm_common.cl:66-70) against round-to-nearest-even computed independently in
 * double precision, over the bit patterns whose high half lies in [hi0, hi1)
 * (all 2^32 patterns for [0, 65536)).  For finite x with exponent e, the bf16
 * quantum is 2^(max(e, -126) - 7); x / quantum is exact in double, so nearbyint
 * (ties to even) gives the correctly rounded bf16 value, and values that round to
 * 2^128 overflow to infinity.  NaN inputs must map to a NaN.  Returns the number
 * of mismatching patterns; *first receives the smallest one.  plant != 0 checks
 * plain truncation (u >> 16) instead, which the check must reject. */
int64_t refcpu_bf16_rne_check(int plant, uint32_t hi0, uint32_t hi1, uint32_t* first) {
  int64_t bad = 0;
  uint32_t first_bad = 0xFFFFFFFFu;
#pragma omp parallel for schedule(static) reduction(+ : bad) reduction(min : first_bad)
  for (int64_t hi = hi0; hi < (int64_t)hi1; ++hi) {
    for (uint32_t lo = 0; lo < 65536; ++lo) {
      const uint32_t u = (uint32_t)(hi << 16) | lo;
      float f;
      memcpy(&f, &u, 4);
      const uint16_t got = plant ? (uint16_t)(u >> 16) : f32_to_bf16_rne(f);
      uint16_t want;
      if (isnan(f)) {
        if ((got & 0x7F80u) == 0x7F80u && (got & 0x7Fu) != 0) continue;
        want = 0xFFFF;   /* any non-NaN result is a mismatch */
      } else if (f == 0.0f || isinf(f)) {
        want = (uint16_t)(u >> 16);
      } else {
        const double d = (double)f;
        int e = ilogb(d);
        if (e < -126) e = -126;
        const double q = ldexp(1.0, e - 7);
        const double r = nearbyint(d / q) * q;
        const float rf = (float)r; /* exact, or +-inf for |r| = 2^128 */
        uint32_t rb;
        memcpy(&rb, &rf, 4);
        want = (uint16_t)(rb >> 16);
      }
      if (got != want) {
        ++bad;
        if (u < first_bad) first_bad = u;
      }
    }
  }
  if (first) *first = first_bad;
  return bad;
}
