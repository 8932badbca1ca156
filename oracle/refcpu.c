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
 *     (vm_main.cl:419-518), row panels split over the cores.
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

int refcpu_max_threads(void) { return omp_get_max_threads(); }
