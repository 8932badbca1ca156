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
 *   - f32 matmul (config 3 in f32): the packed SGEMM the reference's CPU engine
 *     peels matmul phases to, mm2_pack + mm2p with KC = 1024 sweeps
 *     (vm_main.cl:419-518; runtime.cc:1226-1306, 1698-1800);
 *   - config 1, the f32 MLP: two packed SGEMM phases with the bias in their
 *     store (mm2p_epi) and the relu as an elementwise phase between them;
 *   - configs 4 and 5, which the reference cannot run (bf16 flash attention; a
 *     variadic-reduce argmax): their f32-widened computation in the same style,
 *     labelled as such wherever it is reported.
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

/* ---- packed SGEMM: the reference's CPU matmul ------------------------------------------
 * mm2_pack + mm2p (vm_main.cl:419-518) as the host enqueues them
 * (LoadedProgram::EnqueuePackedMM, runtime.cc:1226-1306):
 *   - B [K, N] is copied into 16-column panels, Bp[p K 16 + k 16 + j] = B[k, 16 p + j],
 *     so the k loop reads each panel sequentially;
 *   - K is swept in blocks of KC = 1024; each sweep runs a 2D grid of 6-row blocks x
 *     groups of PC = 2 panels, one work-item per cell (PoCL: one host thread);
 *   - a cell keeps a 6 x 16 block of C in twelve 8-float registers, starts from 0 on
 *     the first sweep and from C in memory on later ones, and accumulates
 *     c += a[r, k] * panel[k, :] in k order;
 *   - rows past the last whole 6-row block take one scalar full-K pass on the
 *     first sweep.
 * N must be a multiple of 16 (the reference falls back to another kernel
 * otherwise).  `bp` holds K * N floats. */
typedef float v8f __attribute__((vector_size(32), aligned(4)));

enum { kMmKC = 1024, kMmPC = 2 };

static void mm_pack(const float* B, int64_t ldb, int trans, float* bp, int64_t K, int64_t N) {
  const int64_t np = N / 16;
#pragma omp parallel for schedule(static)
  for (int64_t pk = 0; pk < np * K; ++pk) {
    const int64_t p = pk / K, k = pk % K;
    float* dst = bp + p * K * 16 + k * 16;
    for (int j = 0; j < 16; ++j) dst[j] = trans ? B[(p * 16 + j) * ldb + k] : B[k * ldb + p * 16 + j];
  }
}

/* one KC sweep [kc0, kc1) of the 2D grid */
static void mm_sweep(const float* A, int64_t lda, const float* bp, float* C, int64_t ldc, int64_t M, int64_t N,
                     int64_t K, int64_t kc0, int64_t kc1) {
  const int64_t np = N / 16, nrb = (M + 5) / 6, npg = (np + kMmPC - 1) / kMmPC;
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t rb = 0; rb < nrb; ++rb) {
    for (int64_t pg0 = 0; pg0 < npg; ++pg0) {
      const int64_t r0 = rb * 6, pg = pg0 * kMmPC, pe = pg + kMmPC < np ? pg + kMmPC : np;
      if (r0 + 6 > M) {
        if (kc0 == 0)
          for (int64_t p = pg; p < pe; ++p)
            for (int64_t c0 = p * 16; c0 < p * 16 + 16; ++c0)
              for (int64_t i = 0; i < M - r0; ++i) {
                float s = 0.0f;
                for (int64_t k = 0; k < K; ++k) s = fmaf(A[(r0 + i) * lda + k], bp[p * K * 16 + k * 16 + (c0 % 16)], s);
                C[(r0 + i) * ldc + c0] = s;
              }
        continue;
      }
      const float* a0 = A + (r0 + 0) * lda;
      const float* a1 = A + (r0 + 1) * lda;
      const float* a2 = A + (r0 + 2) * lda;
      const float* a3 = A + (r0 + 3) * lda;
      const float* a4 = A + (r0 + 4) * lda;
      const float* a5 = A + (r0 + 5) * lda;
      for (int64_t p = pg; p < pe; ++p) {
        const float* panel = bp + p * K * 16;
        float* cp = C + r0 * ldc + p * 16;
        v8f c00, c01, c02, c03, c04, c05, c10, c11, c12, c13, c14, c15;
        if (kc0 == 0) {
          c00 = c01 = c02 = c03 = c04 = c05 = c10 = c11 = c12 = c13 = c14 = c15 = (v8f){0};
        } else {
          c00 = *(const v8f*)(cp + 0 * ldc); c10 = *(const v8f*)(cp + 0 * ldc + 8);
          c01 = *(const v8f*)(cp + 1 * ldc); c11 = *(const v8f*)(cp + 1 * ldc + 8);
          c02 = *(const v8f*)(cp + 2 * ldc); c12 = *(const v8f*)(cp + 2 * ldc + 8);
          c03 = *(const v8f*)(cp + 3 * ldc); c13 = *(const v8f*)(cp + 3 * ldc + 8);
          c04 = *(const v8f*)(cp + 4 * ldc); c14 = *(const v8f*)(cp + 4 * ldc + 8);
          c05 = *(const v8f*)(cp + 5 * ldc); c15 = *(const v8f*)(cp + 5 * ldc + 8);
        }
        for (int64_t k = kc0; k < kc1; ++k) {
          const v8f b0 = *(const v8f*)(panel + k * 16), b1 = *(const v8f*)(panel + k * 16 + 8);
          c00 += a0[k] * b0; c10 += a0[k] * b1;
          c01 += a1[k] * b0; c11 += a1[k] * b1;
          c02 += a2[k] * b0; c12 += a2[k] * b1;
          c03 += a3[k] * b0; c13 += a3[k] * b1;
          c04 += a4[k] * b0; c14 += a4[k] * b1;
          c05 += a5[k] * b0; c15 += a5[k] * b1;
        }
        *(v8f*)(cp + 0 * ldc) = c00; *(v8f*)(cp + 0 * ldc + 8) = c10;
        *(v8f*)(cp + 1 * ldc) = c01; *(v8f*)(cp + 1 * ldc + 8) = c11;
        *(v8f*)(cp + 2 * ldc) = c02; *(v8f*)(cp + 2 * ldc + 8) = c12;
        *(v8f*)(cp + 3 * ldc) = c03; *(v8f*)(cp + 3 * ldc + 8) = c13;
        *(v8f*)(cp + 4 * ldc) = c04; *(v8f*)(cp + 4 * ldc + 8) = c14;
        *(v8f*)(cp + 5 * ldc) = c05; *(v8f*)(cp + 5 * ldc + 8) = c15;
      }
    }
  }
}

/* C[M,N] = A[M,K] . B[K,N] (B given transposed, Bt[N,K], when `trans_b`), f32
 * row-major; the packed SGEMM above.  Returns -1 when N is not a multiple of 16. */
static int mm_packed(const float* A, int64_t lda, const float* B, int64_t ldb, int trans_b, float* C, int64_t ldc,
                     int64_t M, int64_t N, int64_t K, float* bp) {
  if (N % 16) return -1;
  mm_pack(B, ldb, trans_b, bp, K, N);
  for (int64_t kc = 0; kc < K; kc += kMmKC) mm_sweep(A, lda, bp, C, ldc, M, N, K, kc, kc + kMmKC < K ? kc + kMmKC : K);
  return 0;
}

int refcpu_sgemm_packed(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K, float* bp,
                        int threads) {
  omp_set_num_threads(threads);
  return mm_packed(A, K, B, N, 0, C, N, M, N, K, bp);
}

/* Config 1, the f32 MLP y = relu(x W1 + b1) W2 + b2, as the reference's CPU engine
 * runs it: each matmul phase peeled to the packed SGEMM with the bias fused into
 * its store (mm2p_epi, vm_main.cl:524-579: one K sweep, the epilogue per element
 * at store), the relu as an elementwise phase between them.  `h` holds M * H
 * floats, `bp` max(D * H, H * O) floats. */
int refcpu_mlp_f32(const float* x, const float* w1, const float* b1, const float* w2, const float* b2, float* y,
                   float* h, float* bp, int64_t M, int64_t D, int64_t H, int64_t O, int threads) {
  omp_set_num_threads(threads);
  if (H % 16 || O % 16) return -1;
  mm_pack(w1, H, 0, bp, D, H);
  mm_sweep(x, D, bp, h, H, M, H, D, 0, D);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < M * H; ++i) h[i] += b1[i % H];
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < M * H; ++i) h[i] = h[i] > 0.0f ? h[i] : 0.0f;
  mm_pack(w2, O, 0, bp, H, O);
  mm_sweep(h, H, bp, y, O, M, O, H, 0, H);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < M * O; ++i) y[i] += b2[i % O];
  return 0;
}

/* ---- f32-widened stand-ins for configs the reference cannot run ------------------------
 * Config 4 (bf16 causal flash attention) and config 5 (a bf16 decoder whose argmax
 * is a variadic reduce) are unsupported on the reference (ops/reduce.py:165-168;
 * flash attention off and non-causal by default, lowering.py:2690-2691).  These
 * time the f32 computation the reference's CPU engine would run if widened, in its
 * style: matmul phases on the packed SGEMM, softmax / layernorm / GELU as row and
 * elementwise passes. */

/* Causal (or full) attention o = softmax(scale q k^T [mask]) v over G heads of
 * [S, D], f32, the reference's decomposed chain per head: scores on the packed
 * SGEMM (k read as the transposed operand), scale and mask, row max, exp, row sum,
 * normalise, then p v on the packed SGEMM.  The full S x S scores are computed
 * (the decomposed chain does not skip masked blocks).  `scratch` holds
 * S * S + S * D floats; S and D multiples of 16. */
int refcpu_attention_f32(const float* q, const float* k, const float* v, float* o, int64_t G, int64_t S, int64_t D,
                         float scale, int causal, float* scratch, int threads) {
  omp_set_num_threads(threads);
  if (S % 16 || D % 16) return -1;
  float* s = scratch;
  float* bp = scratch + S * S;
  for (int64_t g = 0; g < G; ++g) {
    const float* qg = q + g * S * D;
    const float* kg = k + g * S * D;
    const float* vg = v + g * S * D;
    mm_packed(qg, D, kg, D, 1, s, S, S, S, D, bp);
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < S; ++r) {
      float* row = s + r * S;
      float m = -INFINITY;
      for (int64_t c = 0; c < S; ++c) {
        row[c] = (causal && c > r) ? -INFINITY : row[c] * scale;
        m = row[c] > m ? row[c] : m;
      }
      float sum = 0.0f;
      for (int64_t c = 0; c < S; ++c) {
        row[c] = expf(row[c] - m);
        sum += row[c];
      }
      const float inv = 1.0f / sum;
      for (int64_t c = 0; c < S; ++c) row[c] *= inv;
    }
    mm_packed(s, S, vg, D, 0, o + g * S * D, D, S, D, S, bp);
  }
  return 0;
}

static void layernorm_row(const float* x, const float* g, const float* b, float* y, int64_t d, float eps) {
  float s = 0.0f;
  for (int64_t j = 0; j < d; ++j) s += x[j];
  const float mu = s / (float)d;
  float q = 0.0f;
  for (int64_t j = 0; j < d; ++j) q += (x[j] - mu) * (x[j] - mu);
  const float rstd = 1.0f / sqrtf(q / (float)d + eps);
  for (int64_t j = 0; j < d; ++j) y[j] = (x[j] - mu) * rstd * g[j] + b[j];
}

/* y[N] = x[K] . W[K, N] (+ bias): the decode-time matmul of one token, threads over
 * column blocks, each streaming its columns of every weight row */
static void gemv_row(const float* x, const float* W, const float* bias, float* y, int64_t K, int64_t N) {
  const int64_t NB = 256;
#pragma omp parallel for schedule(static)
  for (int64_t n0 = 0; n0 < N; n0 += NB) {
    const int64_t n1 = n0 + NB < N ? n0 + NB : N;
    float acc[256];
    for (int64_t j = n0; j < n1; ++j) acc[j - n0] = bias ? bias[j] : 0.0f;
    for (int64_t k = 0; k < K; ++k) {
      const float a = x[k];
      const float* w = W + k * N;
      for (int64_t j = n0; j < n1; ++j) acc[j - n0] += a * w[j];
    }
    for (int64_t j = n0; j < n1; ++j) y[j] = acc[j - n0];
  }
}

/* The config-5 decoder (prefill of the prompt, then `steps` greedy tokens), every
 * parameter widened to f32 and every activation kept in f32.  `P` lists the
 * parameters in the program's input order: wte, wpe, then per layer ln1_g, ln1_b,
 * w_qkv, b_qkv, w_o, b_o, ln2_g, ln2_b, w_fc, b_fc, w_proj, b_proj, then lnf_g,
 * lnf_b, lm_head.  Writes 1 + steps tokens, the logits of each when `logits` is
 * not null, and the prefill and decode wall times (seconds) to times[0..1].
 * Returns 0, or -1 on a shape the packed SGEMM cannot take or no memory. */
int refcpu_gpt_f32(const int32_t* ids, const float* const* P, int64_t layers, int64_t d, int64_t heads, int64_t mlp,
                   int64_t vocab, int64_t prompt, int64_t steps, float eps, int32_t* toks, float* logits,
                   double* times, int threads) {
  omp_set_num_threads(threads);
  const int64_t T = prompt, ctx = prompt + steps, hd = d / heads, d3 = 3 * d;
  if (d % 16 || d3 % 16 || mlp % 16 || T % 16 || hd % 16) return -1;
  const float scale = 1.0f / sqrtf((float)hd);
  const int64_t bp_n = (d * mlp > d * d3 ? d * mlp : d * d3) > T * hd ? (d * mlp > d * d3 ? d * mlp : d * d3) : T * hd;
  float* x = malloc(sizeof(float) * T * d);
  float* h = malloc(sizeof(float) * T * d);
  float* qkv = malloc(sizeof(float) * T * d3);
  float* att = malloc(sizeof(float) * T * d);
  float* f = malloc(sizeof(float) * T * mlp);
  float* kc = malloc(sizeof(float) * layers * heads * ctx * hd);
  float* vc = malloc(sizeof(float) * layers * heads * ctx * hd);
  float* sc = malloc(sizeof(float) * heads * T * (T > ctx ? T : ctx));
  float* bp = malloc(sizeof(float) * bp_n);
  float* lg = malloc(sizeof(float) * vocab);
  if (!x || !h || !qkv || !att || !f || !kc || !vc || !sc || !bp || !lg) {
    free(x); free(h); free(qkv); free(att); free(f); free(kc); free(vc); free(sc); free(bp); free(lg);
    return -1;
  }
  const float* wte = P[0];
  const float* wpe = P[1];
  const float* const* L0 = P + 2;
  const float* lnf_g = P[2 + 12 * layers];
  const float* lnf_b = P[3 + 12 * layers];
  const float* head = P[4 + 12 * layers];
  double t0 = omp_get_wtime();
  /* ---- prefill ---- */
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < T; ++t)
    for (int64_t j = 0; j < d; ++j) x[t * d + j] = wte[(int64_t)ids[t] * d + j] + wpe[t * d + j];
  for (int64_t l = 0; l < layers; ++l) {
    const float* const* W = L0 + 12 * l;
    float* Kl = kc + l * heads * ctx * hd;
    float* Vl = vc + l * heads * ctx * hd;
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < T; ++t) layernorm_row(x + t * d, W[0], W[1], h + t * d, d, eps);
    mm_packed(h, d, W[2], d3, 0, qkv, d3, T, d3, d, bp);
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < T; ++t)
      for (int64_t j = 0; j < d3; ++j) qkv[t * d3 + j] += W[3][j];
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t hh = 0; hh < heads; ++hh)
      for (int64_t t = 0; t < T; ++t)
        for (int64_t e = 0; e < hd; ++e) {
          Kl[(hh * ctx + t) * hd + e] = qkv[t * d3 + d + hh * hd + e];
          Vl[(hh * ctx + t) * hd + e] = qkv[t * d3 + 2 * d + hh * hd + e];
        }
    /* causal attention per head and query row: scores, softmax, weighted values */
#pragma omp parallel for collapse(2) schedule(dynamic, 8)
    for (int64_t hh = 0; hh < heads; ++hh)
      for (int64_t t = 0; t < T; ++t) {
        float* s = sc + (hh * T + t) * T;
        const float* qr = qkv + t * d3 + hh * hd;
        float m = -INFINITY;
        for (int64_t c = 0; c <= t; ++c) {
          const float* kr = Kl + (hh * ctx + c) * hd;
          float a = 0.0f;
          for (int64_t e = 0; e < hd; ++e) a += qr[e] * kr[e];
          s[c] = a * scale;
          m = s[c] > m ? s[c] : m;
        }
        float sum = 0.0f;
        for (int64_t c = 0; c <= t; ++c) {
          s[c] = expf(s[c] - m);
          sum += s[c];
        }
        float* o = att + t * d + hh * hd;
        for (int64_t e = 0; e < hd; ++e) o[e] = 0.0f;
        for (int64_t c = 0; c <= t; ++c) {
          const float pw = s[c] / sum;
          const float* vr = Vl + (hh * ctx + c) * hd;
          for (int64_t e = 0; e < hd; ++e) o[e] += pw * vr[e];
        }
      }
    mm_packed(att, d, W[4], d, 0, h, d, T, d, d, bp);
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < T; ++t)
      for (int64_t j = 0; j < d; ++j) x[t * d + j] += h[t * d + j] + W[5][j];
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < T; ++t) layernorm_row(x + t * d, W[6], W[7], h + t * d, d, eps);
    mm_packed(h, d, W[8], mlp, 0, f, mlp, T, mlp, d, bp);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < T * mlp; ++i) f[i] = gelu_tanh(f[i] + W[9][i % mlp]);
    mm_packed(f, mlp, W[10], d, 0, h, d, T, d, mlp, bp);
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < T; ++t)
      for (int64_t j = 0; j < d; ++j) x[t * d + j] += h[t * d + j] + W[11][j];
  }
  double t1 = omp_get_wtime();
  /* ---- logits of the last prompt row, then the decode loop ---- */
  float* xr = x + (T - 1) * d;
  for (int64_t step = 0; step <= steps; ++step) {
    if (step > 0) {
      const int64_t pos = T + step - 1;
      xr = x;
      for (int64_t j = 0; j < d; ++j) xr[j] = wte[(int64_t)toks[step - 1] * d + j] + wpe[pos * d + j];
      for (int64_t l = 0; l < layers; ++l) {
        const float* const* W = L0 + 12 * l;
        float* Kl = kc + l * heads * ctx * hd;
        float* Vl = vc + l * heads * ctx * hd;
        layernorm_row(xr, W[0], W[1], h, d, eps);
        gemv_row(h, W[2], W[3], qkv, d, d3);
        for (int64_t hh = 0; hh < heads; ++hh)
          for (int64_t e = 0; e < hd; ++e) {
            Kl[(hh * ctx + pos) * hd + e] = qkv[d + hh * hd + e];
            Vl[(hh * ctx + pos) * hd + e] = qkv[2 * d + hh * hd + e];
          }
#pragma omp parallel for schedule(static)
        for (int64_t hh = 0; hh < heads; ++hh) {
          float* s = sc + hh * ctx;
          const float* qr = qkv + hh * hd;
          float m = -INFINITY;
          for (int64_t c = 0; c <= pos; ++c) {
            const float* kr = Kl + (hh * ctx + c) * hd;
            float a = 0.0f;
            for (int64_t e = 0; e < hd; ++e) a += qr[e] * kr[e];
            s[c] = a * scale;
            m = s[c] > m ? s[c] : m;
          }
          float sum = 0.0f;
          for (int64_t c = 0; c <= pos; ++c) {
            s[c] = expf(s[c] - m);
            sum += s[c];
          }
          float* o = att + hh * hd;
          for (int64_t e = 0; e < hd; ++e) o[e] = 0.0f;
          for (int64_t c = 0; c <= pos; ++c) {
            const float pw = s[c] / sum;
            const float* vr = Vl + (hh * ctx + c) * hd;
            for (int64_t e = 0; e < hd; ++e) o[e] += pw * vr[e];
          }
        }
        gemv_row(att, W[4], W[5], h, d, d);
        for (int64_t j = 0; j < d; ++j) xr[j] += h[j];
        layernorm_row(xr, W[6], W[7], h, d, eps);
        gemv_row(h, W[8], W[9], f, d, mlp);
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < mlp; ++i) f[i] = gelu_tanh(f[i]);
        gemv_row(f, W[10], W[11], h, mlp, d);
        for (int64_t j = 0; j < d; ++j) xr[j] += h[j];
      }
    }
    layernorm_row(xr, lnf_g, lnf_b, h, d, eps);
    gemv_row(h, head, NULL, lg, d, vocab);
    int64_t best = 0;
    for (int64_t j = 1; j < vocab; ++j)
      if (lg[j] > lg[best]) best = j;
    toks[step] = (int32_t)best;
    if (logits) memcpy(logits + step * vocab, lg, sizeof(float) * vocab);
  }
  double t2 = omp_get_wtime();
  if (times) {
    times[0] = t1 - t0;
    times[1] = t2 - t1;
  }
  free(x); free(h); free(qkv); free(att); free(f); free(kc); free(vc); free(sc); free(bp); free(lg);
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
