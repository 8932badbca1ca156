// Scalar math of the VM's f32 domain, shared by the elementwise tile op, the fused
// map-region micro-ALU and the matmul store epilogue so a fused chain computes
// exactly what the unfused elementwise ops compute (reference contract:
// vm_common.cl:161-196 must byte-match ops/ew.cl).
#pragma once
#include "vm_device.h"

namespace vm {

// tanh-GELU 0.5*x*(1 + tanh(c0*(x + c1*x^3))) with c0 = 0.7978845608,
// c1 = 0.044715 (ew.cl:7-17), evaluated as x * sigmoid(2*c0*(x + c1*x^3)):
// 0.5*(1 + tanh(u)) == 1/(1 + exp(-2u)), so one v_exp_f32 and one v_rcp_f32
// replace tanh.  exp(-2u) = 2^(-2*log2(e)*u).
// With the constants folded, -2*log2(e)*u = x * (k0 + k1*x^2):
// mul, fma, mul, v_exp_f32, add, v_rcp_f32, mul.
VM_DEV float gelu(float x) {
  constexpr double kC0 = 0.7978845608, kC1 = 0.044715, kNeg2Log2e = -2.0 * 1.4426950408889634;
  constexpr float k0 = float(kNeg2Log2e * kC0);
  constexpr float k1 = float(kNeg2Log2e * kC0 * kC1);
  const float t = x * fmaf(k1, x * x, k0);
  const float e = __builtin_amdgcn_exp2f(t);
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}

VM_DEV float round_afz(float x) {            // C roundf: half away from zero
  return roundf(x);
}

VM_DEV bool is_bin(uint32_t sub) { return sub <= SUB_POW || (sub >= SUB_ATAN2 && sub <= SUB_REMAINDER); }
VM_DEV bool is_un(uint32_t sub) {
  return (sub >= SUB_COPY && sub <= SUB_SIGN) || (sub >= SUB_LOG1P && sub <= SUB_ROUND) || sub == SUB_GELU;
}

// Binary f32 subops (ew.cl:19-30).  fmax/fmin ignore a NaN operand.
VM_DEV float ew_bin(uint32_t sub, float x, float y) {
  switch (sub) {
    case SUB_ADD: return x + y;
    case SUB_MUL: return x * y;
    case SUB_SUB: return x - y;
    case SUB_DIV: return x / y;
    case SUB_MAX: return fmaxf(x, y);
    case SUB_MIN: return fminf(x, y);
    case SUB_POW: return powf(x, y);
    case SUB_ATAN2: return atan2f(x, y);
    case SUB_REMAINDER: return fmodf(x, y);
    default: return 0.0f;
  }
}

// Unary f32 subops (ew.cl:31-50).
VM_DEV float ew_un(uint32_t sub, float x) {
  switch (sub) {
    case SUB_COPY: return x;
    case SUB_NEG: return -x;
    case SUB_EXP: return expf(x);
    case SUB_LOG: return logf(x);
    case SUB_SQRT: return sqrtf(x);
    case SUB_RSQRT: return rsqrtf(x);
    case SUB_TANH: return tanhf(x);
    case SUB_ABS: return fabsf(x);
    case SUB_FLOOR: return floorf(x);
    case SUB_CEIL: return ceilf(x);
    case SUB_SIGN: return x > 0.0f ? 1.0f : (x < 0.0f ? -1.0f : x);
    case SUB_LOG1P: return log1pf(x);
    case SUB_EXPM1: return expm1f(x);
    case SUB_CBRT: return cbrtf(x);
    case SUB_SIN: return sinf(x);
    case SUB_COS: return cosf(x);
    case SUB_TAN: return tanf(x);
    case SUB_RINT: return rintf(x);
    case SUB_ROUND: return round_afz(x);
    case SUB_GELU: return gelu(x);
    default: return 0.0f;
  }
}

// Micro-op of the map-region / matmul epilogue programs: EW subop kinds plus
// AFFINE (x*s + t) (vm_common.cl:173-196).
VM_DEV float micro(uint32_t kind, float x, float y, float s, float t) {
  if (kind == SUB_AFFINE) return fmaf(x, s, t);
  if (is_bin(kind)) return ew_bin(kind, x, y);
  if (is_un(kind)) return ew_un(kind, x);
  return x;
}

}  // namespace vm
