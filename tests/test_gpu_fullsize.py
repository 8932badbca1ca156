"""GPU parity at BASELINE.json's full sizes, and the paths the smaller tests leave
open (the N = 1 dot mode of the row-reduce tile, the constant epilogue operand).

Elementwise bars for contractions: |got - want| <= rtol * (|A| @ |B|), the
forward-error bound of a dot product (and of P @ V for attention), with rtol
1e-3 for f32 operands and 1e-2 for bf16 (the north star's GEMM / attention
tolerances), against float64 math on the same (already rounded) operands."""
import dataclasses
import math
import sys

import numpy as np
import pytest

from gpu_util import as_f32, assert_rel, blob_for, check_decoder, run_both, runtime
from oracle import vmref
from pjrt_amd import configs as CF
from pjrt_amd import graph as G
from pjrt_amd import vmprogram as V

pytestmark = pytest.mark.gpu

BF16_ULP = 2.0 ** -7


def say(*a):
    print("[gpu]", *a, file=sys.stderr, flush=True)


def assert_within_bound(got, want, bound, rtol, what):
    err = np.abs(np.asarray(got, np.float64) - want)
    lim = rtol * bound + 1e-30
    bad = err > lim
    if bad.any():
        i = tuple(np.argwhere(bad)[0])
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} outside {rtol} x |A||B|; "
                             f"first at {i}: got {float(np.asarray(got)[i])}, want {float(want[i])}, "
                             f"bound {float(lim[i])}")


def test_red_seg_dot_mode_exact():
    """A matmul with N = 1 and M > 8 is the reference's RED_SEG dot mode
    (ops/dot.py:94-161; reduce.cl:165-281): integer-valued operands give the
    exact result."""
    rng = np.random.default_rng(80)
    M, K = 3000, 1537
    a = rng.integers(-4, 5, (M, K)).astype(np.float32)
    x = rng.integers(-4, 5, (K, 1)).astype(np.float32)
    g = G.Graph()
    ga, gx = g.input(a.shape), g.input(x.shape)
    g.output(g.dot(ga, gx))
    blob, _ = blob_for(g.build())
    tasks = vmref.parse(blob).tasks
    assert tasks[0].top == V.TOP_RED_SEG and tasks[0].p[3] == 1, "expected the RED_SEG dot mode"
    got, want = run_both(blob, [a, x])
    np.testing.assert_array_equal(got[0], want[0])
    np.testing.assert_array_equal(got[0], a.astype(np.float64) @ x.astype(np.float64))


@pytest.mark.parametrize("kind", ["gemm", "gemv"])
def test_epilogue_constant_operand(kind):
    """Epilogue source 3 (constant operand s) on the bf16 MMA fast path (M, N
    multiples of 256) and on the skinny-matmul tile: bias, min(., 6),
    max(., 0.5) -- a clamp written out by hand."""
    rng = np.random.default_rng(81)
    M, K, N = (512, 256, 768) if kind == "gemm" else (1, 768, 2304)
    a = rng.integers(-2, 3, (M, K)).astype(np.float32)
    b = rng.integers(-2, 3, (K, N)).astype(np.float32)
    bias = rng.integers(-8, 9, N).astype(np.float32)
    g = G.Graph()
    x, y, bb = g.input(a.shape, "bf16"), g.input(b.shape, "bf16"), g.input(bias.shape)
    g.output(g.dot(x, y, residual=bb, tile=256 if kind == "gemm" else 0,
                   epilogue=[(V.SUB_ADD, 2, 0.0, 0.0), (V.SUB_MIN, 3, 6.0, 0.0), (V.SUB_MAX, 3, 0.5, 7.0)]))
    blob, _ = blob_for(g.build())
    tops = {t.top for t in vmref.parse(blob).tasks}
    assert (V.TOP_MMA if kind == "gemm" else V.TOP_GEMV) in tops
    got, want = run_both(blob, [a, b, bias])
    exact = np.clip(a.astype(np.float64) @ b.astype(np.float64) + bias, 0.5, 6.0)
    np.testing.assert_array_equal(got[0], exact)
    np.testing.assert_array_equal(got[0], want[0])


@pytest.mark.timeout(300)
@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_c3_full_size_gemm(dt):
    """Config 3 at 4096^3.  Integer-valued operands (|a|, |b| <= 2): every partial
    sum is an integer below 2^24, so the result is exact.  Then the benchmark's
    own draws (N(0, 1/64), seed 1003) on 256 sampled rows, elementwise against
    float64 within rtol x |A||B|."""
    M = N = K = 4096
    rt = runtime()
    g = G.Graph()
    x, y = g.input((M, K), dt), g.input((K, N), dt)
    g.output(g.dot(x, y))
    lp = rt.compile(g.build())
    try:
        rng = np.random.default_rng(82)
        a = rng.integers(-2, 3, (M, K)).astype(np.float32)
        b = rng.integers(-2, 3, (K, N)).astype(np.float32)
        say(f"C3 {dt} exact case")
        (c,) = lp(a, b)
        np.testing.assert_array_equal(c, a @ b)        # f32 BLAS is exact on these integers
        rng = np.random.default_rng(1003)
        a = rng.standard_normal((M, K), dtype=np.float32) * 0.125
        b = rng.standard_normal((K, N), dtype=np.float32) * 0.125
        if dt == "bf16":
            a, b = V.bf16_to_f32(V.f32_to_bf16(a)), V.bf16_to_f32(V.f32_to_bf16(b))
        say(f"C3 {dt} random case")
        (c,) = lp(a, b)
    finally:
        lp.close()
    rows = np.random.default_rng(0).choice(M, 256, replace=False)
    want = a[rows].astype(np.float64) @ b.astype(np.float64)
    bound = np.abs(a[rows]).astype(np.float64) @ np.abs(b).astype(np.float64)
    assert_within_bound(c[rows], want, bound, 1e-3 if dt == "f32" else 1e-2, f"C3 {dt}")


@pytest.mark.timeout(300)
def test_c4_full_size_attention():
    """Config 4 (B4 H16 S2048 d128, causal, bf16), every head computed, six heads
    checked against float64 softmax(QK^T / sqrt(d), causal) V, elementwise within
    1e-2 x (P |V|) plus one bf16 ulp of the output."""
    B, H, S, D = 4, 16, 2048, 128
    rng = np.random.default_rng(1004)
    shape = (B * H, S, D)
    q, k, v = (V.f32_to_bf16(rng.standard_normal(shape, dtype=np.float32)) for _ in range(3))
    g = G.Graph()
    Q, K_, Vv = g.input(shape, "bf16"), g.input(shape, "bf16"), g.input(shape, "bf16")
    g.output(g.flash_attention(Q, K_, Vv, 1.0 / math.sqrt(D), True, out_dtype="bf16"))
    lp = runtime().compile(g.build())
    try:
        say("C4 full size")
        (o,) = lp(q, k, v)
    finally:
        lp.close()
    o = V.bf16_to_f32(o)
    for h in (0, 13, 27, 38, 51, 63):
        qh, kh, vh = (V.bf16_to_f32(t[h]).astype(np.float64) for t in (q, k, v))
        s = (qh @ kh.T) / math.sqrt(D)
        s[np.triu_indices(S, 1)] = -np.inf
        p = np.exp(s - s.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        want = p @ vh
        bound = 1e-2 * (p @ np.abs(vh)) + BF16_ULP * np.abs(want)
        err = np.abs(o[h] - want)
        assert (err <= bound).all(), f"head {h}: {int((err > bound).sum())} elements outside the bound"


@pytest.mark.timeout(420)
def test_c5_full_128_step_loop_against_oracle():
    """The benchmarked config-5 program (prompt 512, 128 greedy decode steps in one
    FOR loop), with per-step logits, against the CPU oracle's execution of the same
    bytes: logits within 5e-3 of the largest, tokens equal until the first
    near-tie (gpu_util.check_decoder).  Measured on the MI355X: all 129 steps are
    token-exact.  Step 70 is a near-tie of the oracle's logits (top-two gap 5.4e-3
    against a tolerance of 2.8e-2), so a change of summation order in the GEMVs may
    flip it: that ends the comparison there, below the pin, and the pin is then
    re-measured, not lowered silently."""
    c = CF.C5
    args = CF.gpt_inputs(c)
    blob, _ = blob_for(CF.gpt_c5(c, emit_logits=True))
    say("C5 full 128-step program")
    got, want = run_both(blob, args, oracle="tensor")
    check_decoder(got, want, 5e-3, pinned=129, what="config-5 decoder, 128 steps")
