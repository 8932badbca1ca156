"""The C restatement of the reference's CPU path (oracle/refcpu.c, timed as the
CPU baseline) computes the same results as the numpy oracle."""
import ctypes
import os

import numpy as np
import pytest

from oracle import vmref

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "oracle", "librefcpu.so")


@pytest.fixture(scope="module")
def lib():
    if not os.path.isfile(LIB):
        pytest.skip("oracle/librefcpu.so not built (make -C oracle)")
    lib = ctypes.CDLL(LIB)
    lib.refcpu_ln_gelu_bf16.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int64, ctypes.c_int64, ctypes.c_float,
                                                               ctypes.c_void_p, ctypes.c_int]
    lib.refcpu_sgemm_packed.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int64] * 3 + [ctypes.c_void_p, ctypes.c_int]
    lib.refcpu_mlp_f32.argtypes = [ctypes.c_void_p] * 8 + [ctypes.c_int64] * 4 + [ctypes.c_int]
    lib.refcpu_attention_f32.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int64] * 3 + [ctypes.c_float, ctypes.c_int,
                                                                                      ctypes.c_void_p, ctypes.c_int]
    lib.refcpu_gpt_f32.argtypes = [ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_int64] * 7 + [
        ctypes.c_float, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
    return lib


def test_decomposed_layernorm_gelu_bf16(lib):
    rng = np.random.default_rng(1002)
    rows, d = 96, 1536
    x = rng.standard_normal((rows, d)).astype(np.float32)
    g = rng.uniform(0.5, 1.5, d).astype(np.float32)
    b = (rng.standard_normal(d) * 0.1).astype(np.float32)
    out = np.empty((rows, d), np.uint16)
    scratch = np.empty(2 * rows * d + 2 * rows, np.float32)
    lib.refcpu_ln_gelu_bf16(x.ctypes.data, g.ctypes.data, b.ctypes.data, out.ctypes.data, rows, d, 1e-5,
                            scratch.ctypes.data, 4)
    z = vmref.layernorm_core(x, 1e-5, two_pass=True).astype(np.float64) * g + b
    want = 0.5 * z * (1 + np.tanh(0.7978845608 * (z + 0.044715 * z ** 3)))
    got = vmref.bf16_to_f32(out).astype(np.float64)
    assert np.all(np.abs(got - want) <= 2.0 ** -8 * np.abs(want) + 1e-6)


@pytest.mark.parametrize("M,K,N", [(70, 300, 528), (13, 2100, 48), (5, 40, 16), (6, 1024, 32)])
def test_sgemm_packed_exact(lib, M, K, N):
    """The packed SGEMM (mm2_pack + mm2p): integer-valued operands give exact f32
    products, across edge rows (M % 6), several KC = 1024 sweeps (K = 2100, C
    reloaded between them) and a single whole sweep (K = 1024)."""
    rng = np.random.default_rng(5)
    a = rng.integers(-3, 4, (M, K)).astype(np.float32)
    b = rng.integers(-3, 4, (K, N)).astype(np.float32)
    c = np.full((M, N), np.nan, np.float32)
    bp = np.empty(K * N, np.float32)
    assert lib.refcpu_sgemm_packed(a.ctypes.data, b.ctypes.data, c.ctypes.data, M, N, K, bp.ctypes.data, 4) == 0
    np.testing.assert_array_equal(c, a.astype(np.float64) @ b.astype(np.float64))


def test_sgemm_packed_random_and_shape_rule(lib):
    rng = np.random.default_rng(6)
    M, K, N = 61, 1500, 80
    a = rng.standard_normal((M, K)).astype(np.float32)
    b = rng.standard_normal((K, N)).astype(np.float32)
    c = np.empty((M, N), np.float32)
    bp = np.empty(K * N, np.float32)
    assert lib.refcpu_sgemm_packed(a.ctypes.data, b.ctypes.data, c.ctypes.data, M, N, K, bp.ctypes.data, 4) == 0
    want = a.astype(np.float64) @ b.astype(np.float64)
    scale = np.abs(a.astype(np.float64)) @ np.abs(b.astype(np.float64))
    assert np.all(np.abs(c - want) <= 1e-5 * scale)
    # N not a multiple of 16: the reference takes another kernel; refused here
    assert lib.refcpu_sgemm_packed(a.ctypes.data, b.ctypes.data, c.ctypes.data, M, 40, K, bp.ctypes.data, 4) == -1


@pytest.mark.parametrize("causal", [True, False])
def test_attention_f32_matches_float64(lib, causal):
    rng = np.random.default_rng(8)
    G, S, D = 3, 64, 32
    q, k, v = (rng.standard_normal((G, S, D)).astype(np.float32) for _ in range(3))
    o = np.empty((G, S, D), np.float32)
    scratch = np.empty(S * S + S * D, np.float32)
    scale = 1.0 / np.sqrt(D)
    assert lib.refcpu_attention_f32(q.ctypes.data, k.ctypes.data, v.ctypes.data, o.ctypes.data, G, S, D, scale,
                                    int(causal), scratch.ctypes.data, 4) == 0
    s = np.einsum("gsd,gtd->gst", q.astype(np.float64), k.astype(np.float64)) * scale
    if causal:
        s = np.where(np.arange(S)[None, None, :] > np.arange(S)[None, :, None], -np.inf, s)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    want = p @ v.astype(np.float64)
    np.testing.assert_allclose(o, want, rtol=1e-4, atol=1e-5)
    if causal:   # row 0 sees only key 0
        np.testing.assert_allclose(o[:, 0], v[:, 0], rtol=1e-6)


def test_gpt_f32_matches_numpy_decoder(lib):
    """The f32-widened config-5 decoder (prefill on the packed SGEMM, decode on
    row GEMVs) against the independent numpy decoder without bf16 rounding:
    logits within 1e-4 of the largest, tokens equal."""
    from pjrt_amd import configs as CF
    from pjrt_amd import vmprogram as V
    c = CF.GptConfig(layers=2, d=64, heads=2, mlp=256, vocab=500, prompt=32, steps=8)
    arrays = CF.gpt_inputs(c, seed=3)
    toks_want, logits_want = CF.gpt_reference(c, arrays, bf16_stores=False)
    ids = arrays[0].astype(np.int32)
    params = [V.bf16_to_f32(a) if a.dtype == np.uint16 else a.astype(np.float32) for a in arrays[1:]]
    params = [np.ascontiguousarray(p, np.float32) for p in params]
    ptrs = (ctypes.c_void_p * len(params))(*[p.ctypes.data for p in params])
    toks = np.empty(c.steps + 1, np.int32)
    logits = np.empty((c.steps + 1, c.vocab), np.float32)
    times = np.zeros(2, np.float64)
    assert lib.refcpu_gpt_f32(ids.ctypes.data, ptrs, c.layers, c.d, c.heads, c.mlp, c.vocab, c.prompt, c.steps,
                              c.eps, toks.ctypes.data, logits.ctypes.data, times.ctypes.data, 4) == 0
    tol = 1e-4 * float(np.abs(logits_want).max())
    assert float(np.abs(logits - logits_want).max()) <= tol
    np.testing.assert_array_equal(toks, toks_want)
    assert times[0] > 0 and times[1] > 0


def test_bf16_rne_formula_exhaustive(lib):
    """All 2^32 f32 patterns: the bit formula equals round-to-nearest-even
    computed in double precision; NaN stays NaN."""
    lib.refcpu_bf16_rne_check.restype = ctypes.c_int64
    lib.refcpu_bf16_rne_check.argtypes = [ctypes.c_int, ctypes.c_uint32, ctypes.c_uint32,
                                          ctypes.POINTER(ctypes.c_uint32)]
    first = ctypes.c_uint32(0)
    assert lib.refcpu_bf16_rne_check(0, 0, 65536, ctypes.byref(first)) == 0, hex(first.value)
    # a planted mistake (truncation instead of rounding) must be caught
    assert lib.refcpu_bf16_rne_check(1, 0x3F80, 0x3F81, ctypes.byref(first)) > 0


def test_bf16_formula_matches_numpy_oracle(lib):
    """The numpy oracle's f32_to_bf16 is the same bit formula (sampled patterns)."""
    rng = np.random.default_rng(7)
    u = np.concatenate([rng.integers(0, 2 ** 32, 1 << 20, dtype=np.uint64).astype(np.uint32),
                        np.array([0x7F7FFFFF, 0x7F7F8000, 0x3F808000, 0x3F818000, 0x00008000, 0x7FC00001,
                                  0xFF800000, 0x80000000], np.uint32)])
    got = vmref.f32_to_bf16(u.view(np.float32))
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    want = ((u.astype(np.uint64) + 0x7FFF + ((u.astype(np.uint64) >> 16) & 1)) >> 16).astype(np.uint16)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all(((got[nan] & 0x7F80) == 0x7F80) & ((got[nan] & 0x7F) != 0))


def test_mlp_f32_matches_numpy(lib):
    from pjrt_amd import configs as CF
    x, w1, b1, w2, b2 = CF.mlp_c1_inputs(batch=40, d_in=24, d_hidden=64, d_out=16)
    y = np.empty((40, 16), np.float32)
    h = np.empty((40, 64), np.float32)
    bp = np.empty(64 * 24, np.float32)
    assert lib.refcpu_mlp_f32(x.ctypes.data, w1.ctypes.data, b1.ctypes.data, w2.ctypes.data, b2.ctypes.data,
                              y.ctypes.data, h.ctypes.data, bp.ctypes.data, 40, 24, 64, 16, 3) == 0
    want = np.maximum(x.astype(np.float64) @ w1 + b1, 0) @ w2 + b2
    np.testing.assert_allclose(y, want, rtol=1e-4, atol=1e-5)
