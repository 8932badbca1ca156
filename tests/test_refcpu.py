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
    lib.refcpu_sgemm.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int64] * 3 + [ctypes.c_int]
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


def test_sgemm(lib):
    rng = np.random.default_rng(5)
    M, K, N = 70, 300, 530
    a = rng.integers(-3, 4, (M, K)).astype(np.float32)
    b = rng.integers(-3, 4, (K, N)).astype(np.float32)
    c = np.empty((M, N), np.float32)
    lib.refcpu_sgemm(a.ctypes.data, b.ctypes.data, c.ctypes.data, M, N, K, 4)
    np.testing.assert_array_equal(c, a.astype(np.float64) @ b.astype(np.float64))


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
    lib.refcpu_mlp_f32.argtypes = [ctypes.c_void_p] * 7 + [ctypes.c_int64] * 4 + [ctypes.c_int]
    from pjrt_amd import configs as CF
    x, w1, b1, w2, b2 = CF.mlp_c1_inputs(batch=40, d_in=24, d_hidden=56, d_out=12)
    y = np.empty((40, 12), np.float32)
    h = np.empty((40, 56), np.float32)
    lib.refcpu_mlp_f32(x.ctypes.data, w1.ctypes.data, b1.ctypes.data, w2.ctypes.data, b2.ctypes.data,
                       y.ctypes.data, h.ctypes.data, 40, 24, 56, 12, 3)
    want = np.maximum(x.astype(np.float64) @ w1 + b1, 0) @ w2 + b2
    np.testing.assert_allclose(y, want, rtol=1e-4, atol=1e-5)
