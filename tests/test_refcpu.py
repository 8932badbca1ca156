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
