"""Pins the CPU oracle (oracle/vmref.py) before it is trusted as the checker.

Each semantic function is checked against a known answer the reference's own
tests hold (runtime_test.cc, _while_e2e_body.py, test_ops_*.py tricks) or
against an independent closed form (float64 numpy, brute-force Python loops on
tiny inputs).  The last tests plant mistakes in the oracle and require that a
pin catches each one."""
import math

import numpy as np
import pytest

import vmprogs as P
from pjrt_amd import graph as G
from pjrt_amd import scheduler as S
from pjrt_amd import vmprogram as V
from oracle import vmref

CFG = S.DeviceConfig(nlanes=4, ew_ts=256, mma_t=64)


def both(prog_or_blob, args, cfg=CFG):
    blob = prog_or_blob if isinstance(prog_or_blob, bytes) else \
        V.serialize(prog_or_blob, S.schedule_program(prog_or_blob, cfg))
    b = vmref.execute_schedule(blob, args, ew_ts=cfg.ew_ts, mma_t=cfg.mma_t)
    if vmref.parse(blob).main_len == 0:      # schedule-only blob (runtime_test.cc)
        return b
    a = vmref.execute(blob, args, ew_ts=cfg.ew_ts, mma_t=cfg.mma_t)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)
    return a


# --- reference known answers ----------------------------------------------------------

def test_runtime_test_a_two_level_ew():
    blob, args, want = P.raw_two_level_ew(256)
    (got,) = both(blob, args)
    np.testing.assert_array_equal(got, want[0])


def test_runtime_test_b_while_doubling():
    blob, args, want = P.raw_while_doubling(256)
    (got,) = both(blob, args)
    np.testing.assert_array_equal(got, want[0])


def test_runtime_test_c_region_gelu():
    blob, args, want = P.raw_region_gelu(256)
    (got,) = both(blob, args)
    assert np.max(np.abs(got - want[0])) <= 1e-5


@pytest.mark.parametrize("name", sorted(P.WHILE_CASES))
def test_while_closed_forms(name):
    prog, args, want = P.WHILE_CASES[name]()
    got = both(prog, args)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g.reshape(np.shape(w)), w)


# --- elementwise ------------------------------------------------------------------------

F64 = {
    "add": lambda a, b: a + b, "mul": lambda a, b: a * b, "sub": lambda a, b: a - b,
    "div": lambda a, b: a / b, "maximum": np.fmax, "minimum": np.fmin,
    "atan2": np.arctan2,
}


@pytest.mark.parametrize("name", sorted(F64))
def test_ew_binary_f32_closed_form(name):
    rng = np.random.default_rng(5)
    a = rng.standard_normal(1000).astype(np.float32)
    b = (rng.standard_normal(1000) + 3.0).astype(np.float32)
    g = G.Graph()
    x, y = g.input((1000,)), g.input((1000,))
    g.output(getattr(g, name)(x, y))
    (got,) = both(g.build(), [a, b])
    want = F64[name](a.astype(np.float64), b.astype(np.float64))
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-7)


UN = {"exp": np.exp, "tanh": np.tanh, "sqrt": np.sqrt, "log": np.log,
      "rsqrt": lambda x: 1 / np.sqrt(x), "abs": np.abs, "neg": np.negative,
      "floor": np.floor, "ceil": np.ceil, "sin": np.sin, "cos": np.cos,
      "log1p": np.log1p, "expm1": np.expm1, "cbrt": np.cbrt,
      "rint": np.rint, "sign": np.sign,
      "round": lambda x: np.copysign(np.where(np.abs(x) - np.floor(np.abs(x)) >= 0.5, np.floor(np.abs(x)) + 1, np.floor(np.abs(x))), x),
      "gelu": lambda x: 0.5 * x * (1 + np.tanh(0.7978845608 * (x + 0.044715 * x ** 3)))}


@pytest.mark.parametrize("name", sorted(UN))
def test_ew_unary_f32_closed_form(name):
    rng = np.random.default_rng(6)
    a = (np.abs(rng.standard_normal(777)) + 0.1).astype(np.float32)
    if name in ("rint", "round", "floor", "ceil", "sign", "neg", "abs", "gelu", "sin",
                "cos", "tanh", "expm1", "cbrt"):
        a = (a - 1.5).astype(np.float32)
    if name in ("rint", "round"):
        a = np.concatenate([a, np.array([0.5, 1.5, 2.5, -0.5, -2.5], np.float32)])
    g = G.Graph()
    x = g.input(a.shape)
    g.output(g.unary(name, x))
    (got,) = both(g.build(), [a])
    np.testing.assert_allclose(got, UN[name](a.astype(np.float64)), rtol=2e-6, atol=1e-6)


def _math_pow(a, b):
    """C pow semantics from Python's math module (an implementation independent of
    numpy): a negative base with a non-integer exponent is NaN, 0 ** negative is
    +inf (ew.cl:19-50 maps pow onto the device libm's pow)."""
    try:
        return math.pow(a, b)
    except ValueError:
        return math.nan
    except ZeroDivisionError:
        return math.inf
    except OverflowError:
        return math.copysign(math.inf, a) if (b == int(b) and int(b) % 2 and a < 0) else math.inf


def _signed_operands():
    rng = np.random.default_rng(17)
    a = (rng.standard_normal(600) * 3.0).astype(np.float32)
    b = (rng.standard_normal(600) * 2.0).astype(np.float32)
    b[::3] = rng.integers(-4, 5, b[::3].size).astype(np.float32)   # integer exponents
    b[b == 0] = 2.0
    a[a == 0] = -1.5
    # fixed cases: remainder takes the dividend's sign; pow of negative bases
    fa = np.array([-5, 5, -5, 5, -0.0, -6, 7.5, -7.5, -2, -2, -8, 0.5, -3], np.float32)
    fb = np.array([3, -3, -3, 3, 3, 3, 2, 2, 3, 2, 1 / 3, -1, 0.5], np.float32)
    return np.concatenate([fa, a]), np.concatenate([fb, b]), fa.size


def test_ew_remainder_sign_of_dividend():
    """remainder is C fmod: the result takes the dividend's sign (ew.cl:27):
    -5 % 3 = -2, 5 % -3 = 2, -0.0 % 3 = -0.0, -6 % 3 = -0.0; checked against
    math.fmod element by element, signs of zeros included."""
    a, b, nf = _signed_operands()
    g = G.Graph()
    x, y = g.input(a.shape), g.input(b.shape)
    g.output(g.remainder(x, y))
    (got,) = both(g.build(), [a, b])
    want = np.array([math.fmod(float(p), float(q)) for p, q in zip(a, b)])
    assert got[:4].tolist() == [-2.0, 2.0, -2.0, 2.0]
    assert math.copysign(1, got[4]) == -1 and math.copysign(1, got[5]) == -1
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=0)
    assert np.array_equal(np.signbit(got), np.signbit(want.astype(np.float32)))


def test_ew_pow_signed_bases():
    """pow over signed bases and integer / fractional exponents against
    math.pow: (-2)^3 = -8, (-2)^2 = 4, (-8)^(1/3) = NaN, 0.5^-1 = 2, (-3)^0.5 = NaN."""
    a, b, nf = _signed_operands()
    g = G.Graph()
    x, y = g.input(a.shape), g.input(b.shape)
    g.output(g.pow(x, y))
    (got,) = both(g.build(), [a, b])
    want = np.array([_math_pow(float(p), float(q)) for p, q in zip(a, b)])
    assert got[8] == -8.0 and got[9] == 4.0 and np.isnan(got[10]) and got[11] == 2.0 and np.isnan(got[12])
    nan_g, nan_w = np.isnan(got), np.isnan(want)
    assert np.array_equal(nan_g, nan_w)
    np.testing.assert_allclose(got[~nan_g], want[~nan_w], rtol=2e-6, atol=0)


def test_ew_tan_closed_form():
    """tan against math.tan over (-pi/2, pi/2) and a few periods out."""
    x = np.concatenate([np.linspace(-1.5, 1.5, 301), np.linspace(-20, 20, 173)]).astype(np.float32)
    g = G.Graph()
    a = g.input(x.shape)
    g.output(g.unary("tan", a))
    (got,) = both(g.build(), [x])
    want = np.array([math.tan(float(v)) for v in x])
    np.testing.assert_allclose(got, want, rtol=4e-6, atol=1e-7)


def test_rounding_modes_exact():
    a = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 0.49999997], np.float32)
    g = G.Graph()
    x = g.input(a.shape)
    g.output(g.unary("rint", x), g.unary("round", x))
    r, q = both(g.build(), [a])
    assert r.tolist() == [0, 2, 2, -0, -2, -2, 0]
    assert q.tolist() == [1, 2, 3, -1, -2, -3, 0]


def _int_brute(op, x, y, bits, signed):
    m = (1 << bits) - 1

    def s(v):
        v &= m
        return v - (1 << bits) if signed and v >> (bits - 1) else v

    out = []
    for a, b in zip(x.tolist(), y.tolist()):
        if op == "add": r = a + b
        elif op == "mul": r = a * b
        elif op == "sub": r = a - b
        elif op == "div": r = 0 if b == 0 else int(abs(a) // abs(b)) * (1 if (a < 0) == (b < 0) else -1)
        elif op == "maximum": r = max(a, b)
        elif op == "minimum": r = min(a, b)
        elif op == "bit_and": r = a & b
        elif op == "bit_or": r = a | b
        elif op == "bit_xor": r = a ^ b
        elif op == "shl": r = (a & m) << (b & (bits - 1))
        elif op == "shr_l": r = (a & m) >> (b & (bits - 1))
        elif op == "shr_a":      # sign-fill on the bit pattern, any signedness
            sa = (a & m) - (1 << bits) if (a & m) >> (bits - 1) else (a & m)
            r = sa >> (b & (bits - 1))
        out.append(s(r))
    return out


@pytest.mark.parametrize("dt", ["i32", "u32", "i64"])
@pytest.mark.parametrize("op", ["add", "mul", "sub", "div", "maximum", "minimum",
                                "bit_and", "bit_or", "bit_xor", "shl", "shr_l", "shr_a"])
def test_ew_integer_bit_exact(dt, op):
    rng = np.random.default_rng(7)
    bits = 64 if dt == "i64" else 32
    npdt = {"i32": np.int32, "u32": np.uint32, "i64": np.int64}[dt]
    info = np.iinfo(npdt)
    x = rng.integers(info.min, info.max, 300, dtype=npdt)
    y = rng.integers(info.min, info.max, 300, dtype=npdt)
    y[:20] = np.arange(20).astype(npdt)          # shift counts / div by zero
    x[20:25] = np.array([info.min, info.max, 0, 1, 7]).astype(npdt)
    g = G.Graph()
    a, b = g.input((300,), dt), g.input((300,), dt)
    g.output(getattr(g, op)(a, b))
    (got,) = both(g.build(), [x, y])
    want = _int_brute(op, x, y, bits, dt != "u32")
    assert [int(v) for v in got] == [int(v) for v in want]


def test_compare_select_convert_bool():
    a = np.array([1.0, -2.0, 3.0, np.nan, 0.0], np.float32)
    b = np.array([1.0, 2.0, -3.0, 1.0, -0.0], np.float32)
    g = G.Graph()
    x, y = g.input((5,)), g.input((5,))
    outs = [g.compare(x, y, p) for p in ("EQ", "NE", "LT", "LE", "GT", "GE")]
    sel = g.select(outs[2], x, y)
    ci = g.convert(x, "i32")
    cb = g.convert(x, "bool")
    cbf = g.convert(y, "bf16")
    fin = g.is_finite(x)
    g.output(*outs, sel, ci, cb, cbf, fin)
    got = both(g.build(), [a, b])
    with np.errstate(invalid="ignore"):
        want = [a == b, a != b, a < b, a <= b, a > b, a >= b]
    for gg, w in zip(got[:6], want):
        assert gg.tolist() == w.astype(np.uint8).tolist()
    np.testing.assert_array_equal(got[6], np.where(a < b, a, b))
    assert got[7][[0, 1, 2, 4]].tolist() == [1, -2, 3, 0]
    assert got[8].tolist() == [1, 1, 1, 1, 0]
    assert got[9].tolist() == [0x3F80, 0x4000, 0xC040, 0x3F80, 0x8000]
    assert got[10].tolist() == [1, 1, 1, 0, 1]


def test_convert_integer_widths():
    x = np.array([-1, 2**31 - 1, -2**31, 5], np.int32)
    g = G.Graph()
    a = g.input((4,), "i32")
    w = g.convert(a, "i64")
    u = g.convert(a, "u32")
    back = g.convert(w, "i32")
    g.output(w, u, back)
    w_, u_, b_ = both(g.build(), [x])
    assert w_.tolist() == [-1, 2**31 - 1, -2**31, 5]
    assert u_.tolist() == [2**32 - 1, 2**31 - 1, 2**31, 5]
    assert b_.tolist() == x.tolist()


def test_bf16_elementwise_storage():
    rng = np.random.default_rng(8)
    a = rng.standard_normal(300).astype(np.float32)
    b = rng.standard_normal(300).astype(np.float32)
    g = G.Graph()
    x, y = g.input((300,), "bf16"), g.input((300,), "bf16")
    g.output(g.add(x, y))
    (got,) = both(g.build(), [a, b])
    ab, bb = vmref.bf16_to_f32(vmref.f32_to_bf16(a)), vmref.bf16_to_f32(vmref.f32_to_bf16(b))
    assert got.dtype == np.uint16
    np.testing.assert_array_equal(got, vmref.f32_to_bf16(ab + bb))


# --- reductions ---------------------------------------------------------------------------

def test_reductions_closed_forms_and_identities():
    rng = np.random.default_rng(9)
    x = rng.standard_normal((37, 129)).astype(np.float32)
    g = G.Graph()
    a = g.input(x.shape)
    outs = [g.reduce_last(a, k) for k in (0, 1, 2)]
    full = [g.reduce_all(a, k, ew_ts=256) for k in (0, 1, 2)]
    ax0 = g.reduce_axis(a, 0, 0)
    g.output(*outs, *full, ax0)
    got = both(g.build(), [x])
    x64 = x.astype(np.float64)
    np.testing.assert_allclose(got[0], x64.sum(1), rtol=1e-5, atol=1e-5)
    np.testing.assert_array_equal(got[1], x.max(1))
    np.testing.assert_array_equal(got[2], x.min(1))
    np.testing.assert_allclose(got[3], x64.sum(), rtol=1e-5)
    assert got[4] == x.max() and got[5] == x.min()
    np.testing.assert_allclose(got[6], x64.sum(0), rtol=1e-5, atol=1e-5)
    yi = rng.integers(-100, 100, (5, 16)).astype(np.int32)
    g = G.Graph()
    a = g.input(yi.shape, "i32")
    g.output(*[g.reduce_last(a, k) for k in range(7)])
    got = both(g.build(), [yi])
    assert got[0].tolist() == yi.sum(1).tolist()
    assert got[1].tolist() == yi.max(1).tolist()
    assert got[2].tolist() == yi.min(1).tolist()
    assert got[3].tolist() == [int(np.prod(r.astype(np.int64)) & 0xFFFFFFFF) - (1 << 32 if int(np.prod(r.astype(np.int64)) & 0xFFFFFFFF) >= 1 << 31 else 0) for r in yi]
    assert got[4].tolist() == [int(np.bitwise_and.reduce(r)) for r in yi]
    assert got[5].tolist() == [int(np.bitwise_or.reduce(r)) for r in yi]
    assert got[6].tolist() == [int(np.bitwise_xor.reduce(r)) for r in yi]


def test_argmax_first_index():
    x = np.array([[1, 3, 3, 0], [5, 1, 5, 9], [-1, -1, -1, -1]], np.float32)
    g = G.Graph()
    a = g.input(x.shape)
    v, i = g.argmax_last(a)
    g.output(v, i)
    vv, ii = both(g.build(), [x])
    assert ii.tolist() == [1, 3, 0]
    assert vv.tolist() == [3, 9, -1]


# --- fused norms ---------------------------------------------------------------------

def ln_ref(x, g, b, eps):
    """Explicit two-pass formula, float64 per row."""
    out = np.empty_like(x, dtype=np.float64)
    for r in range(x.shape[0]):
        row = x[r].astype(np.float64)
        mu = sum(row) / len(row)
        var = sum((v - mu) ** 2 for v in row) / len(row)
        out[r] = (row - mu) / math.sqrt(var + eps) * g + b
    return out


def test_layernorm_affine_gelu_convert():
    rng = np.random.default_rng(10)
    x = rng.standard_normal((6, 300)).astype(np.float32)
    gam = rng.uniform(0.5, 1.5, 300).astype(np.float32)
    bet = (rng.standard_normal(300) * 0.1).astype(np.float32)
    g = G.Graph()
    a, gg, bb = g.input(x.shape), g.input((300,)), g.input((300,))
    y32 = g.layernorm(a, gg, bb, 1e-5)
    ybf = g.layernorm(a, gg, bb, 1e-5, gelu=True, out_dtype="bf16")
    g.output(y32, ybf)
    y, yb = both(g.build(), [x, gam, bet])
    ref = ln_ref(x, gam, bet, 1e-5)
    np.testing.assert_allclose(y, ref, rtol=1e-5, atol=1e-5)
    gel = UN["gelu"](ref)
    got = vmref.bf16_to_f32(yb)
    np.testing.assert_allclose(got, gel, rtol=2 ** -7, atol=1e-6)


def test_layernorm_core_one_pass_matches_reference_formula():
    rng = np.random.default_rng(11)
    x = rng.standard_normal((4, 64)).astype(np.float32)
    g = G.Graph()
    a = g.input(x.shape)
    g.output(g.layernorm_core(a, 1e-5))
    (y,) = both(g.build(), [x])
    np.testing.assert_allclose(y, ln_ref(x, 1.0, 0.0, 1e-5), rtol=1e-5, atol=1e-5)


def test_softmax_rows():
    rng = np.random.default_rng(12)
    x = rng.standard_normal((9, 50)).astype(np.float32) * 4
    g = G.Graph()
    a = g.input(x.shape)
    g.output(g.softmax_last(a))
    (y,) = both(g.build(), [x])
    for r in range(9):
        e = [math.exp(v - max(x[r])) for v in x[r].tolist()]
        np.testing.assert_allclose(y[r], np.array(e) / sum(e), rtol=2e-6)


# --- contractions ----------------------------------------------------------------------------

@pytest.mark.parametrize("M,K,N", [(1, 1, 1), (3, 4, 5), (17, 17, 17), (65, 33, 70),
                                   (130, 64, 3), (64, 64, 64)])
def test_dot_integer_valued_exact(M, K, N):
    rng = np.random.default_rng(M * 1000 + K * 10 + N)
    a = rng.integers(0, 5, (M, K)).astype(np.float32)
    b = rng.integers(0, 5, (K, N)).astype(np.float32)
    g = G.Graph()
    x, y = g.input(a.shape), g.input(b.shape)
    g.output(g.dot(x, y))
    (got,) = both(g.build(), [a, b])
    want = [[sum(int(a[i, k]) * int(b[k, j]) for k in range(K)) for j in range(N)]
            for i in range(M)]
    assert got.astype(np.int64).tolist() == want


def test_dot_views_batch_and_epilogue():
    rng = np.random.default_rng(13)
    G_, M, K, N = 3, 20, 12, 9
    a = rng.integers(-3, 4, (G_, M, K)).astype(np.float32)
    bt = rng.integers(-3, 4, (G_, N, K)).astype(np.float32)    # stored transposed
    res = rng.integers(-3, 4, (G_, M, N)).astype(np.float32)
    g = G.Graph()
    x, y, r = g.input(a.shape), g.input(bt.shape), g.input(res.shape)
    yv = g.transpose_view(y, (0, 2, 1))
    out = g.dot(x, yv, epilogue=[(V.SUB_AFFINE, 0, 2.0, 1.0), (V.SUB_ADD, 1, 0, 0)],
                residual=r)
    g.output(out)
    (got,) = both(g.build(), [a, bt, res])
    want = (np.einsum("gmk,gnk->gmn", a, bt) * 2 + 1) + res
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("M", [40, 3])
def test_dot_epilogue_constant_operand(M):
    """Epilogue source 3 (the operand is the constant s): bias, then
    min(., 6), then max(., 0.5) with t = 7 -- a clamp to [0.5, 6] written out
    by hand.  Taking t for the operand would give max(., 7) and fail.  M = 3
    schedules the skinny-matmul (GEMV) tile, M = 40 the MMA tile."""
    rng = np.random.default_rng(15)
    K, N = 24, 37
    a = rng.integers(-3, 4, (M, K)).astype(np.float32)
    b = rng.integers(-3, 4, (K, N)).astype(np.float32)
    bias = rng.integers(-4, 5, N).astype(np.float32)
    g = G.Graph()
    x, y, bb = g.input(a.shape), g.input(b.shape), g.input(bias.shape)
    g.output(g.dot(x, y, residual=bb, epilogue=[(V.SUB_ADD, 2, 0.0, 0.0), (V.SUB_MIN, 3, 6.0, 0.0),
                                                (V.SUB_MAX, 3, 0.5, 7.0)]))
    (got,) = both(g.build(), [a, b, bias])
    want = [[min(max(sum(int(a[i, k]) * int(b[k, j]) for k in range(K)) + int(bias[j]), 0.5), 6.0)
             if sum(int(a[i, k]) * int(b[k, j]) for k in range(K)) + int(bias[j]) < 6.0 else 6.0
             for j in range(N)] for i in range(M)]
    np.testing.assert_array_equal(got, np.array(want, np.float32))


def test_planted_epilogue_constant_is_caught(monkeypatch):
    orig = vmref.TaskRunner._epilogue

    def wrong(self, t, v, g, r0, r1, c0, c1, M, N, res):
        aux = list(self.m.p.aux)
        off = t.p[6] - 1
        for k in range(aux[off]):          # use t where the constant operand is s
            if aux[off + 2 + 4 * k] == 3:
                aux[off + 3 + 4 * k] = aux[off + 4 + 4 * k]
        saved = self.m.p.aux
        self.m.p.aux = aux
        try:
            return orig(self, t, v, g, r0, r1, c0, c1, M, N, res)
        finally:
            self.m.p.aux = saved

    monkeypatch.setattr(vmref.TaskRunner, "_epilogue", wrong)
    with pytest.raises(AssertionError):
        test_dot_epilogue_constant_operand(40)


def test_gemv_dot_mode():
    rng = np.random.default_rng(14)
    A = rng.integers(-4, 5, (50, 33)).astype(np.float32)
    xv = rng.integers(-4, 5, (33, 1)).astype(np.float32)
    g = G.Graph()
    a, x = g.input(A.shape), g.input(xv.shape)
    g.output(g.dot(a, x))
    prog = g.build()
    sched = S.schedule_program(prog, CFG)
    assert sched.tasks[0].tile_op == V.TOP_RED_SEG and sched.tasks[0].p3 == 1
    (got,) = both(prog, [A, xv])
    np.testing.assert_array_equal(got, A @ xv)


def attention_loops(Q, K, Vv, scale, causal):
    """Brute-force attention with Python loops (independent of einsum)."""
    H, T, hd = Q.shape
    C = K.shape[1]
    out = np.zeros((H, T, hd))
    for h in range(H):
        for m in range(T):
            s = []
            for j in range(C):
                if causal and j > m + (C - T):
                    continue
                s.append((j, scale * sum(float(Q[h, m, d]) * float(K[h, j, d]) for d in range(hd))))
            mx = max(v for _, v in s)
            w = [(j, math.exp(v - mx)) for j, v in s]
            z = sum(v for _, v in w)
            for d in range(hd):
                out[h, m, d] = sum(p * float(Vv[h, j, d]) for j, p in w) / z
    return out


@pytest.mark.parametrize("causal", [False, True])
def test_flash_attention_brute_force(causal):
    rng = np.random.default_rng(15)
    H, T, C, hd = 2, 5, 7, 4
    q = rng.standard_normal((H, T, hd)).astype(np.float32)
    k = rng.standard_normal((H, C, hd)).astype(np.float32)
    v = rng.standard_normal((H, C, hd)).astype(np.float32)
    g = G.Graph()
    Q, K, Vv = g.input(q.shape), g.input(k.shape), g.input(v.shape)
    g.output(g.flash_attention(Q, K, Vv, 0.5, causal))
    (got,) = both(g.build(), [q, k, v])
    np.testing.assert_allclose(got, attention_loops(q, k, v, 0.5, causal), rtol=1e-5, atol=1e-6)


def test_flash_attention_rows_without_keys_are_nan():
    """Causal with T > C: query m sees keys j <= m + C - T, so rows m < T - C see
    none.  The reference's kernel normalises by its running sum, 0 for such a
    row (pjrt_plugin/kernels/ops/attention.cl:153-157, run_l starts at 0 and
    only masked keys add 0), so the row is 0 * inf = NaN, as the softmax of an
    all -inf row is.  The oracle stores NaN there and matches the brute force on
    the other rows."""
    rng = np.random.default_rng(16)
    H, T, C, hd = 2, 7, 3, 4
    q = rng.standard_normal((H, T, hd)).astype(np.float32)
    k = rng.standard_normal((H, C, hd)).astype(np.float32)
    v = rng.standard_normal((H, C, hd)).astype(np.float32)
    g = G.Graph()
    Q, K, Vv = g.input(q.shape), g.input(k.shape), g.input(v.shape)
    g.output(g.flash_attention(Q, K, Vv, 0.5, True))
    with np.errstate(invalid="ignore", divide="ignore"):
        (got,) = both(g.build(), [q, k, v])
    assert np.isnan(got[:, :T - C]).all()
    want = attention_loops(q[:, T - C:], k, v, 0.5, True)    # the last C rows: query m - (T - C) of a T = C problem
    np.testing.assert_allclose(got[:, T - C:], want, rtol=1e-5, atol=1e-6)


def decode_attention_loops(q, Kt, Vc, k, v, pos, scale):
    """Brute-force decode step with Python loops: keys are the cache columns
    [0, p) then the step's own key, p = pos clamped to [0, C]."""
    H, hd, C = Kt.shape
    p = min(max(int(pos), 0), C)
    out = np.zeros((H, hd))
    for h in range(H):
        keys = [[float(Kt[h, d, j]) for d in range(hd)] for j in range(p)] + [[float(x) for x in k[h]]]
        vals = [[float(Vc[h, j, d]) for d in range(hd)] for j in range(p)] + [[float(x) for x in v[h]]]
        s = [scale * sum(float(q[h, d]) * kj[d] for d in range(hd)) for kj in keys]
        mx = max(s)
        w = [math.exp(x - mx) for x in s]
        z = sum(w)
        for d in range(hd):
            out[h, d] = sum(wj * vj[d] for wj, vj in zip(w, vals)) / z
    return out


def _decode_inputs(H=3, hd=8, C=16, seed=21):
    rng = np.random.default_rng(seed)
    return [rng.standard_normal(sh).astype(np.float32)
            for sh in ((H, hd), (H, hd), (H, hd), (H, hd, C), (H, C, hd))]


def _decode_graph(H, hd, C, scale, dt="f32"):
    g = G.Graph()
    Q, K, Vv = (g.input((H, hd), dt) for _ in range(3))
    CK, CV = g.input((H, hd, C), dt), g.input((H, C, hd), dt)
    POS = g.input((), "i32")
    g.output(g.decode_attention(Q, K, Vv, CK, CV, POS, scale))
    return g.build()


@pytest.mark.parametrize("pos", [0, 1, 9, 16, -3, 40])
def test_decode_attention_brute_force(pos):
    """Extension op OP_DECODE_ATTN: cache prefix plus the step's own key/value,
    pos clamped to [0, C] (16 = a full cache, -3 and 40 clamp)."""
    q, k, v, ckt, cv = _decode_inputs()
    args = [q, k, v, ckt, cv, np.array(pos, np.int32)]
    (got,) = both(_decode_graph(3, 8, 16, 0.35), args)
    np.testing.assert_allclose(got, decode_attention_loops(q, ckt, cv, k, v, pos, 0.35), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("krow", [False, True])
@pytest.mark.parametrize("masked", [False, True])
@pytest.mark.parametrize("pos", [0, 9, 15, 16, 40, -3])
def test_decode_attention_row_keys_and_masked_form(krow, masked, pos):
    """``krow`` reads the key cache as rows [H, C, hd] (the same keys as the
    K^T layout); ``masked`` (the decoder that stored k, v at pos first) clamps
    pos to [0, C - 1] like that store, and a negative pos leaves no key: NaN."""
    H, hd, C, scale = 3, 8, 16, 0.35
    q, k, v, ckt, cv = _decode_inputs()
    kc = np.ascontiguousarray(ckt.transpose(0, 2, 1)) if krow else ckt
    g = G.Graph()
    Q, K, Vv = (g.input((H, hd)) for _ in range(3))
    CK, CV = g.input(kc.shape), g.input((H, C, hd))
    POS = g.input((), "i32")
    g.output(g.decode_attention(Q, K, Vv, CK, CV, POS, scale, krow=krow, masked=masked))
    (got,) = both(g.build(), [q, k, v, kc, cv, np.array(pos, np.int32)])
    if masked and pos < 0:
        assert np.isnan(got).all()
        return
    p = min(max(pos, 0), C - 1 if masked else C)
    np.testing.assert_allclose(got, decode_attention_loops(q, ckt, cv, k, v, p, scale), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("pos", [0, 5, 15])
def test_decode_attention_equals_decomposed_chain(pos):
    """The fused step equals the decomposed chain of pinned ops: cache update at
    pos, then dot(q, K^T[:, :, :pos + 1]) * scale -> softmax -> dot(P, V[:, :pos + 1])."""
    H, hd, C, scale = 3, 8, 16, 0.35
    q, k, v, ckt, cv = _decode_inputs()
    args = [q, k, v, ckt, cv, np.array(pos, np.int32)]
    (fused,) = both(_decode_graph(H, hd, C, scale), args)
    g = G.Graph()
    Q, K, Vv = (g.input((H, hd)) for _ in range(3))
    CK, CV = g.input((H, hd, C)), g.input((H, C, hd))
    POS = g.input((), "i32")
    zero = g.scalar(0, "i32")
    ck, cvv = g.fill((H, hd, C), 0.0), g.fill((H, C, hd), 0.0)
    g.copy_into(ck, CK)
    g.copy_into(cvv, CV)
    g.dynamic_update_slice(ck, g.reshape(K, (H, hd, 1)), [zero, zero, POS])
    g.dynamic_update_slice(cvv, g.reshape(Vv, (H, 1, hd)), [zero, POS, zero])
    s = g.dot(g.reshape(Q, (H, 1, hd)), g.slice(ck, (0, 0, 0), (H, hd, pos + 1)),
              epilogue=[(V.SUB_AFFINE, 0, scale, 0.0)])
    o = g.dot(g.softmax_last(s), g.slice(cvv, (0, 0, 0), (H, pos + 1, hd)))
    g.output(o)
    (chain,) = both(g.build(), args)
    np.testing.assert_allclose(fused, chain.reshape(H, hd), rtol=1e-5, atol=1e-6)


def test_planted_decode_new_key_is_caught(monkeypatch):
    """An oracle that reads the cache's column pos instead of the step's own key
    and value fails the brute-force check."""
    def wrong(q, Kt, Vc, k, v, pos, scale, krow=False, masked=False):
        C = Kt.shape[2]
        p = min(max(int(pos), 0), C - 1)
        s = np.einsum("hd,hdc->hc", q.astype(np.float64), Kt[:, :, :p + 1].astype(np.float64)) * scale
        e = np.exp(s - s.max(-1, keepdims=True))
        e /= e.sum(-1, keepdims=True)
        return np.einsum("hc,hcd->hd", e, Vc[:, :p + 1].astype(np.float64))

    monkeypatch.setattr(vmref, "decode_attention", wrong)
    with pytest.raises(AssertionError):
        test_decode_attention_brute_force(9)


@pytest.mark.parametrize("M,gelu", [(1, False), (3, True)])
def test_gemv_layernorm_prologue(M, gelu):
    """A layernorm staged inside its GEMV (schedule-level fusion): the lane
    simulator's result equals the tensor interpreter's, which stores the
    layernorm result in bf16 and reads it back, and float64 math."""
    rng = np.random.default_rng(31)
    K, N = 96, 40
    x = rng.standard_normal((M, K)).astype(np.float32)
    gam = rng.uniform(0.5, 1.5, K).astype(np.float32)
    bet = rng.normal(0, 0.1, K).astype(np.float32)
    w = vmref.bf16_to_f32(vmref.f32_to_bf16(rng.standard_normal((K, N)).astype(np.float32)))
    g = G.Graph()
    X, GA, BE, W = g.input((M, K)), g.input((K,)), g.input((K,)), g.input((K, N), "bf16")
    g.output(g.dot(g.layernorm(X, GA, BE, 1e-5, gelu=gelu, out_dtype="bf16"), W))
    prog = g.build()
    cfg = S.DeviceConfig(nlanes=4, ew_ts=256, mma_t=64)
    sched = S.schedule_program(prog, cfg)
    assert any(t.tile_op == V.TOP_GEMV and t.p5 for t in sched.tasks)
    (got,) = both(prog, [x, gam, bet, w], cfg)
    mu = x.astype(np.float64).mean(1, keepdims=True)
    var = ((x - mu) ** 2).mean(1, keepdims=True)
    hn = (x - mu) / np.sqrt(var + 1e-5) * gam + bet
    if gelu:
        hn = 0.5 * hn * (1 + np.tanh(math.sqrt(2 / math.pi) * (hn + 0.044715 * hn ** 3)))
    want = vmref.bf16_to_f32(vmref.f32_to_bf16(hn.astype(np.float32))).astype(np.float64) @ w
    np.testing.assert_allclose(got, want, rtol=2e-2, atol=2e-2 * np.abs(want).max())


# --- data movement -----------------------------------------------------------------------------

def test_gather_scatter_dyn_embedding_brute_force():
    rng = np.random.default_rng(16)
    x = rng.standard_normal((4, 6, 5)).astype(np.float32)
    tab = rng.standard_normal((10, 8)).astype(np.float32)
    ids = np.array([3, 0, 9, 12, -2], np.int32)
    start = np.array(2, np.int32)
    g = G.Graph()
    a = g.input(x.shape)
    t = g.input(tab.shape)
    i = g.input(ids.shape, "i32")
    s = g.input((), "i32")
    tr = g.transpose(a, (2, 0, 1))
    sl = g.slice(a, [1, 0, 2], [4, 6, 5], [2, 3, 1])
    cat = g.concatenate([a, a], 1)
    zero = g.scalar(0, "i32")
    dyn = g.dynamic_slice(a, [s, zero, s], [2, 3, 2])
    emb = g.take_rows(t, i)
    io = g.iota((3, 4), 1, "i32")
    g.output(tr, sl, cat, dyn, emb, io)
    got = both(g.build(), [x, tab, ids, start])
    assert np.array_equal(got[0], x.transpose(2, 0, 1))
    assert np.array_equal(got[1], x[1:4:2, 0:6:3, 2:5])
    assert np.array_equal(got[2], np.concatenate([x, x], 1))
    # start 2 clamps to dim - size: axis0 4-2=2, axis2 5-2=3 -> 2
    assert np.array_equal(got[3], x[2:4, 0:3, 2:4])
    rows = [min(max(int(r), 0), 9) for r in ids]
    assert np.array_equal(got[4], tab[rows])
    assert got[5].tolist() == [[0, 1, 2, 3]] * 3


# --- planted mistakes: each pin must catch its mistake ---------------------------------------------

def test_planted_gelu_constant_is_caught(monkeypatch):
    orig = vmref.gelu_f32

    def wrong(x):
        x = np.asarray(x, np.float32)
        inner = np.float32(0.7978845608) * (x + np.float32(0.04715) * x * x * x)
        return (np.float32(0.5) * x * (1 + np.tanh(inner))).astype(np.float32)

    monkeypatch.setattr(vmref, "gelu_f32", wrong)
    with pytest.raises(AssertionError):
        test_runtime_test_c_region_gelu.__wrapped__() if hasattr(
            test_runtime_test_c_region_gelu, "__wrapped__") else _region_gelu_via_ew()
    monkeypatch.setattr(vmref, "gelu_f32", orig)


def _region_gelu_via_ew():
    x = np.linspace(-4, 4, 301).astype(np.float32)
    g = G.Graph()
    a = g.input(x.shape)
    g.output(g.gelu(a))
    (got,) = both(g.build(), [x])
    np.testing.assert_allclose(got, UN["gelu"](x.astype(np.float64)), rtol=2e-6, atol=1e-6)


def test_planted_layernorm_variance_is_caught(monkeypatch):
    def wrong(x, eps, two_pass):
        x64 = x.astype(np.float64)
        mu = x64.mean(-1, keepdims=True)
        var = ((x64 - mu) ** 2).sum(-1, keepdims=True) / (x.shape[-1] - 1)   # n-1
        return ((x64 - mu) / np.sqrt(var + eps)).astype(np.float32)

    monkeypatch.setattr(vmref, "layernorm_core", wrong)
    with pytest.raises(AssertionError):
        test_layernorm_affine_gelu_convert()


def test_planted_causal_offset_is_caught(monkeypatch):
    orig = vmref.attention

    def wrong(Q, Kb, Vb, scale, causal):
        H, T, hd = Q.shape
        C = Kb.shape[2]
        s = np.einsum("htd,hdc->htc", Q.astype(np.float64), Kb.astype(np.float64)) * scale
        if causal:
            qpos = np.arange(T)[:, None]             # drops the (C - T) offset
            s = np.where(np.arange(C)[None, :] > qpos, -np.inf, s)
        p = np.exp(s - s.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        return np.einsum("htc,hcd->htd", p, Vb.astype(np.float64)).astype(np.float32)

    monkeypatch.setattr(vmref, "attention", wrong)
    with pytest.raises(AssertionError):
        test_flash_attention_brute_force(True)
    monkeypatch.setattr(vmref, "attention", orig)


@pytest.mark.parametrize("sub,wrong_fn,pin", [
    (26, np.remainder, "test_ew_remainder_sign_of_dividend"),    # sign of the divisor
    (6, lambda x, y: np.power(np.abs(x), y), "test_ew_pow_signed_bases"),
    (32, None, "test_ew_tan_closed_form"),
])
def test_planted_float_op_is_caught(monkeypatch, sub, wrong_fn, pin):
    """A wrong remainder (np.remainder: sign of the divisor), a pow that drops the
    base's sign, and a tan that is really sin/cos of a shifted angle each fail
    their pin."""
    orig_bin, orig_un = vmref._float_bin, vmref._float_un
    if sub == 32:
        def wrong_un(s, x):
            if s == 32:
                with np.errstate(all="ignore"):
                    return (np.sin(x) / np.cos(x + np.float32(1e-3))).astype(x.dtype)
            return orig_un(s, x)
        monkeypatch.setattr(vmref, "_float_un", wrong_un)
    else:
        def wrong_bin(s, x, y):
            if s == sub:
                with np.errstate(all="ignore"):
                    return wrong_fn(x, y).astype(x.dtype)
            return orig_bin(s, x, y)
        monkeypatch.setattr(vmref, "_float_bin", wrong_bin)
    with pytest.raises(AssertionError):
        globals()[pin]()


def test_planted_shift_mask_is_caught(monkeypatch):
    orig = vmref._int_op

    def wrong(sub, x, y, dt):
        if sub == 42:
            return (x.astype(np.uint64) << (y.astype(np.uint64) & np.uint64(63))).astype(x.dtype)
        return orig(sub, x, y, dt)

    monkeypatch.setattr(vmref, "_int_op", wrong)
    with pytest.raises(AssertionError):
        test_ew_integer_bit_exact("i32", "shl")


def test_elementwise_product_bound_catches_a_planted_error():
    """The GPU tests' elementwise GEMM / attention check (|got - want| <= rtol
    |A||B| per element) passes a bf16-rounded product and fails one element
    perturbed by 2 % of its scale, including where the product cancels to ~0."""
    from gpu_util import assert_product_elementwise
    rng = np.random.default_rng(3)
    a = rng.standard_normal((32, 48))
    b = rng.standard_normal((48, 40))
    want = a @ b
    scale = np.abs(a) @ np.abs(b)
    got = V.bf16_to_f32(V.f32_to_bf16(want.astype(np.float32)))
    assert_product_elementwise(got, want, scale, 1e-2)
    i = np.unravel_index(np.argmin(np.abs(want)), want.shape)
    bad = got.astype(np.float64).copy()
    bad[i] += 0.02 * scale[i]
    with pytest.raises(AssertionError):
        assert_product_elementwise(bad, want, scale, 1e-2)
