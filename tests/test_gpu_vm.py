"""GPU parity: the HIP megakernel VM (libvmrt.so, called through its C ABI) against
the CPU oracle on the same seeded inputs.

Bars: bit-exact for integer, bool, index and control
flow; rel 1e-5 for f32 elementwise / reduce (a few ulp of device libm); GEMM and
attention rel 1e-3 (f32) / 1e-2 (bf16) against float64; bf16 outputs of f32 math
within one bf16 ulp of the oracle's rounding (the device's f32 result and the
oracle's float64 one can straddle a bf16 rounding boundary); one ulp is at most
2^-7 of the value."""
import dataclasses
import sys

import numpy as np
import pytest

import vmprogs as P
from gpu_util import as_f32, assert_product_elementwise, assert_rel, attention_abs_scale, blob_for, run_both, run_gpu, runtime
from oracle import vmref
from pjrt_amd import graph as G
from pjrt_amd import vmprogram as V

pytestmark = pytest.mark.gpu

BF16_ULP = 2.0 ** -7


def test_runtime_opens_device():
    info = runtime().info
    assert info["arch"].startswith("gfx950")
    assert info["n_lanes"] >= 1 and info["max_lanes"] >= info["n_lanes"]


# --- reference known answers (runtime_test.cc:136-267) --------------------------------

def test_runtime_test_a_two_level_ew():
    blob, args, want = P.raw_two_level_ew(256)
    got, _ = run_both(blob, args, ew_ts=256, oracle=None)
    np.testing.assert_array_equal(got[0], want[0])


def test_runtime_test_b_while_doubling():
    blob, args, want = P.raw_while_doubling(256)
    got, _ = run_both(blob, args, ew_ts=256, oracle=None)
    np.testing.assert_array_equal(got[0], want[0])


def test_runtime_test_c_region_gelu():
    blob, args, want = P.raw_region_gelu(256)
    got, _ = run_both(blob, args, ew_ts=256, oracle=None)
    assert np.max(np.abs(got[0] - want[0])) <= 1e-5


@pytest.mark.parametrize("name", sorted(P.WHILE_CASES))
@pytest.mark.parametrize("nlanes", [3, 256])
def test_control_flow_closed_forms(name, nlanes):
    prog, args, want = P.WHILE_CASES[name]()
    got, _ = run_both(prog, args, nlanes=nlanes, ew_ts=256, oracle=None)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g.reshape(np.shape(w)), w)


# --- elementwise ----------------------------------------------------------------------------

BIN = ["add", "mul", "sub", "div", "maximum", "minimum", "pow", "atan2", "remainder"]
UN = ["copy", "neg", "exp", "log", "sqrt", "rsqrt", "tanh", "abs", "floor", "ceil", "sign", "log1p",
      "expm1", "cbrt", "sin", "cos", "tan", "rint", "round", "gelu"]


@pytest.mark.parametrize("signed", [False, True])
@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("n", [1, 1000, 70001])
def test_ew_float_ops(dt, n, signed):
    """Every float EW op; the signed variant draws negative operands and integer
    exponents too, so remainder's sign-of-dividend rule (C fmod), pow of negative
    bases and the NaN domains of log / sqrt / rsqrt are compared (NaN == NaN)."""
    rng = np.random.default_rng(11)
    if signed:
        a = (rng.standard_normal(n) * 3.0).astype(np.float32)
        b = (rng.standard_normal(n) * 2.0).astype(np.float32)
        b[::3] = rng.integers(-4, 5, b[::3].size).astype(np.float32)
        a[a == 0] = -1.5
        b[b == 0] = 2.0
        if n >= 8:
            a[:8] = [-5, 5, -5, 5, -6, -2, -2, -8]
            b[:8] = [3, -3, -3, 3, 3, 3, 2, 0.5]
    else:
        a = (np.abs(rng.standard_normal(n)) + 0.25).astype(np.float32)
        b = (np.abs(rng.standard_normal(n)) + 0.5).astype(np.float32)
    g = G.Graph()
    x, y = g.input((n,), dt), g.input((n,), dt)
    outs = [getattr(g, op)(x, y) for op in BIN] + [g.unary(op, x) for op in UN]
    outs.append(g.affine(x, 1.5, -0.25))
    g.output(*outs)
    got, want = run_both(g.build(), [a, b], ew_ts=1024)
    for k, (gv, wv) in enumerate(zip(got, want)):
        tol = BF16_ULP if dt == "bf16" else 4e-6
        assert_rel(as_f32(gv, V.DT_BY_NAME[dt]), as_f32(wv, V.DT_BY_NAME[dt]), tol, 1e-6, f"{dt} op {k}")


@pytest.mark.parametrize("dt", ["i32", "u32", "i64"])
def test_ew_integer_ops_bit_exact(dt):
    rng = np.random.default_rng(12)
    n = 5003
    npdt = V.DT_NUMPY[V.DT_BY_NAME[dt]]
    info = np.iinfo(npdt)
    a = rng.integers(info.min // 2, info.max // 2, n, dtype=np.int64).astype(npdt)
    b = rng.integers(-70, 70, n).astype(npdt)
    b[::7] = 0
    g = G.Graph()
    x, y = g.input((n,), dt), g.input((n,), dt)
    outs = [g.add(x, y), g.sub(x, y), g.mul(x, y), g.div(x, y), g.maximum(x, y), g.minimum(x, y),
            g.bit_and(x, y), g.bit_or(x, y), g.bit_xor(x, y), g.shl(x, y), g.shr_l(x, y), g.shr_a(x, y),
            g.unary("neg", x), g.unary("abs", x), g.unary("sign", x), g.unary("not", x)]
    g.output(*outs)
    got, want = run_both(g.build(), [a, b], ew_ts=512)
    for k, (gv, wv) in enumerate(zip(got, want)):
        np.testing.assert_array_equal(gv, wv, err_msg=f"{dt} op {k}")


def test_compare_select_convert_bitcast_isfinite():
    rng = np.random.default_rng(13)
    n = 4099
    a = rng.standard_normal(n).astype(np.float32) * 3e9
    a[::11] = np.nan
    a[::13] = np.inf
    b = rng.standard_normal(n).astype(np.float32)
    g = G.Graph()
    x, y = g.input((n,)), g.input((n,))
    outs = []
    for pred in ("EQ", "NE", "LT", "LE", "GT", "GE"):
        outs.append(g.compare(x, y, pred))
    c = g.compare(x, y, "GT")
    outs.append(g.select(c, x, y))
    for dt in ("i32", "u32", "i64", "bf16", "f16", "bool", "f64"):
        outs.append(g.convert(x, dt))
    outs.append(g.bitcast(x, "i32"))
    outs.append(g.is_finite(x))
    i = g.convert(y, "i32")
    outs.append(g.convert(i, "i64"))
    outs.append(g.convert(g.convert(i, "i64"), "u32"))
    g.output(*outs)
    got, want = run_both(g.build(), [a, b], ew_ts=256)
    for k, (gv, wv) in enumerate(zip(got, want)):
        np.testing.assert_array_equal(gv.view(np.uint8), wv.view(np.uint8), err_msg=f"output {k}")


@pytest.mark.parametrize("ew_ts", [256, 64])
def test_convert_between_float_types(ew_ts):
    """f32 / bf16 / f16 to one another (four elements a step, ragged tail one at a
    time), bit-exact with the oracle: NaN, Inf, -0, f16 overflow and f16 denormals
    in the f32 input, every bit pattern class (signalling NaNs too) in the 16-bit
    inputs."""
    rng = np.random.default_rng(14)
    n = 4099
    a = (rng.standard_normal(n) * 100).astype(np.float32)
    a[::11] = np.nan
    a[::13] = -np.inf
    a[::17] = 7.0e4
    a[::19] = 3.0e-6
    a[::23] = -0.0
    hb = rng.integers(0, 2 ** 16, n, dtype=np.uint64).astype(np.uint16)
    hf = rng.integers(0, 2 ** 16, n, dtype=np.uint64).astype(np.uint16).view(np.float16)
    g = G.Graph()
    x, xb, xf = g.input((n,)), g.input((n,), "bf16"), g.input((n,), "f16")
    g.output(g.convert(x, "bf16"), g.convert(x, "f16"), g.convert(xb, "f32"), g.convert(xb, "f16"),
             g.convert(xf, "f32"), g.convert(xf, "bf16"))
    ins = [a.view(np.uint32)] * 2 + [hb] * 2 + [hf.view(np.uint16)] * 2
    got, want = run_both(g.build(), [a, hb, hf], ew_ts=ew_ts)
    bad = {}
    for k, (gv, wv) in enumerate(zip(got, want)):
        u = np.uint16 if gv.itemsize == 2 else np.uint32
        gb, wb = gv.view(u), wv.view(u)
        idx = np.nonzero(gb != wb)[0]
        if idx.size:
            bad[k] = (idx.size, [(hex(int(ins[k][i])), hex(int(gb[i])), hex(int(wb[i]))) for i in idx[:4]])
    assert not bad, bad


@pytest.mark.parametrize("ew_ts", [256, 64])
def test_ew_viewed_operands(ew_ts):
    """f32 elementwise ops reading views in place, against the oracle: a
    transposed view and a middle-axis broadcast (per-element path, decoded
    index maps), row and matrix broadcasts with source offsets that are
    multiples of four (16-byte periodic path) and one that is not (per-element
    again)."""
    rng = np.random.default_rng(15)
    A, B, C = 7, 33, 20
    at = rng.standard_normal((C, B, A)).astype(np.float32)
    xp = rng.standard_normal((A, B, C)).astype(np.float32)
    bias = rng.standard_normal(B).astype(np.float32)
    row = rng.standard_normal(C + 2).astype(np.float32)
    mat = rng.standard_normal(B * C + 4).astype(np.float32)
    g = G.Graph()
    xt, xc, bb, rr, mm = g.input((C, B, A)), g.input((A, B, C)), g.input((B,)), g.input((C + 2,)), g.input((B * C + 4,))
    x = g.transpose_view(xt, (2, 1, 0))                        # [A,B,C] view of [C,B,A]
    y = g.broadcast_view(bb, (A, B, C), (1,))
    r0 = g.view(rr, (A, B, C), (0, 0, 1))                      # row broadcast, P = C
    m4 = g.view(mm, (A, B, C), (0, C, 1), 4)                   # matrix broadcast, P = B*C, offset 4
    r2 = g.view(rr, (A, B, C), (0, 0, 1), 2)                   # offset 2: not 16-byte aligned
    g.output(g.add(x, y), g.mul(y, x), g.sub(x, y), g.unary("exp", x), g.unary("tanh", y),
             g.add(xc, r0), g.mul(m4, xc), g.sub(r0, m4), g.maximum(xc, r2), g.div(r2, r0), g.minimum(m4, xc))
    got, want = run_both(g.build(), [at, xp, bias, row, mat], ew_ts=ew_ts)
    for k, (gv, wv) in enumerate(zip(got, want)):
        assert_rel(gv, wv, 4e-6, 1e-6, f"op {k}")


def test_convert_f32_to_bf16_bit_patterns():
    """f32 -> bf16 rounds to nearest even, bit-exact with the closed-form rule
    (u + 0x7fff + ((u >> 16) & 1)) >> 16 (vm_common.cl:66-70), NaN kept a quiet NaN,
    over 2^24 random patterns plus ties, boundaries and specials."""
    rng = np.random.default_rng(7)
    u = rng.integers(0, 2 ** 32, 2 ** 24, dtype=np.uint64).astype(np.uint32)
    hi = rng.integers(0, 2 ** 16, 4096, dtype=np.uint64).astype(np.uint32) << 16
    ties = np.concatenate([hi | 0x8000, hi | 0x7FFF, hi | 0x8001, hi | 0xFFFF, hi])
    specials = np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x7F800001, 0x7FC00000, 0xFFFFFFFF,
                         0x7FFFFFFF, 0x00000001, 0x007FFFFF, 0x3F808000, 0x3F818000, 0x7F7FFFFF,
                         0x7F7F8000, 0xFF7FFFFF, 0x00008000, 0x80008000], np.uint32)
    bits = np.concatenate([u, ties, specials])
    x = bits.view(np.float32)
    g = G.Graph()
    xi = g.input(x.shape)
    g.output(g.convert(xi, "bf16"))
    got, _ = run_both(g.build(), [x], oracle=None)
    want = vmref.f32_to_bf16(x)
    bad = np.nonzero(got[0] != want)[0]
    assert bad.size == 0, [(hex(int(bits[i])), hex(int(got[0][i])), hex(int(want[i]))) for i in bad[:8]]


# --- reductions and row ops ------------------------------------------------------------------

@pytest.mark.parametrize("kind", [0, 1, 2, 3])
def test_float_reductions(kind):
    rng = np.random.default_rng(20 + kind)
    a = (rng.standard_normal((37, 1000)) * (0.01 if kind == 3 else 1.0) + (1.0 if kind == 3 else 0.0))
    a = a.astype(np.float32)
    g = G.Graph()
    x = g.input(a.shape)
    g.output(g.reduce_all(x, kind, ew_ts=1024), g.reduce_last(x, kind), g.reduce_axis(x, 0, kind))
    got, want = run_both(g.build(), [a], ew_ts=1024)
    for k, (gv, wv) in enumerate(zip(got, want)):
        assert_rel(gv, wv, 1e-5 if kind != 3 else 1e-4, 1e-5, f"kind {kind} out {k}")


@pytest.mark.parametrize("dt", ["i32", "u32", "i64", "bool"])
@pytest.mark.parametrize("kind", [0, 1, 2, 3, 4, 5, 6])
def test_integer_reductions_bit_exact(dt, kind):
    rng = np.random.default_rng(30 + kind)
    npdt = V.DT_NUMPY[V.DT_BY_NAME[dt]]
    if dt == "bool":
        a = (rng.random((9, 700)) < 0.5).astype(np.uint8)
    else:
        a = rng.integers(-5 if dt != "u32" else 0, 6, (9, 700)).astype(npdt)
    g = G.Graph()
    x = g.input(a.shape, dt)
    g.output(g.reduce_all(x, kind, ew_ts=512), g.reduce_last(x, kind), g.reduce_axis(x, 0, kind))
    got, want = run_both(g.build(), [a], ew_ts=512)
    for k, (gv, wv) in enumerate(zip(got, want)):
        np.testing.assert_array_equal(gv, wv, err_msg=f"{dt} kind {kind} out {k}")


@pytest.mark.parametrize("rows,seg", [(33, 513), (7, 516), (5, 32000)])
def test_argmax_rows(rows, seg):
    """First index of the row maximum, a NaN winning (its first index); f32 rows
    of a multiple of 4 take the 16-byte-load path; rows of 8192 or more are split
    over CUs and combined by the last split."""
    rng = np.random.default_rng(40)
    a = rng.standard_normal((rows, seg)).astype(np.float32)
    a[3, 100] = a[3].max() + 1
    a[3, 200] = a[3, 100]          # tie: first index wins
    a[4, seg - 1] = a[4].max() + 1
    a[4, seg // 2 + 1] = a[4, seg - 1]   # tie across threads' ranges
    a[1, seg - 2] = np.nan
    a[1, seg - 1] = np.nan
    g = G.Graph()
    x = g.input(a.shape)
    val, idx = g.argmax_last(x)
    g.output(val, idx)
    blob, _ = blob_for(g.build())
    splits = next(tk.p[3] for tk in vmref.parse(blob).tasks if tk.top == V.TOP_ARGMAX_SEG)
    assert (splits > 1) == (seg >= 8192), splits
    for _ in range(2):                  # split rows: the arrival counters reset themselves
        got, want = run_both(blob, [a])
        np.testing.assert_array_equal(got[1], want[1])
        np.testing.assert_array_equal(got[0].view(np.uint32), want[0].view(np.uint32))


@pytest.mark.parametrize("seg", [96, 768, 1000, 4096, 8192])
def test_softmax_and_layernorm_rows(seg):
    rng = np.random.default_rng(50)
    rows = 61
    a = (rng.standard_normal((rows, seg)) * 2 + 0.5).astype(np.float32)
    g = G.Graph()
    x = g.input(a.shape)
    g.output(g.softmax_last(x), g.layernorm_core(x, 1e-5))
    got, want = run_both(g.build(), [a])
    assert_rel(got[0], want[0], 2e-5, 1e-9, "softmax")
    assert_rel(got[1], want[1], 1e-5, 2e-5, "layernorm core")


@pytest.mark.parametrize("in_dt", ["f32", "bf16"])
@pytest.mark.parametrize("out_dt", ["f32", "bf16"])
def test_fused_layernorm_affine_gelu(in_dt, out_dt):
    rng = np.random.default_rng(1002)
    rows, d = 64, 4096
    x_np = rng.standard_normal((rows, d)).astype(np.float32)
    gamma = rng.uniform(0.5, 1.5, d).astype(np.float32)
    beta = (rng.standard_normal(d) * 0.1).astype(np.float32)
    g = G.Graph()
    x = g.input((rows, d), in_dt)
    ga, be = g.input((d,)), g.input((d,))
    g.output(g.layernorm(x, ga, be, 1e-5, gelu=True, out_dtype=out_dt))
    got, want = run_both(g.build(), [x_np, gamma, beta])
    odt = V.DT_BY_NAME[out_dt]
    assert_rel(as_f32(got[0], odt), as_f32(want[0], odt), BF16_ULP if out_dt == "bf16" else 1e-5, 1e-5, "ln")


@pytest.mark.parametrize("d,in_dt", [(100, "f32"), (6000, "f32"), (768, "f16"), (768, "f32")])
def test_layernorm_row_interleave(d, in_dt):
    """Rows a multiple of the lane count: the scheduler interleaves the lanes'
    rows (task p5) and every row kernel (streaming, per-wave, per-block,
    generic) honours it."""
    rng = np.random.default_rng(1003)
    rows = 2 * runtime().info["n_lanes"]
    x_np = rng.standard_normal((rows, d)).astype(np.float32)
    gamma = rng.uniform(0.5, 1.5, d).astype(np.float32)
    beta = (rng.standard_normal(d) * 0.1).astype(np.float32)
    g = G.Graph()
    x = g.input((rows, d), in_dt)
    ga, be = g.input((d,)), g.input((d,))
    g.output(g.layernorm(x, ga, be, 1e-5, gelu=True, out_dtype="bf16"))
    blob, _ = blob_for(g.build())
    assert any(tk.top == V.TOP_LAYERNORM_SEG and tk.p[5] == 2 for tk in vmref.parse(blob).tasks)
    got, want = run_both(blob, [x_np, gamma, beta])
    assert_rel(as_f32(got[0], V.DT_BF16), as_f32(want[0], V.DT_BF16), BF16_ULP, 1e-5, "ln")


@pytest.mark.parametrize("d", [1024, 2048, 4096])
@pytest.mark.parametrize("out_dt,gelu", [("bf16", True), ("f32", False)])
@pytest.mark.parametrize("per_lane", [1, 9])
def test_layernorm_streamed_rows(d, out_dt, gelu, per_lane):
    """f32 rows of 1024 / 2048 / 4096 through the streaming row kernel (three
    or two rotating register buffers per wave): lanes with a few rows (some
    waves with none) and with nine and a ragged tail (several buffer rotations,
    the prefetch re-reading the last row past the end), against the oracle."""
    rng = np.random.default_rng(1004 + d + per_lane)
    lanes = runtime().info["n_lanes"]
    rows = per_lane * lanes + 5
    x_np = (rng.standard_normal((rows, d)) * 1.5 + 0.25).astype(np.float32)
    gamma = rng.uniform(0.5, 1.5, d).astype(np.float32)
    beta = (rng.standard_normal(d) * 0.1).astype(np.float32)
    g = G.Graph()
    x = g.input((rows, d))
    ga, be = g.input((d,)), g.input((d,))
    g.output(g.layernorm(x, ga, be, 1e-5, gelu=gelu, out_dtype=out_dt))
    got, want = run_both(g.build(), [x_np, gamma, beta])
    odt = V.DT_BY_NAME[out_dt]
    assert_rel(as_f32(got[0], odt), as_f32(want[0], odt), BF16_ULP if out_dt == "bf16" else 1e-5, 1e-5, "ln")


def test_config2_full_size_layernorm_gelu_bf16():
    """Config 2 at its real shape [8192, 4096] (seed 1002)."""
    rng = np.random.default_rng(1002)
    rows, d = 8192, 4096
    x_np = rng.standard_normal((rows, d), dtype=np.float32)
    gamma = rng.uniform(0.5, 1.5, d).astype(np.float32)
    beta = (rng.standard_normal(d) * 0.1).astype(np.float32)
    g = G.Graph()
    x = g.input((rows, d))
    ga, be = g.input((d,)), g.input((d,))
    g.output(g.layernorm(x, ga, be, 1e-5, gelu=True, out_dtype="bf16"))
    got, _ = run_both(g.build(), [x_np, gamma, beta], oracle=None)
    x64 = x_np.astype(np.float64)
    mu = x64.mean(1, keepdims=True)
    var = ((x64 - mu) ** 2).mean(1, keepdims=True)
    z = (x64 - mu) / np.sqrt(var + 1e-5) * gamma + beta
    want = 0.5 * z * (1 + np.tanh(0.7978845608 * (z + 0.044715 * z ** 3)))
    assert_rel(vmref.bf16_to_f32(got[0]), want, BF16_ULP, 1e-6, "config 2")


# --- data movement ---------------------------------------------------------------------------

def test_gather_scatter_iota_dyn_embedding():
    rng = np.random.default_rng(60)
    a = rng.standard_normal((6, 7, 5)).astype(np.float32)
    table = rng.standard_normal((50, 16)).astype(np.float32)
    ids = np.array([3, 0, 49, 77, -4, 12], np.int32)
    start = np.array([2], np.int32)
    g = G.Graph()
    x = g.input(a.shape)
    tb = g.input(table.shape)
    ix = g.input(ids.shape, "i32")
    st = g.input((1,), "i32")
    outs = [g.transpose(x, (2, 0, 1)), g.slice(x, (1, 2, 0), (5, 7, 5), (2, 1, 2)),
            g.broadcast(g.slice(x, (0, 0, 0), (1, 7, 5)), (3, 7, 5), (0, 1, 2)),
            g.concatenate([x, g.slice(x, (0, 0, 0), (2, 7, 5))], 0),
            g.iota((4, 9, 3), 1, "i32"), g.iota((5, 6), 0, "f32"),
            g.take_rows(tb, ix)]
    s0 = g.reshape(st, ())
    zero = g.const(np.array(0, np.int32))
    outs.append(g.dynamic_slice(x, [s0, zero, zero], (3, 7, 5)))
    buf = g.unary("copy", x)
    g.dynamic_update_slice(buf, g.slice(x, (0, 0, 0), (1, 7, 5)), [s0, zero, zero])
    outs.append(buf)
    g.output(*outs)
    got, want = run_both(g.build(), [a, table, ids, start], ew_ts=64)
    for k, (gv, wv) in enumerate(zip(got, want)):
        np.testing.assert_array_equal(gv, wv, err_msg=f"output {k}")


@pytest.mark.parametrize("ew_ts", [64, 4096])
def test_gather_scatter_16_byte_runs(ew_ts):
    """Views whose innermost axis is contiguous move 16-byte runs (four loads in
    flight per thread): a transpose keeping the inner axis, row slices (one
    contiguous run), an inner slice at a 16-byte offset, a broadcast, concat
    pieces (scatters), in f32, bf16, bool and i64; an inner slice at an odd
    offset takes the element path.  Bit-exact against the oracle, tiles cut
    inside rows (ew_ts 64)."""
    rng = np.random.default_rng(61)
    a = rng.standard_normal((6, 10, 8)).astype(np.float32)
    b = rng.standard_normal((4, 6, 16)).astype(np.float32)
    c = rng.integers(0, 2, (3, 5, 32)).astype(V.DT_NUMPY[V.DT_BOOL])
    e = rng.integers(-2 ** 40, 2 ** 40, (4, 3, 6)).astype(np.int64)
    g = G.Graph()
    x, y, z, w = g.input(a.shape), g.input(b.shape, "bf16"), g.input(c.shape, "bool"), g.input(e.shape, "i64")
    outs = [g.transpose(x, (1, 0, 2)), g.slice(x, (2, 0, 0), (5, 10, 8)), g.slice(x, (0, 0, 4), (6, 10, 8)),
            g.slice(x, (0, 0, 1), (6, 10, 5)), g.broadcast(g.slice(x, (0, 0, 0), (1, 10, 8)), (3, 10, 8), (0, 1, 2)),
            g.concatenate([x, g.slice(x, (0, 0, 0), (6, 3, 8))], 1), g.transpose(y, (1, 0, 2)),
            g.concatenate([y, y], 2), g.transpose(z, (1, 0, 2)), g.slice(z, (1, 0, 16), (3, 5, 32)),
            g.transpose(w, (1, 0, 2))]
    g.output(*outs)
    got, want = run_both(g.build(), [a, V.f32_to_bf16(b), c, e], ew_ts=ew_ts)
    for k, (gv, wv) in enumerate(zip(got, want)):
        np.testing.assert_array_equal(gv, wv, err_msg=f"output {k}")
    np.testing.assert_array_equal(got[0], a.transpose(1, 0, 2))
    np.testing.assert_array_equal(got[5], np.concatenate([a, a[:, :3]], 1))
    np.testing.assert_array_equal(got[8], c.transpose(1, 0, 2))
    np.testing.assert_array_equal(got[10], e.transpose(1, 0, 2))


@pytest.mark.parametrize("ew_ts", [64, 4096])
def test_gather_and_dynamic_slice_row_runs(ew_ts):
    """The 16-byte row-run paths of take_rows (OP_GATHER_INDEX) and dynamic
    slice / update slice: bf16 rows of 768 and f32 rows of 16 with ids past both
    ends (clamped), a dynamic slice and update at a row start (aligned runs),
    and at a column offset of 3 (not 16-byte aligned: the element path).
    Bit-exact against the oracle, tiles cut inside rows at ew_ts 64."""
    rng = np.random.default_rng(62)
    tb16 = V.f32_to_bf16(rng.standard_normal((40, 768)).astype(np.float32))
    tb32 = rng.standard_normal((30, 16)).astype(np.float32)
    ids = np.array([5, 0, 39, 77, -3, 12, 30, 1], np.int32)
    cache = V.f32_to_bf16(rng.standard_normal((4, 48, 64)).astype(np.float32))
    upd = V.f32_to_bf16(rng.standard_normal((4, 8, 64)).astype(np.float32))
    small = rng.standard_normal((3, 5, 8)).astype(np.float32)
    pos = np.array([17], np.int32)
    g = G.Graph()
    t16, t32 = g.input(tb16.shape, "bf16"), g.input(tb32.shape)
    ix = g.input(ids.shape, "i32")
    cv, uv = g.input(cache.shape, "bf16"), g.input(upd.shape, "bf16")
    sm = g.input(small.shape)
    ps = g.reshape(g.input((1,), "i32"), ())
    zero = g.const(np.array(0, np.int32))
    three = g.const(np.array(3, np.int32))
    outs = [g.take_rows(t16, ix), g.take_rows(t32, ix),
            g.dynamic_slice(cv, [zero, ps, zero], (4, 8, 64)),          # row runs
            g.dynamic_slice(sm, [zero, zero, three], (3, 5, 4))]        # column offset 3: element path
    c1 = g.unary("copy", cv)
    g.dynamic_update_slice(c1, uv, [zero, ps, zero])                    # row runs (scatter)
    c2 = g.unary("copy", sm)
    g.dynamic_update_slice(c2, g.slice(sm, (0, 0, 0), (3, 5, 4)), [zero, zero, three])
    outs += [c1, c2]
    g.output(*outs)
    got, want = run_both(g.build(), [tb16, tb32, ids, cache, upd, small, pos], ew_ts=ew_ts)
    for k, (gv, wv) in enumerate(zip(got, want)):
        np.testing.assert_array_equal(gv, wv, err_msg=f"output {k}")
    clip = np.clip(ids, 0, None)
    np.testing.assert_array_equal(got[0], tb16[np.minimum(clip, 39)])
    np.testing.assert_array_equal(got[2], cache[:, 17:25])
    want_c1 = cache.copy()
    want_c1[:, 17:25] = upd
    np.testing.assert_array_equal(got[4], want_c1)


# --- matmul --------------------------------------------------------------------------------------

@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("M,K,N,tile", [(64, 64, 64, 64), (100, 37, 130, 64), (256, 96, 256, 128),
                                        (300, 200, 260, 256), (1, 768, 2304, 64)])
def test_dot_integer_valued_exact(dt, M, K, N, tile):
    """Small-integer operands: every product and partial sum is exact in f32, so the
    result is exact (the reference's own trick, tests/test_ops_dot.py:1-20)."""
    rng = np.random.default_rng(70)
    a = rng.integers(-3, 4, (M, K)).astype(np.float32)
    b = rng.integers(-3, 4, (K, N)).astype(np.float32)
    g = G.Graph()
    x, y = g.input((M, K), dt), g.input((K, N), dt)
    g.output(g.dot(x, y, tile=tile))
    got, want = run_both(g.build(), [a, b])
    np.testing.assert_array_equal(got[0], a.astype(np.float64) @ b.astype(np.float64))


@pytest.mark.parametrize("dt,rtol", [("f32", 1e-3), ("bf16", 1e-2)])
def test_dot_random_tolerance_and_tiles(dt, rtol):
    rng = np.random.default_rng(1003)
    M, K, N = 512, 384, 640
    a = (rng.standard_normal((M, K)) * 0.125).astype(np.float32)
    b = (rng.standard_normal((K, N)) * 0.125).astype(np.float32)
    if dt == "bf16":
        a, b = vmref.bf16_to_f32(vmref.f32_to_bf16(a)), vmref.bf16_to_f32(vmref.f32_to_bf16(b))
    want = a.astype(np.float64) @ b.astype(np.float64)
    for tile in (64, 128, 256):
        g = G.Graph()
        x, y = g.input((M, K), dt), g.input((K, N), dt)
        g.output(g.dot(x, y, tile=tile))
        got, _ = run_both(g.build(), [a, b], oracle=None)
        err = np.abs(got[0] - want).max() / np.abs(want).max()
        assert err <= rtol, (tile, err)
        assert_product_elementwise(got[0], want, np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64), rtol,
                                   f"{dt} tile {tile}")


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("Gb,M,K,N", [(1, 512, 320, 768), (1, 1024, 128, 2048), (2, 256, 192, 1024),
                                      (1, 256, 64, 512)])
def test_dot_fast_path_exact(dt, Gb, M, K, N):
    """256 x 256 output tiles (the MFMA fast paths: 16-bit operands in K slabs of
    64, f32 in slabs of 16; 1024 x 2048 also takes the XCD tile swizzle, Gb=2 the
    batch offsets, K=64 a single 16-bit slab): integer-valued operands give the
    exact f32 result."""
    rng = np.random.default_rng(72)
    a = rng.integers(-3, 4, (Gb, M, K)).astype(np.float32)
    b = rng.integers(-3, 4, (Gb, K, N)).astype(np.float32)
    g = G.Graph()
    x, y = g.input(a.shape, dt), g.input(b.shape, dt)
    g.output(g.dot(x, y, tile=256))
    got, _ = run_both(g.build(), [a, b], oracle=None)
    np.testing.assert_array_equal(got[0], np.matmul(a.astype(np.float64), b.astype(np.float64)))


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("Gb,M,K,N", [(1, 300, 200, 264), (1, 256, 72, 512), (1, 512, 40, 256), (2, 130, 136, 520),
                                      (1, 9, 8, 8), (1, 777, 1000, 1032), (1, 100, 36, 132)])
def test_dot_fast_path_ragged_exact(dt, Gb, M, K, N):
    """The fast paths on ragged shapes (256 x 256 tiles with M or N not a multiple
    of 256, or K not a multiple of the slab; 16-bit with K and N multiples of 8,
    f32 with multiples of 4): edge rows and columns read clamped addresses and are
    not stored, the k past K are zeroed (in LDS for 16-bit, in registers for f32).
    K = 40 and 8 are one short 16-bit slab, 72 two slabs, 200 and 136 several with
    a tail, 1000 sixteen; 100 x 36 x 132 takes the f32 ragged tile and the 16-bit
    general one.  Integer-valued operands give the exact product, twice in a row."""
    rng = np.random.default_rng(77)
    a = rng.integers(-3, 4, (Gb, M, K)).astype(np.float32)
    b = rng.integers(-3, 4, (Gb, K, N)).astype(np.float32)
    g = G.Graph()
    x, y = g.input(a.shape, dt), g.input(b.shape, dt)
    g.output(g.dot(x, y, tile=256))
    blob, _ = blob_for(g.build())
    print(f"[gpu] case: ragged fast path {dt} G={Gb} M={M} K={K} N={N}", file=sys.stderr, flush=True)
    want = np.matmul(a.astype(np.float64), b.astype(np.float64))
    for _ in range(2):
        got = run_gpu(blob, [a, b])
        np.testing.assert_array_equal(got[0], want)


def test_dot_fast_path_ragged_epilogue():
    """A ragged fast-path tile with a fused epilogue (affine, + residual, GELU) and
    a bf16 output, against the oracle: the residual is read only inside the
    output."""
    rng = np.random.default_rng(78)
    M, K, N = 300, 200, 264
    a = rng.integers(-2, 3, (M, K)).astype(np.float32)
    b = rng.integers(-2, 3, (K, N)).astype(np.float32)
    res = (rng.standard_normal((M, N)) * 2).astype(np.float32)
    g = G.Graph()
    x, y, r = g.input(a.shape, "bf16"), g.input(b.shape, "bf16"), g.input(res.shape)
    g.output(g.dot(x, y, out_dtype="bf16", tile=256, residual=r,
                   epilogue=[(V.SUB_AFFINE, 0, 0.125, -0.5), (V.SUB_ADD, 1, 0.0, 0.0), (V.SUB_GELU, 0, 0.0, 0.0)]))
    got, want = run_both(g.build(), [a, b, res], oracle="tensor")
    assert_rel(as_f32(got[0], V.DT_BF16), as_f32(want[0], V.DT_BF16), BF16_ULP, 1e-6, "ragged fast epilogue")


@pytest.mark.parametrize("in_dt,out_dt", [("bf16", "bf16"), ("f32", "f32"), ("f32", "bf16")])
def test_dot_fast_path_epilogue(in_dt, out_dt):
    """Fast paths with a fused store epilogue (affine, + residual, GELU), against
    the oracle (one bf16 ulp for a bf16 output, rel 1e-5 for f32)."""
    rng = np.random.default_rng(73)
    M, K, N = 512, 256, 512
    a = rng.integers(-2, 3, (M, K)).astype(np.float32)
    b = rng.integers(-2, 3, (K, N)).astype(np.float32)
    res = (rng.standard_normal((M, N)) * 2).astype(np.float32)
    g = G.Graph()
    x, y, r = g.input(a.shape, in_dt), g.input(b.shape, in_dt), g.input(res.shape)
    g.output(g.dot(x, y, out_dtype=out_dt, tile=256, residual=r,
                   epilogue=[(V.SUB_AFFINE, 0, 0.125, -0.5), (V.SUB_ADD, 1, 0.0, 0.0), (V.SUB_GELU, 0, 0.0, 0.0)]))
    got, want = run_both(g.build(), [a, b, res], oracle="tensor")
    odt = V.DT_BY_NAME[out_dt]
    assert_rel(as_f32(got[0], odt), as_f32(want[0], odt), BF16_ULP if out_dt == "bf16" else 1e-5, 1e-6, "fast epilogue")


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("Gb,M,K,N", [(1, 256, 512, 64), (2, 100, 300, 70), (1, 64, 1000, 128), (1, 256, 128, 512)])
def test_dot_split_k_exact(dt, Gb, M, K, N):
    """K-split matmul tiles (few output tiles, deep K; K = 300 leaves the last
    split short, or empty): each split publishes its partial tile, the last to
    arrive sums them in split order and applies the bias + relu epilogue.
    Integer-valued operands give the exact product; the program runs twice, so the
    second run finds the arrival counters reset."""
    rng = np.random.default_rng(74)
    a = rng.integers(-3, 4, (Gb, M, K)).astype(np.float32)
    b = rng.integers(-3, 4, (Gb, K, N)).astype(np.float32)
    bias = rng.integers(-9, 10, N).astype(np.float32)
    g = G.Graph()
    x, y, bb = g.input(a.shape, dt), g.input(b.shape, dt), g.input(bias.shape)
    g.output(g.dot(x, y, residual=bb, epilogue=[(V.SUB_ADD, 2, 0.0, 0.0), (V.SUB_MAX, 3, 0.0, 0.0)]))
    blob, cfg = blob_for(g.build())
    task = vmref.parse(blob).tasks[0]
    assert task.top == V.TOP_MMA and task.p[3] >> V.MMA_SPLIT_SHIFT >= 1, hex(task.p[3])
    want = np.maximum(np.matmul(a.astype(np.float64), b.astype(np.float64)) + bias, 0.0).astype(np.float32)
    lp = runtime().load(blob)
    try:
        for run in range(2):
            np.testing.assert_array_equal(lp(a, b, bias)[0], want, err_msg=f"run {run}")
    finally:
        lp.close()


def test_dot_fast_path_random_bf16():
    rng = np.random.default_rng(1003)
    M = K = N = 1024
    a = vmref.bf16_to_f32(vmref.f32_to_bf16((rng.standard_normal((M, K)) * 0.125).astype(np.float32)))
    b = vmref.bf16_to_f32(vmref.f32_to_bf16((rng.standard_normal((K, N)) * 0.125).astype(np.float32)))
    g = G.Graph()
    x, y = g.input((M, K), "bf16"), g.input((K, N), "bf16")
    g.output(g.dot(x, y, tile=256))
    got, _ = run_both(g.build(), [a, b], oracle=None)
    want = a.astype(np.float64) @ b.astype(np.float64)
    assert np.abs(got[0] - want).max() / np.abs(want).max() <= 1e-3


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("Gb,M,K,N", [(1, 1, 768, 2304), (1, 1, 3072, 768), (1, 3, 200, 1000), (12, 1, 640, 64),
                                      (1, 8, 64, 32000), (2, 5, 7, 8)])
def test_gemv_split_k_exact(dt, Gb, M, K, N):
    """Skinny matmuls (TOP_GEMV, split K with the last-arriving split summing the
    partials): integer-valued operands give the exact result, on two executions
    in a row (the arrival counters reset themselves)."""
    rng = np.random.default_rng(74)
    a = rng.integers(-3, 4, (Gb, M, K)).astype(np.float32)
    b = rng.integers(-3, 4, (Gb, K, N)).astype(np.float32)
    g = G.Graph()
    x, y = g.input(a.shape, dt), g.input(b.shape, dt)
    g.output(g.dot(x, y))
    blob, cfg = blob_for(g.build())
    assert any(tk.top == V.TOP_GEMV for tk in vmref.parse(blob).tasks)
    lp = runtime().load(blob)
    try:
        want = np.matmul(a.astype(np.float64), b.astype(np.float64))
        for _ in range(2):
            np.testing.assert_array_equal(lp(a, b)[0], want)
    finally:
        lp.close()


def test_gemv_epilogue_bf16_out():
    rng = np.random.default_rng(75)
    M, K, N = 1, 768, 3072
    a = (rng.standard_normal((M, K)) * 0.5).astype(np.float32)
    b = (rng.standard_normal((K, N)) * 0.05).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    res = rng.standard_normal((M, N)).astype(np.float32)
    g = G.Graph()
    x, y, bb, rr = g.input(a.shape, "bf16"), g.input(b.shape, "bf16"), g.input(bias.shape), g.input(res.shape)
    h = g.dot(x, y, out_dtype="bf16", residual=bb, epilogue=[(V.SUB_ADD, 2, 0.0, 0.0), (V.SUB_GELU, 0, 0.0, 0.0)])
    o = g.dot(x, y, residual=rr, epilogue=[(V.SUB_AFFINE, 0, 0.5, 0.25), (V.SUB_ADD, 1, 0.0, 0.0)])
    g.output(h, o)
    got, want = run_both(g.build(), [a, b, bias, res], oracle="tensor")
    assert_rel(as_f32(got[0], V.DT_BF16), as_f32(want[0], V.DT_BF16), BF16_ULP, 1e-6, "gemv gelu bf16")
    assert_rel(got[1], want[1], 1e-5, 1e-5, "gemv affine + residual")


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_dot_operand_views_with_contiguous_runs(dt):
    """General matmul tiles reading operand views: A as the [tokens, heads *
    head_dim] view of a [heads, tokens, head_dim] tensor (the lowered decoder's
    attention output), read through 16-byte runs; B as the [K, N] view of
    column blocks [N / 32, K, 32] (element path); then a head size of 12, whose
    runs are not whole 16-byte chunks (element path for A too).  Integer
    operands keep every product exact, so the results equal the oracle's bit
    for bit."""
    rng = np.random.default_rng(31)
    for H, S, hd, N, tile in ((4, 96, 64, 96, 64), (4, 96, 64, 96, 128), (3, 70, 12, 64, 64)):
        K = H * hd
        att = rng.integers(-2, 3, (H, S, hd)).astype(np.float32)
        wb = rng.integers(-2, 3, (N // 32, K, 32)).astype(np.float32)
        cvt = (lambda x: vmref.f32_to_bf16(x)) if dt == "bf16" else (lambda x: x.astype(np.float16))
        g = G.Graph()
        ai, bi = g.input(att.shape, dt), g.input(wb.shape, dt)
        a3 = g.view(ai, (S, H, hd), (hd, S * hd, 1))
        b3 = g.view(bi, (K, N // 32, 32), (32, K * 32, 1))
        a2 = G.Tensor(a3.buf, (S, K), a3.dtype, view=a3.view)
        b2 = G.Tensor(b3.buf, (K, N), b3.dtype, view=b3.view)
        g.output(g.dot(a2, b2, tile=tile))
        got, want = run_both(g.build(), [cvt(att), cvt(wb)], oracle="tensor")
        ref = att.transpose(1, 0, 2).reshape(S, K) @ wb.transpose(1, 0, 2).reshape(K, N)
        np.testing.assert_array_equal(got[0], want[0], err_msg=f"{(H, S, hd, N, tile)}")
        np.testing.assert_array_equal(got[0], ref.astype(np.float32), err_msg=f"{(H, S, hd, N, tile)}")


@pytest.mark.parametrize("ew_ts", [256, 64])
def test_broadcast_of_one_element(ew_ts):
    """A view with every stride 0 (a constant broadcast into a buffer, as the
    lowering emits for zero-filled caches): one load and 16-byte stores, the
    ragged end element by element, for 1-, 2-, 4- and 8-byte elements."""
    shape = (7, 9, 13)
    g = G.Graph()
    srcs = [np.array([3.25], np.float32), vmref.f32_to_bf16(np.array([-1.5], np.float32)),
            np.array([-123456789012], np.int64), np.array([True])]
    dts = ["f32", "bf16", "i64", "bool"]
    ins = [g.input((1,), d) for d in dts]
    g.output(*[g.materialize(g.view(t, shape, (0, 0, 0))) for t in ins])
    got, want = run_both(g.build(), srcs, ew_ts=ew_ts)
    for k, (gv, wv) in enumerate(zip(got, want)):
        np.testing.assert_array_equal(gv, wv, err_msg=dts[k])
        assert (np.asarray(gv).reshape(-1) == np.asarray(srcs[k]).reshape(-1)[0]).all(), dts[k]


def _gemv_chain(dt, M, seed):
    """x -> three skinny matmuls in a row (each a phase after a grid barrier) ->
    a fourth against weights the program rewrites first.  Integer operands in
    {-1, 0, 1} and K <= 16 keep every value exact in bf16."""
    rng = np.random.default_rng(seed)
    x = rng.integers(-1, 2, (M, 16)).astype(np.float32)
    ws = [rng.integers(-1, 2, s).astype(np.float32) for s in ((16, 64), (64, 16), (16, 128))]
    w4 = rng.integers(-1, 2, (128, 40)).astype(np.float32)
    g = G.Graph()
    xi = g.input(x.shape, dt)
    wi = [g.input(w.shape, dt) for w in ws]
    w4i = g.input(w4.shape, dt)
    h = xi
    for w in wi:
        h = g.dot(h, w, out_dtype=dt)
    zero = g.const(np.zeros((), np.int32))
    g.dynamic_update_slice(w4i, g.slice(h, (0, 0), (1, 40)), [zero, zero])
    g.output(h, g.dot(h, w4i))
    want_h = x.astype(np.float64)
    for w in ws:
        want_h = want_h @ w
    w4b = w4.astype(np.float64).copy()
    w4b[0, :] = want_h[0, :40]
    return g.build(), [x] + ws + [w4], want_h, want_h @ w4b


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("M", [1, 3])
@pytest.mark.parametrize("nlanes", [3, None])
def test_gemv_chain_across_barriers(dt, M, nlanes):
    """Skinny matmuls in a row, each a phase of its own after a grid barrier,
    then one against weights the program rewrites first (the matmul must see
    the rewrite): exact results, twice in a row, on 3 lanes and on the
    device's lanes."""
    prog, args, want_h, want_o = _gemv_chain(dt, M, 90 + M)
    blob, _ = blob_for(prog, nlanes=nlanes)
    assert sum(t.tile_op == V.TOP_GEMV for t in V.parse(blob).schedule.tasks) == 4
    print(f"[gpu] case: gemv chain {dt} M={M} lanes={V.parse(blob).schedule.n_lanes}", file=sys.stderr, flush=True)
    lp = runtime().load(blob)
    f64 = (lambda a: as_f32(a, V.DT_BF16).astype(np.float64)) if dt == "bf16" else (lambda a: np.asarray(a, np.float64))
    try:
        for _ in range(2):
            h, o = lp(*args)
            np.testing.assert_array_equal(f64(h), want_h)
            np.testing.assert_array_equal(np.asarray(o, np.float64), want_o)
    finally:
        lp.close()


def test_dot_views_batch_epilogue():
    rng = np.random.default_rng(71)
    Gb, M, K, N = 3, 40, 24, 56
    a = rng.integers(-2, 3, (Gb, M, K)).astype(np.float32)
    bt = rng.integers(-2, 3, (Gb, N, K)).astype(np.float32)
    res = rng.integers(-4, 5, (Gb, M, N)).astype(np.float32)
    w = rng.integers(-2, 3, (N, K)).astype(np.float32)
    bias = rng.integers(-4, 5, (N,)).astype(np.float32)
    g = G.Graph()
    x = g.input(a.shape)
    yt = g.input(bt.shape)
    r = g.input(res.shape)
    wt = g.input(w.shape)
    bb = g.input(bias.shape)
    y = g.transpose_view(yt, (0, 2, 1))                        # [G,K,N] view of [G,N,K]
    out1 = g.dot(x, y, epilogue=[(V.SUB_AFFINE, 0, 0.5, 1.0), (V.SUB_ADD, 1, 0.0, 0.0)], residual=r)
    out2 = g.dot(g.reshape(x, (Gb * M, K)), g.transpose_view(wt, (1, 0)),
                 epilogue=[(V.SUB_ADD, 2, 0.0, 0.0), (V.SUB_GELU, 0, 0.0, 0.0)], residual=bb)
    g.output(out1, out2)
    got, want = run_both(g.build(), [a, bt, res, w, bias], mma_t=64)
    np.testing.assert_array_equal(got[0], want[0])
    assert_rel(got[1], want[1], 1e-5, 1e-6, "epilogue gelu")


# --- attention ------------------------------------------------------------------------------------

@pytest.mark.parametrize("dt,hd,causal,T,C", [("bf16", 128, True, 256, 256), ("bf16", 128, False, 128, 384),
                                              ("bf16", 64, True, 384, 512), ("f16", 128, True, 128, 128),
                                              ("bf16", 128, True, 96, 200), ("f16", 64, False, 64, 130),
                                              ("f32", 32, True, 40, 56), ("bf16", 80, False, 64, 100),
                                              # head sizes run on the zero-padded 128 / 64 kernels
                                              ("f16", 96, True, 300, 300), ("bf16", 120, True, 257, 320),
                                              ("bf16", 40, False, 200, 264), ("f16", 8, True, 64, 70),
                                              ("bf16", 72, False, 513, 130),
                                              # f32 matrix-core kernel (128-row blocks, 32-key blocks)
                                              ("f32", 64, True, 300, 300), ("f32", 128, False, 200, 264),
                                              ("f32", 100, True, 129, 200), ("f32", 128, True, 640, 700),
                                              ("f32", 4, False, 33, 40),
                                              # wide 16-bit kernel (hd in (128, 256])
                                              ("bf16", 256, True, 300, 300), ("f16", 256, False, 129, 200),
                                              ("bf16", 192, True, 640, 700), ("f16", 136, True, 64, 90)])
def test_flash_attention(dt, hd, causal, T, C):
    rng = np.random.default_rng(1004)
    H = 3
    q = rng.standard_normal((H, T, hd)).astype(np.float32)
    k = rng.standard_normal((H, C, hd)).astype(np.float32)
    v = rng.standard_normal((H, C, hd)).astype(np.float32)
    if dt == "bf16":
        q, k, v = (vmref.bf16_to_f32(vmref.f32_to_bf16(t)) for t in (q, k, v))
    elif dt == "f16":
        q, k, v = (t.astype(np.float16).astype(np.float32) for t in (q, k, v))
    g = G.Graph()
    Q, K, Vv = g.input(q.shape, dt), g.input(k.shape, dt), g.input(v.shape, dt)
    g.output(g.flash_attention(Q, K, Vv, 1.0 / np.sqrt(hd), causal, out_dtype="f32"))
    got, _ = run_both(g.build(), [q, k, v], oracle=None)
    want = vmref.attention(q, np.transpose(k, (0, 2, 1)), v, 1.0 / np.sqrt(hd), causal)
    # f32: f32 products and sums (matrix cores or the row kernel); 16-bit: P in bf16 / f16
    tol = 2e-5 if dt == "f32" else 1e-2
    err = np.abs(got[0] - want).max() / max(1e-6, np.abs(want).max())
    assert err <= tol, err
    assert_product_elementwise(got[0], want.astype(np.float64),
                               attention_abs_scale(q, np.transpose(k, (0, 2, 1)), v, 1.0 / np.sqrt(hd), causal), tol,
                               f"flash {dt} hd {hd}")


@pytest.mark.parametrize("hd,dt", [(64, "bf16"), (128, "bf16"), (96, "bf16"), (24, "bf16"), (128, "f32"), (36, "f32"),
                                   (256, "bf16"), (200, "f16")])
def test_flash_attention_partial_block_inf_value(hd, dt):
    """Matrix-core path with a partial last key block (C = 200): every query sees
    key C - 1, whose value row is +inf, so every output is +inf.  The block's
    slots past C hold copies of key C - 1 and get probability 0; they must add 0
    (zeroed), not 0 * inf = NaN.  f32: the staged V rows past C are zeros."""
    rng = np.random.default_rng(1005)
    H, T, C = 2, 64, 200
    cast = (lambda x: vmref.bf16_to_f32(vmref.f32_to_bf16(x))) if dt == "bf16" else (lambda x: x)
    q = cast(rng.standard_normal((H, T, hd)).astype(np.float32))
    k = cast(rng.standard_normal((H, C, hd)).astype(np.float32))
    v = cast(rng.standard_normal((H, C, hd)).astype(np.float32))
    v[:, C - 1, :] = np.inf
    g = G.Graph()
    Q, K, Vv = g.input(q.shape, dt), g.input(k.shape, dt), g.input(v.shape, dt)
    g.output(g.flash_attention(Q, K, Vv, 1.0 / np.sqrt(hd), False, out_dtype="f32"))
    got, _ = run_both(g.build(), [q, k, v], oracle=None)
    assert np.isposinf(vmref.attention(q, np.transpose(k, (0, 2, 1)), v, 1.0 / np.sqrt(hd), False)).all()
    assert np.isposinf(got[0]).all(), int(np.isnan(got[0]).sum())


@pytest.mark.parametrize("dt,hd", [("bf16", 128), ("f16", 64), ("bf16", 96), ("f32", 64), ("bf16", 256),
                                   ("f32", 200)])
def test_flash_attention_rows_without_keys(dt, hd):
    """Causal with more queries than keys (T > C): query m sees keys up to
    m + C - T, so the first T - C rows see none.  The reference's kernel divides
    by the running sum (0) and the softmax of an all -inf row is NaN, so those
    rows are NaN; the rest match float64 math.  Each matrix-core path (16-bit,
    padded head, f32, wide 16-bit) and the row kernel (f32, hd 200)."""
    rng = np.random.default_rng(1007)
    H, T, C = 2, 300, 100
    q, k, v = (rng.standard_normal((H, n, hd)).astype(np.float32) for n in (T, C, C))
    if dt == "bf16":
        q, k, v = (vmref.bf16_to_f32(vmref.f32_to_bf16(t)) for t in (q, k, v))
    elif dt == "f16":
        q, k, v = (t.astype(np.float16).astype(np.float32) for t in (q, k, v))
    g = G.Graph()
    Q, K, Vv = g.input(q.shape, dt), g.input(k.shape, dt), g.input(v.shape, dt)
    g.output(g.flash_attention(Q, K, Vv, 1.0 / np.sqrt(hd), True, out_dtype="f32"))
    got, _ = run_both(g.build(), [q, k, v], oracle=None)
    with np.errstate(invalid="ignore"):
        want = vmref.attention(q, np.transpose(k, (0, 2, 1)), v, 1.0 / np.sqrt(hd), True)
    assert np.isnan(want[:, :T - C]).all() and np.isfinite(want[:, T - C:]).all()
    np.testing.assert_array_equal(np.isnan(got[0]), np.isnan(want))
    tol = 2e-5 if dt == "f32" else 1e-2
    err = np.abs(got[0][:, T - C:] - want[:, T - C:]).max() / np.abs(want[:, T - C:]).max()
    assert err <= tol, err


@pytest.mark.parametrize("dt,causal,T,C,target,hd", [("bf16", True, 512, 512, 150.0, 128),
                                                     ("f16", False, 256, 384, 22.0, 128),
                                                     ("bf16", True, 300, 320, 150.0, 96),
                                                     ("bf16", True, 300, 320, 150.0, 256)])
def test_flash_attention_score_jump(dt, causal, T, C, target, hd):
    """A key late in the sequence whose scaled score with one query is `target`
    above the rest: probabilities against the first block's maximum would
    overflow (f32 for bf16 at 150, f16 at 22), so the kernel must take its exact
    two-pass route for that block; the result still matches float64 math (also
    with a padded head size, whose zeroed slots every sweep sets again)."""
    rng = np.random.default_rng(1006)
    H = 2
    q = rng.standard_normal((H, T, hd)).astype(np.float32)
    k = rng.standard_normal((H, C, hd)).astype(np.float32)
    v = rng.standard_normal((H, C, hd)).astype(np.float32)
    qi, kj = T - 3, C - 20                 # query row and the far key (past the first block)
    for h in range(H):
        k[h, kj] = q[h, qi] * (target * np.sqrt(hd) / float(q[h, qi] @ q[h, qi]))
    if dt == "bf16":
        q, k, v = (vmref.bf16_to_f32(vmref.f32_to_bf16(t)) for t in (q, k, v))
    else:
        q, k, v = (t.astype(np.float16).astype(np.float32) for t in (q, k, v))
    g = G.Graph()
    Q, K, Vv = g.input(q.shape, dt), g.input(k.shape, dt), g.input(v.shape, dt)
    g.output(g.flash_attention(Q, K, Vv, 1.0 / np.sqrt(hd), causal, out_dtype="f32"))
    got, _ = run_both(g.build(), [q, k, v], oracle=None)
    want = vmref.attention(q, np.transpose(k, (0, 2, 1)), v, 1.0 / np.sqrt(hd), causal)
    assert np.isfinite(got[0]).all()
    err = np.abs(got[0] - want).max() / max(1e-6, np.abs(want).max())
    assert err <= 1e-2, err
    # the jump row follows the far key's value row
    np.testing.assert_allclose(got[0][:, qi], want[:, qi], rtol=0, atol=2e-2 * np.abs(want).max())


@pytest.mark.parametrize("dt,H,hd,C,pos,jump,mode", [
    ("bf16", 12, 64, 640, 600, None, ""),       # the decoder's shape
    ("bf16", 12, 64, 640, 0, None, ""),         # the step's own key only
    ("f16", 3, 8, 16, 16, None, ""),            # full cache
    ("f32", 2, 24, 24, -1, None, ""),           # clamped position; 3 threads per V row
    ("f32", 1, 256, 1032, 1030, None, ""),      # widest head, 17 splits
    ("bf16", 2, 128, 2056, 2050, 1500, ""),     # 33 splits; a dominant key in an early one
    ("bf16", 2, 64, 640, 300, "new", ""),       # a dominant new key
    ("bf16", 4, 64, 640, 640, "new", ""),       # position past the cache: the step's key joins the last split
    ("bf16", 12, 64, 640, 600, None, "krow masked"),   # the lowered JAX decoder's form
    ("bf16", 12, 64, 640, 700, None, "krow masked"),   # past the cache: clamped to its last column
    ("f16", 3, 256, 1032, 1030, None, "krow"),         # 32 threads per key row
    ("bf16", 2, 128, 2056, 2050, 1500, "krow"),        # 33 splits, a dominant early key
    ("f32", 1, 8, 64, 33, "new", "krow masked"),       # one thread per key row
    ("bf16", 4, 96, 640, 600, None, "krow masked"),    # 12 threads per key row, in groups of 16
    ("f16", 3, 24, 136, 100, "new", "krow"),           # 3 threads per key row, in groups of 4
    ("f32", 2, 80, 1032, 1031, 700, "krow"),           # 10 of 16, 17 splits, a dominant early key
    ("f32", 2, 16, 32, -1, None, "masked"),            # no key left: NaN, as the softmax makes it
])
def test_decode_attention(dt, H, hd, C, pos, jump, mode):
    """TOP_DECODE_ATTN against float64 math on the same (rounded) inputs: keys
    are the cache prefix [0, pos) then the step's own key; splits of 64 cache
    keys combine their partial softmax results.  ``krow``: the key cache is
    [H, C, hd] rows; ``masked``: pos clamps to [0, C - 1], negative is NaN."""
    krow, masked = "krow" in mode, "masked" in mode
    rng = np.random.default_rng(2024 + hd + C)
    q = rng.standard_normal((H, hd)).astype(np.float32)
    k = rng.standard_normal((H, hd)).astype(np.float32)
    v = rng.standard_normal((H, hd)).astype(np.float32)
    ckt = rng.standard_normal((H, hd, C)).astype(np.float32)
    cv = rng.standard_normal((H, C, hd)).astype(np.float32)
    scale = 1.0 / np.sqrt(hd)
    for h in range(H):
        big = q[h] * (40.0 / (scale * float(q[h] @ q[h])))
        if jump == "new":
            k[h] = big
        elif jump is not None:
            ckt[h, :, jump] = big
    if dt == "bf16":
        q, k, v, ckt, cv = (vmref.bf16_to_f32(vmref.f32_to_bf16(t)) for t in (q, k, v, ckt, cv))
    elif dt == "f16":
        q, k, v, ckt, cv = (t.astype(np.float16).astype(np.float32) for t in (q, k, v, ckt, cv))
    kc = np.ascontiguousarray(ckt.transpose(0, 2, 1)) if krow else ckt
    g = G.Graph()
    Q, K, Vv = (g.input((H, hd), dt) for _ in range(3))
    CK, CV = g.input(kc.shape, dt), g.input((H, C, hd), dt)
    POS = g.input((), "i32")
    g.output(g.decode_attention(Q, K, Vv, CK, CV, POS, scale, krow=krow, masked=masked))
    prog = g.build()
    want = vmref.decode_attention(q, kc, cv, k, v, pos, scale, krow, masked)
    tol = 1e-3 if dt == "f32" else 1e-2
    # keys split over CUs, 64 per split; a few lanes run several tiles each
    for nlanes in (None, 7):
        blob, _ = blob_for(prog, nlanes=nlanes)
        tk = next(tk for tk in vmref.parse(blob).tasks if tk.top == V.TOP_DECODE_ATTN)
        assert tk.p[4] >> 16 == -(-C // 64), tk.p[4]
        for _ in range(2):              # the arrival counters reset themselves
            got, _ = run_both(blob, [q, k, v, kc, cv, np.array(pos, np.int32)], oracle=None)
            got = as_f32(got[0], V.DT_BY_NAME[dt]).astype(np.float64).reshape(H, hd)
            if masked and pos < 0:
                assert np.isnan(got).all() and np.isnan(want).all()
                continue
            err = np.abs(got - want).max() / max(1e-6, np.abs(want).max())
            assert np.isfinite(got).all() and err <= tol, (nlanes, err)


def test_decode_attention_runs_twice_with_moving_position():
    """The same loaded program at two positions (the position is read at run
    time, nothing is cached between executions)."""
    H, hd, C = 4, 64, 640
    rng = np.random.default_rng(77)
    arrs = [rng.standard_normal(sh).astype(np.float32) for sh in ((H, hd),) * 3 + ((H, hd, C), (H, C, hd))]
    g = G.Graph()
    ins = [g.input(a.shape) for a in arrs] + [g.input((), "i32")]
    g.output(g.decode_attention(*ins, 0.125))
    blob, _ = blob_for(g.build())
    lp = runtime().load(blob)
    try:
        for pos in (511, 17):
            got = np.asarray(lp(*arrs, np.array(pos, np.int32))[0], np.float64).reshape(H, hd)
            want = vmref.decode_attention(arrs[0], arrs[3], arrs[4], arrs[1], arrs[2], pos, 0.125)
            assert np.abs(got - want).max() <= 1e-3 * np.abs(want).max()
    finally:
        lp.close()


@pytest.mark.parametrize("dt,M,K,N,gelu", [("bf16", 1, 768, 2304, False), ("bf16", 3, 200, 96, True),
                                           ("f16", 2, 512, 64, False), ("f32", 1, 300, 40, True)])
def test_gemv_layernorm_prologue(dt, M, K, N, gelu):
    """A layernorm read only by a skinny matmul runs inside the GEMV's x staging
    (task p5): same result as the oracle (layernorm rounded to the matmul's
    dtype, then the product) within the bf16 / f16 / f32 matmul bar."""
    rng = np.random.default_rng(90 + K)
    x = (rng.standard_normal((M, K)) * 2 + 0.5).astype(np.float32)
    gam = rng.uniform(0.5, 1.5, K).astype(np.float32)
    bet = rng.normal(0, 0.1, K).astype(np.float32)
    w = rng.standard_normal((K, N)).astype(np.float32) / np.sqrt(K)
    g = G.Graph()
    X, GA, BE, W = g.input((M, K)), g.input((K,)), g.input((K,)), g.input((K, N), dt)
    g.output(g.dot(g.layernorm(X, GA, BE, 1e-5, gelu=gelu, out_dtype=dt), W))
    blob, _ = blob_for(g.build())
    p = vmref.parse(blob)
    assert any(tk.top == V.TOP_GEMV and tk.p[5] for tk in p.tasks)
    got, want = run_both(blob, [x, gam, bet, w])
    err = np.abs(got[0] - want[0]).max() / np.abs(want[0]).max()
    assert err <= (1e-3 if dt == "f32" else 1e-2), err


# --- loader validation ----------------------------------------------------------------------------

def test_loader_rejects_out_of_bounds_task():
    from pjrt_amd.runtime import VmrtError, INVALID_ARGUMENT
    g = G.Graph()
    x = g.input((100,))
    g.output(g.unary("exp", x))
    prog = g.build()
    prog.instrs[0].n = 10_000            # reads past the 100-element buffers
    blob = V.serialize(prog, __import__("pjrt_amd.scheduler", fromlist=["x"]).schedule_program(
        prog, __import__("pjrt_amd.scheduler", fromlist=["x"]).DeviceConfig(nlanes=4, ew_ts=256)))
    with pytest.raises(VmrtError) as ei:
        runtime().load(blob, ew_ts=256)
    assert ei.value.code == INVALID_ARGUMENT


def test_loader_rejects_more_lanes_than_resident():
    from pjrt_amd.runtime import VmrtError
    g = G.Graph()
    x = g.input((100,))
    g.output(g.unary("exp", x))
    from pjrt_amd import scheduler as S
    blob = V.serialize(g.build(), S.schedule_program(g.build(), S.DeviceConfig(nlanes=4096, ew_ts=256)))
    with pytest.raises(VmrtError):
        runtime().load(blob, ew_ts=256)


def test_runtime_close_with_live_program():
    """Closing a runtime unloads its live programs first; the program object
    then makes no native call and raises on use (a second Runtime, so the
    session's stays open)."""
    from pjrt_amd.runtime import Runtime, VmrtError
    rt = Runtime(device=0)
    g = G.Graph()
    x = g.input((1000,))
    g.output(g.add(x, x))
    lp = rt.compile(g.build())
    (y,) = lp(np.arange(1000, dtype=np.float32))
    np.testing.assert_array_equal(y, 2 * np.arange(1000, dtype=np.float32))
    rt.close()
    with pytest.raises(VmrtError):
        lp(np.arange(1000, dtype=np.float32))
    lp.close()
    del lp


def test_calibrate_cost_table():
    """vmrt_calibrate measures the reference's four per-tile costs and this
    build's phase-model terms; all positive and of plausible size, and a program
    scheduled with them runs and matches the oracle."""
    import json
    from pjrt_amd import scheduler as S
    rt = runtime()
    costs = rt.calibrate()
    print(f"[gpu] cost table {json.dumps(costs)}", file=sys.stderr, flush=True)
    for k in ("ew_tile_us", "mma_tile_us", "reduce_tile_us", "gather_tile_us", "tile_us", "barrier_us",
              "lane_gbs", "lane_mma_tflops"):
        assert costs[k] > 0, k
    assert costs["tile_us"] < 50 and costs["barrier_us"] < 50 and 1 < costs["lane_gbs"] < 200
    cfg = S.DeviceConfig.from_env({"PJRT_OCL_COST_TABLE": json.dumps(costs)})
    assert S.model_terms(cfg)[0] == costs["tile_us"]
    g = G.Graph()
    x = g.input((70000,))
    g.output(g.unary("exp", g.add(x, x)))
    blob = V.serialize(g.build(), S.schedule_program(g.build(), dataclasses.replace(
        cfg, nlanes=rt.info["n_lanes"], ew_ts=4096, mma_t=128)))
    a = np.linspace(-2, 2, 70000, dtype=np.float32)
    got, want = run_both(blob, [a])
    assert_rel(got[0], want[0], 4e-6, 1e-6, "calibrated schedule")


def test_submitted_launches_report_their_own_status():
    """vmrt_submit: four launches of one program in flight on the runtime's
    stream, each followed by its status epilogue into a slot of its own.  Waited
    for out of order, each completes with its own outputs (a K-split matmul, so
    the task scratch's arrival counters are reused launch after launch), and the
    program's shared status word stays clear for vmrt_program_status."""
    rt = runtime()
    M, K, N = 256, 512, 64
    g = G.Graph()
    a, b = g.input((M, K)), g.input((K, N))
    g.output(g.dot(a, b))
    lp = rt.compile(g.build())
    rng = np.random.default_rng(7)
    ins, outs, want = [], [], []
    for _ in range(4):
        A = rng.integers(-3, 4, (M, K)).astype(np.float32)
        B = rng.integers(-3, 4, (K, N)).astype(np.float32)
        ins.append([rt.to_device(A), rt.to_device(B)])
        outs.append(lp.alloc_outputs())
        want.append(A.astype(np.float64) @ B.astype(np.float64))
    launches = [lp.submit(ins[i], outs[i]) for i in range(4)]
    try:
        for i in reversed(range(4)):
            launches[i].wait()
            assert launches[i].done()
            np.testing.assert_array_equal(outs[i][0].to_host(np.float32, (M, N)), want[i])
        lp.status()
    finally:
        for launch in launches:
            launch.release()
        for buf in [x for row in ins + outs for x in row]:
            buf.free()
        lp.close()


def test_loader_rejects_bad_completion_flags():
    """The loader refuses flag uses whose waits might not end: a flag signaled
    twice, a wait for a flag signaled in another phase, and an entry that
    signals after an entry of its lane and phase waits."""
    import dataclasses as dc
    from pjrt_amd import configs as CF
    from pjrt_amd import scheduler as S
    from pjrt_amd.runtime import VmrtError
    c = CF.GptConfig(layers=2, d=128, heads=2, mlp=256, vocab=300, prompt=32, steps=2)
    prog = CF.gpt_c5(c)
    cfg = S.DeviceConfig(nlanes=16, counters=True, fit_lanes=False)
    sched = S.schedule_program(prog, cfg)
    assert sched.n_flags > 0
    rt = runtime()

    def blob(fn):
        st = [[dc.replace(e) for e in s] for s in sched.lane_streams]
        fn(st)
        return V.serialize(prog, V.Schedule(sched.n_lanes, sched.tasks, st, sched.root_lens, sched.n_flags))

    lp = rt.load(blob(lambda st: None), ew_ts=cfg.ew_ts, mma_t=cfg.mma_t)      # as scheduled: loads
    lp.close()
    ent = [(l, k) for l, s in enumerate(sched.lane_streams) for k, e in enumerate(s)]
    sig = [(l, k) for l, k in ent if sched.lane_streams[l][k].task not in V.CONTROL_SENTINELS
           and sched.lane_streams[l][k].signal_flag != V.FLAG_NONE]
    wt = [(l, k) for l, k in ent if sched.lane_streams[l][k].task not in V.CONTROL_SENTINELS
          and sched.lane_streams[l][k].wait_count]

    def twice(st):
        st[sig[1][0]][sig[1][1]].signal_flag = st[sig[0][0]][sig[0][1]].signal_flag

    def other_phase(st):           # the waiter of the last-numbered flags (layer 1) waits for flag 0 (layer 0)
        l, k = max(wt, key=lambda lk: sched.lane_streams[lk[0]][lk[1]].wait_flag)
        assert st[l][k].wait_flag > 0
        st[l][k].wait_flag, st[l][k].wait_count = 0, 1

    def after_wait(st):
        # a signaling entry of another lane moved into a waiting entry's lane,
        # right after the wait (same phase); both lanes' FOR body ranges follow
        def phase_of(lane, k):
            return sum(1 for x in range(k) if st[lane][x].task == V.ENT_BARRIER)

        lw, kw = wt[0]
        ls, ks = next((l, k) for l, k in sig if l != lw and phase_of(l, k) == phase_of(lw, kw))
        e = st[ls].pop(ks)
        st[lw].insert(kw + 1, e)
        for lane, pos, d in ((ls, ks, -1), (lw, kw + 1, +1)):
            for f in st[lane]:
                if f.task == V.ENT_FOR:
                    if f.tile_lo <= pos < f.tile_lo + f.tile_hi + (d > 0):
                        f.tile_hi += d
                    elif f.tile_lo > pos:
                        f.tile_lo += d

    for name, fn in (("twice", twice), ("other phase", other_phase), ("signal after wait", after_wait)):
        print(f"[gpu] loader flag case: {name}", file=sys.stderr, flush=True)
        with pytest.raises(VmrtError) as ei:
            rt.load(blob(fn), ew_ts=cfg.ew_ts, mma_t=cfg.mma_t)
        assert ei.value.code == 3 and "flag" in str(ei.value), str(ei.value)
