"""The StableHLO front end (pjrt_amd.mlir + lowering + passes), on the CPU oracle.

Each program (tests/hlo_programs.py, MLIR text in the form JAX prints) is
lowered twice -- with the fusion passes and without them -- and both programs
are executed by the oracle; the results must agree with each other and with a
float64 numpy statement of the JAX function.  The fused program must contain the
fused op the pass is for, so a pass that silently stops matching fails here.
"Parity unpinned": the exact StableHLO a given JAX version emits for these
functions is not pinned (no jax in this image); the texts follow JAX's
documented lowering rules."""
import math

import numpy as np
import pytest

import hlo_programs as H
from oracle import vmref
from pjrt_amd import lowering as L
from pjrt_amd import mlir as M
from pjrt_amd import passes
from pjrt_amd import scheduler as S
from pjrt_amd import vmprogram as V

CFG = S.DeviceConfig(nlanes=8, ew_ts=256, mma_t=64)


def run(prog, args, cfg=CFG):
    blob = V.serialize(prog, S.schedule_program(prog, cfg))
    out = vmref.execute(blob, args, ew_ts=cfg.ew_ts, mma_t=cfg.mma_t)
    sched = vmref.execute_schedule(blob, args, ew_ts=cfg.ew_ts, mma_t=cfg.mma_t)
    for a, b in zip(out, sched):
        np.testing.assert_array_equal(a, b)
    return out


def both(text, args):
    fused = L.lower_text(text)
    plain = L.lower_text(text, fuse=False)
    return fused, run(fused, args), run(plain, args)


def live_ops(prog):
    return [i.op for i in prog.instrs if i.op != V.OP_NOP]


def bf16(x):
    return vmref.bf16_to_f32(vmref.f32_to_bf16(np.asarray(x, np.float32)))


# --- the reader ------------------------------------------------------------------------------

def test_reader_pretty_and_generic_forms():
    m = M.parse_module(H.mlp(4, 3, 5, 2))
    assert set(m.funcs) == {"main", "relu"}
    main = m.main
    assert [a.type.shape for a in main.args] == [(4, 3), (3, 5), (5,), (5, 2), (2,)]
    assert [o.name for o in main.body.ops][:3] == ["stablehlo.dot_general", "stablehlo.broadcast_in_dim",
                                                   "stablehlo.add"]
    dn = main.body.ops[0].attr("dot_dimension_numbers").fields
    assert dn["lhs_contracting_dimensions"] == [1] and dn["rhs_contracting_dimensions"] == [0]
    g = M.parse_module(H.generic_chain(64))
    ops = g.main.body.ops
    assert ops[1].attr("value").array().tolist() == 2.0
    assert M.attr_ints(ops[5].attr("permutation")) == [1, 0]


def test_reader_dense_forms():
    t = M.TensorType((2, 2), "f32")
    assert M.dense_to_numpy("[[1.0, 2.0], [3.0, 4.0]]", t).tolist() == [[1, 2], [3, 4]]
    assert M.dense_to_numpy('"0x0000803F000000400000404000008040"', t).tolist() == [[1, 2], [3, 4]]
    assert M.dense_to_numpy("0xFF800000", M.TensorType((), "f32")) == -np.inf
    assert M.dense_to_numpy("true", M.TensorType((3,), "i1")).tolist() == [True] * 3
    assert M.dense_to_numpy("-7", M.TensorType((), "i32")) == -7


def test_reader_rejects_malformed_text():
    with pytest.raises(L.LoweringError):
        L.lower_text("module { func.func public @main(%arg0: tensor<4xf32>) -> tensor<4xf32> { %0 = ")
    with pytest.raises(L.LoweringError):
        L.lower_text(H.mlp().replace("stablehlo.maximum", "stablehlo.frobnicate"))


# --- configs as JAX programs --------------------------------------------------------------------

def test_mlp_config1_epilogue_fusion():
    """Config 1: bias and relu run in the first matmul's store (epilogue sources
    2 and 3), the second bias in the second's: two instructions."""
    rng = np.random.default_rng(1001)
    x = rng.standard_normal((16, 8)).astype(np.float32)
    w1 = (rng.standard_normal((8, 32)) / math.sqrt(8)).astype(np.float32)
    b1 = np.full(32, 0.01, np.float32)
    w2 = (rng.standard_normal((32, 4)) / math.sqrt(32)).astype(np.float32)
    b2 = rng.standard_normal(4).astype(np.float32)
    prog, (got,), (plain,) = both(H.mlp(16, 8, 32, 4), [x, w1, b1, w2, b2])
    assert live_ops(prog) == [V.OP_DOT, V.OP_DOT]
    want = np.maximum(x.astype(np.float64) @ w1 + b1, 0) @ w2 + b2
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(got, plain, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("rows,d", [(8, 64), (16, 4096)])
def test_layernorm_gelu_convert_config2_one_row_op(rows, d):
    """Config 2: the decomposed layernorm (reduce / broadcast / divide / rsqrt),
    gamma / beta, tanh-GELU and the bf16 convert become ONE row op -- the
    reference's fusion stops at seg <= 1024 (lowering.py:1553) and never takes
    the affine, GELU or convert."""
    rng = np.random.default_rng(1002)
    x = rng.standard_normal((rows, d)).astype(np.float32)
    g = rng.uniform(0.5, 1.5, d).astype(np.float32)
    b = (rng.standard_normal(d) * 0.1).astype(np.float32)
    prog, (got,), (plain,) = both(H.ln_gelu(rows, d), [x, g, b])
    assert live_ops(prog) == [V.OP_LAYERNORM_AFFINE]
    ln = next(i for i in prog.instrs if i.op == V.OP_LAYERNORM_AFFINE)
    assert prog.aux[ln.aux] == V.LN_AFFINE | V.LN_GELU | V.LN_TWO_PASS
    assert prog.buffers[ln.dst].dtype == V.DT_BF16
    x64 = x.astype(np.float64)
    mu = x64.mean(1, keepdims=True)
    z = (x64 - mu) / np.sqrt(((x64 - mu) ** 2).mean(1, keepdims=True) + 1e-5) * g + b
    want = 0.5 * z * (1 + np.tanh(0.7978845608 * (z + 0.044715 * z ** 3)))
    gf, pf = vmref.bf16_to_f32(got).astype(np.float64), vmref.bf16_to_f32(plain).astype(np.float64)
    assert np.all(np.abs(gf - want) <= 2.0 ** -7 * np.abs(want) + 1e-6)
    assert np.all(np.abs(gf - pf) <= 2.0 ** -7 * np.abs(pf) + 1e-6)
    # arena: input, gamma, beta, output and the constants, no intermediates
    assert prog.arena_bytes < rows * d * 6 + 3 * d * 4 + 4096


@pytest.mark.parametrize("dt,out", [("bf16", "f32"), ("f32", "f32"), ("bf16", "bf16")])
def test_dot_general_dtypes(dt, out):
    """dot_general with bf16 operands and f32 accumulation; a bf16 result is
    honoured (the reference always produces f32, ops/dot.py:158)."""
    rng = np.random.default_rng(1003)
    a = rng.integers(-3, 4, (64, 32)).astype(np.float32)
    b = rng.integers(-3, 4, (32, 48)).astype(np.float32)
    prog, (got,), _ = both(H.matmul(64, 32, 48, dt, out), [a, b])
    assert live_ops(prog) == [V.OP_DOT]
    want = a.astype(np.float64) @ b
    if out == "bf16":
        np.testing.assert_array_equal(got, vmref.f32_to_bf16(want.astype(np.float32)))
    else:
        np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("dt", ["bf16", "f32"])
@pytest.mark.parametrize("causal", [True, False])
def test_attention_config4_becomes_flash_attention(causal, dt):
    """Config 4's shape of program (bf16 Q/K/V, f32 scores, optional causal mask
    by iota compare, softmax, bf16 P; or the same program in f32): one
    OP_FLASH_ATTN with the causal flag, K read through the plain transpose view
    the matrix-core kernels take, within the attention tolerance of float64
    math and of the unfused program."""
    B, Hh, T, D = 1, 2, 32, 16
    rng = np.random.default_rng(1004)
    cast = bf16 if dt == "bf16" else (lambda x: np.asarray(x, np.float32))
    q, k, v = (cast(rng.standard_normal((B, Hh, T, D))) for _ in range(3))
    prog, (got,), (plain,) = both(H.attention(B, Hh, T, D, dt=dt, causal=causal), [q, k, v])
    assert live_ops(prog) == [V.OP_FLASH_ATTN]
    fa = next(i for i in prog.instrs if i.op == V.OP_FLASH_ATTN)
    G, Mq, C, hd, sbits, cflag, qv, kv, vv = prog.aux[fa.aux:fa.aux + 9]
    assert (G, Mq, C, hd, cflag, qv, vv) == (B * Hh, T, T, D, int(causal), 0, 0)
    assert prog.aux[kv - 1:kv + 7] == [3, G, hd, C, C * hd, 1, hd, 0]
    assert abs(V.bits_f32(sbits) - D ** -0.5) < 1e-7
    s = np.einsum("bhqd,bhkd->bhqk", q.astype(np.float64), k) * D ** -0.5
    if causal:
        s = np.where(np.tril(np.ones((T, T), bool)), s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    want = p @ v
    if dt == "bf16":
        gf, pf, tol = vmref.bf16_to_f32(got), vmref.bf16_to_f32(plain), 1e-2
    else:
        gf, pf, tol = np.asarray(got, np.float32), np.asarray(plain, np.float32), 1e-5
    assert np.abs(gf - want).max() <= tol * np.abs(want).max()
    assert np.abs(gf - pf).max() <= tol * np.abs(pf).max()


def test_argmax_variadic_reduce():
    rng = np.random.default_rng(7)
    x = rng.standard_normal((4, 1000)).astype(np.float32)
    x[1, [10, 700]] = 9.0                          # a tie: the first index wins
    prog, (val, idx), _ = both(H.argmax_rows(4, 1000), [x])
    assert live_ops(prog) == [V.OP_ARGMAX_SEG]
    assert idx.tolist() == np.argmax(x, 1).tolist() and idx[1] == 10
    np.testing.assert_array_equal(val, x.max(1))


# --- control flow (reference tests/_while_e2e_body.py closed forms) ---------------------------------

def test_fori_loop_unrolled_and_composed():
    """fori_loop(0, 5, a + 3) from 2 -> 17: unrolled, then the five affines
    compose into one."""
    prog, (got,), (plain,) = both(H.fori_add(5), [np.float32(2.0)])
    assert float(got) == 17.0 and float(plain) == 17.0
    assert live_ops(prog) == [V.OP_AFFINE_F32]


def test_fori_loop_as_for_when_large(monkeypatch):
    """A counted loop beyond the unroll limits becomes OP_FOR (one barrier per
    trip), its carry updated in place."""
    monkeypatch.setenv("PJRT_OCL_WHILE", "for")
    x = np.arange(1000, dtype=np.float32)
    prog, (got,), _ = both(H.fori_add(100, 1000), [x])
    np.testing.assert_array_equal(got, x + 300)
    ops = live_ops(prog)
    assert V.OP_FOR in ops and ops.count(V.OP_COPY_F32) <= 1


def test_while_data_dependent():
    """while v < 1000: (i + 1, 2 v) from (0, 1) -> (10, 1024): OP_WHILE with a
    cond sub-list."""
    prog, (i, v), _ = both(H.while_double(), [np.float32(1.0)])
    assert int(i) == 10 and float(v) == 1024.0
    assert V.OP_WHILE in live_ops(prog)


@pytest.mark.parametrize("mode", ["unroll", "for"])
@pytest.mark.parametrize("swap", [False, True])
def test_fori_carry_passthrough_and_swap(mode, swap, monkeypatch):
    """(a, b) -> (a + 1, a) from (x, -x): the passed-on carry reads a's value
    from before the update (x + 5, x + 4 after 5 trips), though the update of a
    may run in place; (a, b) -> (b, a) five times gives (-x, x)."""
    monkeypatch.setenv("PJRT_OCL_WHILE", mode)
    prog, got, plain = both(H.fori_shift(5, swap), [np.float32(2.0)])
    want = (-2.0, 2.0) if swap else (7.0, 6.0)
    for out in (got, plain):
        assert tuple(float(x) for x in out) == want
    if mode == "for":
        assert V.OP_FOR in live_ops(prog)


@pytest.mark.parametrize("mode", ["unroll", "for"])
def test_scan_stacking_dynamic_update_slice(mode, monkeypatch):
    """scan-style stacking ys[i] = x * (i + 1) through dynamic_update_slice: as
    OP_FOR the update writes the carry in place (no per-trip copy of ys)."""
    monkeypatch.setenv("PJRT_OCL_WHILE", mode)
    x = np.array([1, 2, 3, 4], np.float32)
    prog, (got,), _ = both(H.scan_stack(6, 4), [x])
    np.testing.assert_array_equal(got, np.outer(np.arange(1, 7), x))
    if mode == "for":
        body = [i for i in prog.instrs if i.op == V.OP_DYNAMIC_UPDATE_SLICE]
        assert body and not any(i.op == V.OP_GATHER_STRIDED for i in prog.instrs[prog.main_len:])


def test_generic_form_chain_fuses_into_a_region():
    x = np.linspace(-2, 2, 64, dtype=np.float32).reshape(8, 8)
    prog, (got,), (plain,) = both(H.generic_chain(64), [x])
    np.testing.assert_allclose(got, (np.exp(x.astype(np.float64)) * 2 - x).T, rtol=2e-6)
    np.testing.assert_allclose(got, plain, rtol=1e-6)


# --- the passes on their own ------------------------------------------------------------------------

def test_reuse_arena_packs_a_chain():
    """Twelve dependent steps sin(transpose(x)) over 64 KiB tensors (each step
    reads across lanes, so each is a phase of its own): the bump layout needs one
    slot per value, the liveness packing a few."""
    t = "tensor<128x128xf32>"
    steps = "\n".join(f"    %t{k} = stablehlo.transpose %{k}, dims = [1, 0] : ({t}) -> {t}\n"
                      f"    %{k + 1} = stablehlo.sine %t{k} : {t}" for k in range(12))
    text = f"""
func.func public @main(%0: {t}) -> {t} {{
{steps}
    return %12 : {t}
}}"""
    for fuse in (False, True):
        prog = L.lower_text(text, fuse=fuse)
        bump = sum(max(64, b.size_bytes) for b in prog.buffers if b.size_bytes)
        assert prog.arena_bytes <= 5 * 65536 < bump
        x = np.linspace(-1, 1, 128 * 128, dtype=np.float32).reshape(128, 128)
        (got,) = run(prog, [x])
        want = x.astype(np.float64)
        for _ in range(12):
            want = np.sin(want.T)
        np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)


def test_reuse_arena_on_the_hand_built_decoder():
    """The liveness packing applied to the config-5 decoder built by hand
    (aliases move with their parent buffer): a smaller arena, the same tokens."""
    from pjrt_amd import configs as CF
    c = CF.GptConfig(layers=2, d=64, heads=2, mlp=128, vocab=97, prompt=8, steps=4)
    args = CF.gpt_inputs(c, seed=5)
    prog = CF.gpt_c5(c, emit_logits=True)
    before = prog.arena_bytes
    want = run(prog, args)
    prog2 = CF.gpt_c5(c, emit_logits=True)
    passes.reuse_arena(prog2, CFG)
    assert prog2.arena_bytes < before
    for a, b in zip(run(prog2, args), want):
        np.testing.assert_array_equal(a, b)


def _barriers(prog, cfg):
    sched = S.schedule_program(prog, cfg)
    return sum(e.task == V.ENT_BARRIER for e in sched.lane_streams[0])


def test_reuse_arena_keeps_the_schedule():
    """Buffers the packing places on the same bytes have disjoint lifetimes; the
    scheduler orders accesses by the true alias groups of the layout before
    packing, so the packed decoder gets the same barriers as the unpacked one
    (ordering every byte-sharing buffer as one, transitively, had doubled the
    decode step's barriers), and a buffer no instruction touches keeps no
    bytes."""
    from pjrt_amd import configs as CF
    c = CF.GptConfig(layers=2, d=64, heads=2, mlp=128, vocab=97, prompt=8, steps=4)
    cfg = S.DeviceConfig(nlanes=16)
    prog = CF.gpt_c5(c)
    prog2 = CF.gpt_c5(c)
    passes.reuse_arena(prog2, cfg)
    assert prog2.arena_bytes < prog.arena_bytes
    assert _barriers(prog2, cfg) == _barriers(prog, cfg)
    # the same program with its alias groups dropped (groups from the packed overlaps)
    prog3 = CF.gpt_c5(c)
    passes.reuse_arena(prog3, cfg)
    prog3.alias_groups = None
    assert _barriers(prog3, cfg) > _barriers(prog, cfg)
    # the lowered attention: the decomposed score matrices the fusion replaced take no arena
    low = L.lower_text(H.attention(1, 2, 256, 64))
    io = sum(low.buffers[b].size_bytes for b in low.inputs + low.outputs)
    assert low.arena_bytes <= io + 64 * len(low.buffers)


def test_donation_aliases():
    """A donated argument (tf.aliasing_output) may share its memory with the
    output when every read of it is a phase earlier than every write of the
    output; in the same phase, or with a size mismatch, it may not."""
    assert L.lower_text(H.donated_chain(64)).io_aliases == [(0, 0)]
    assert L.lower_text(H.donated_chain(64, twice=False)).io_aliases == []
    assert L.lower_text(H.donated_chain(64, alias_to=3)).io_aliases == []
    text = H.donated_chain(64).replace(" {tf.aliasing_output = 0 : i32}", "")
    assert L.lower_text(text).io_aliases == []
    # the parser keeps each argument's attribute dictionary
    m = M.parse_module(H.donated_chain(8))
    assert M.attr_int(m.main.arg_attr(0, "tf.aliasing_output")) == 0 and m.main.arg_attr(1, "x") is None


GPT_TINY = dict(layers=2, d=64, heads=2, mlp=128, vocab=97, prompt=8, steps=4)


def _decode_body(prog):
    """Instructions of the decode loop body (the program's OP_FOR)."""
    fors = [i for i in prog.instrs if i.op == V.OP_FOR]
    assert len(fors) == 1
    return [prog.instrs[j] for j in range(fors[0].n, fors[0].n + fors[0].imm) if prog.instrs[j].op != V.OP_NOP]


@pytest.mark.parametrize("mode", ["unroll", "for"])
def test_gpt_decode_program_lowers_to_the_decoder(mode, monkeypatch):
    """Config 5 as the JAX program (prefill, then a fori_loop decode with KV
    caches updated by dynamic_update_slice, a key <= pos mask, argmax): the
    lowered program gives the tokens of the independent numpy decoder and its
    logits within f32 rounding.  As a loop, each layer's decode step is one
    OP_DECODE_ATTN, each layernorm one row op, and the caches are updated in
    place (nothing copies a cache per step)."""
    from pjrt_amd import configs as CF
    from pjrt_amd import stablehlo_configs as SC
    monkeypatch.setenv("PJRT_OCL_WHILE", mode)
    c = CF.GptConfig(**GPT_TINY)
    prog = L.lower_text(SC.gpt_decode(c, emit_logits=True))
    args = CF.gpt_inputs(c, seed=5)
    first, toks, logits = run(prog, args)
    ref_toks, ref_logits = CF.gpt_reference(c, args)
    np.testing.assert_array_equal(np.concatenate([first, toks]), ref_toks)
    assert np.abs(logits - ref_logits).max() <= 1e-5 * np.abs(ref_logits).max()
    if mode == "for":
        body = _decode_body(prog)
        ops = [i.op for i in body]
        cache = c.heads * (-(-c.ctx // 8) * 8) * c.hd
        assert ops.count(V.OP_DECODE_ATTN) == c.layers and V.OP_SOFTMAX not in ops
        assert ops.count(V.OP_LAYERNORM_AFFINE) == 2 * c.layers + 1 and V.OP_MAP_REGION not in ops
        assert not [i for i in body if i.op in (V.OP_GATHER_STRIDED, V.OP_CONVERT, V.OP_COPY_F32) and i.n == cache]


@pytest.mark.parametrize("d", [128, 192, 512])
def test_gpt_prefill_attention_gets_the_matrix_core_layout(d):
    """The prefill's attention reads q, k, v as head views of the fused QKV
    projection; the flash fusion gathers them into the matrix-core kernel's
    layout (Q, V plain [H, T, hd], K the transpose of a plain [H, T, hd]), also
    for a head size (96) that kernel runs zero-padded and for the wide kernel's
    256, and the decoder's tokens and logits are unchanged."""
    from pjrt_amd import configs as CF
    from pjrt_amd import stablehlo_configs as SC
    c = CF.GptConfig(layers=1, d=d, heads=2, mlp=128, vocab=97, prompt=64, steps=4)
    prog = L.lower_text(SC.gpt_decode(c, emit_logits=True))
    (fa,) = [i for i in prog.instrs if i.op == V.OP_FLASH_ATTN]
    G, M, C, hd, _, causal, qv, kv, vv = prog.aux[fa.aux:fa.aux + 9]
    assert (G, M, C, hd, causal, qv, vv) == (2, 64, 64, d // 2, 1, 0, 0)
    assert prog.aux[kv - 1:kv + 7] == [3, G, hd, C, C * hd, 1, hd, 0]
    args = CF.gpt_inputs(c, seed=3)
    first, toks, logits = run(prog, args)
    ref_toks, ref_logits = CF.gpt_reference(c, args)
    np.testing.assert_array_equal(np.concatenate([first, toks]), ref_toks)
    assert np.abs(logits - ref_logits).max() <= 1e-5 * np.abs(ref_logits).max()


@pytest.mark.parametrize("fused", [True, False])
def test_reference_decode_step(fused, monkeypatch):
    """The reference's decode benchmark step (tools/bench_decode.py: f32, keys
    and values appended with concatenate, no mask) against its float64 numpy
    statement.  Fused, each layer's attention is one OP_DECODE_ATTN reading the
    caches in place (no concatenation is built)."""
    from pjrt_amd import stablehlo_configs as SC
    if not fused:
        monkeypatch.setenv("PJRT_OCL_DECODE_ATTN", "0")
    cfg = (64, 2, 128, 2, 16)
    prog = L.lower_text(SC.decode_step(cfg))
    args = SC.decode_step_inputs(cfg, seed=4)
    (got,) = run(prog, args)
    want = H.decode_step_reference(cfg, args)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5 * np.abs(want).max())
    ops = live_ops(prog)
    if fused:
        assert ops.count(V.OP_DECODE_ATTN) == 2 and V.OP_SCATTER not in ops and V.OP_SOFTMAX not in ops
    else:
        assert V.OP_DECODE_ATTN not in ops


def test_gpt_decode_unfused_and_planted_mask(monkeypatch):
    """Without the decode fusion the decomposed chain (bf16 probabilities) still
    decodes the same tokens; a planted mask (key < pos: the step's own key
    left out) is not fused, and its logits differ from the decoder's."""
    from pjrt_amd import configs as CF
    from pjrt_amd import stablehlo_configs as SC
    c = CF.GptConfig(**GPT_TINY)
    args = CF.gpt_inputs(c, seed=5)
    ref_toks, ref_logits = CF.gpt_reference(c, args)
    monkeypatch.setenv("PJRT_OCL_DECODE_ATTN", "0")
    plain = L.lower_text(SC.gpt_decode(c, emit_logits=True))
    monkeypatch.delenv("PJRT_OCL_DECODE_ATTN")
    assert V.OP_DECODE_ATTN not in live_ops(plain)
    first, toks, logits = run(plain, args)
    np.testing.assert_array_equal(np.concatenate([first, toks]), ref_toks)
    assert np.abs(logits - ref_logits).max() <= 1e-2 * np.abs(ref_logits).max()
    bad = L.lower_text(SC.gpt_decode(c, emit_logits=True, mask_cmp="LT"))
    assert V.OP_DECODE_ATTN not in live_ops(bad)
    _, _, bad_logits = run(bad, args)
    assert np.abs(bad_logits[1:] - ref_logits[1:]).max() > 1e-2 * np.abs(ref_logits).max()


def test_planted_pass_mistake_is_caught(monkeypatch):
    """A GELU fusion that matched the cubic coefficient loosely (0.04715) would
    fuse a different function; the exact-constant gate must refuse, leaving the
    decomposed chain (whose result then still equals numpy)."""
    text = H.ln_gelu(8, 64).replace("4.471500e-02", "4.715000e-02")
    prog = L.lower_text(text)
    assert V.OP_GELU not in live_ops(prog)
    ln = [i for i in prog.instrs if i.op == V.OP_LAYERNORM_AFFINE]
    assert ln and not prog.aux[ln[0].aux] & V.LN_GELU
