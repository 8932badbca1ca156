"""Scheduler behaviour (restating tests/test_lowering.py:469-701 of the
reference) plus schedule invariants checked by the oracle's lane simulator."""
import json

import numpy as np
import pytest

from pjrt_amd import graph as G
from pjrt_amd import scheduler as S
from pjrt_amd import vmprogram as V
from oracle import vmref


def phases(sched):
    counts = {sum(1 for e in s if e.task == V.ENT_BARRIER) for s in sched.lane_streams}
    assert len(counts) == 1
    out = [set() for _ in range(counts.pop() + 1)]
    for s in sched.lane_streams:
        p = 0
        for e in s:
            if e.task == V.ENT_BARRIER:
                p += 1
            elif e.task not in V.CONTROL_SENTINELS:
                out[p].add(e.task)
    return out


def two_independent():
    g = G.Graph()
    a, b, c, d = (g.input((8,)) for _ in range(4))
    g.output(g.add(a, b), g.mul(c, d))
    return g.build()


def test_two_independent_ops_co_scheduled():
    prog = two_independent()
    sched = S.schedule_program(prog, S.DeviceConfig(nlanes=8))
    assert phases(sched) == [{0, 1}]
    lanes = [l for l, s in enumerate(sched.lane_streams) for e in s if e.task in (0, 1)]
    assert len(lanes) == 2 and len(set(lanes)) == 2
    rng = np.random.default_rng(1234)
    args = [rng.integers(-16, 16, 8).astype(np.float32) for _ in range(4)]
    blob = V.serialize(prog, sched)
    out = vmref.execute_schedule(blob, args)
    np.testing.assert_array_equal(out[0], args[0] + args[1])
    np.testing.assert_array_equal(out[1], args[2] * args[3])


def test_dependent_elementwise_chain_shares_a_lane():
    g = G.Graph()
    a, b, c = (g.input((8,)) for _ in range(3))
    g.output(g.sub(g.mul(a, b), c))
    prog = g.build()
    sched = S.schedule_program(prog, S.DeviceConfig(nlanes=8))
    assert phases(sched) == [{0, 1}]
    lanes = {l for l, s in enumerate(sched.lane_streams) for e in s if e.task in (0, 1)}
    assert len(lanes) == 1


def test_shaped_consumer_forces_barrier():
    g = G.Graph()
    x = g.input((64, 32))
    y = g.mul(x, x)
    s = g.reduce_last(y, V.RED_SUM)
    g.output(s)
    prog = g.build()
    sched = S.schedule_program(prog, S.DeviceConfig(nlanes=4))
    assert len(phases(sched)) == 2


def test_nlanes_and_exact_tile_coverage():
    g = G.Graph()
    a, b = g.input((40000,)), g.input((40000,))
    g.output(g.add(a, b))
    prog = g.build()
    cfg = S.DeviceConfig(nlanes=4, ew_ts=16384)
    sched = S.schedule_program(prog, cfg)
    ents = sorted((e.tile_lo, e.tile_hi) for s in sched.lane_streams for e in s if e.task == 0)
    assert ents == [(0, 1), (1, 2), (2, 3)]
    x = np.arange(40000, dtype=np.float32)
    (out,) = vmref.execute_schedule(V.serialize(prog, sched), [x, 2 * x], ew_ts=16384)
    np.testing.assert_array_equal(out, 3 * x)


def two_adds(n0, n1):
    g = G.Graph()
    a, b = g.input((n0,)), g.input((n0,))
    c, d = g.input((n1,)), g.input((n1,))
    g.output(g.add(a, b), g.add(c, d))
    return g.build()


def test_cost_proportional_split_and_lpt_makespan():
    ts = 4096
    prog = two_adds(8 * ts, 2 * ts)
    sched = S.schedule_program(prog, S.DeviceConfig(nlanes=8, ew_ts=ts))
    l0 = {i for i, s in enumerate(sched.lane_streams) for e in s if e.task == 0}
    l1 = {i for i, s in enumerate(sched.lane_streams) for e in s if e.task == 1}
    assert len(l0) > len(l1)
    loads = [sum(e.tile_hi - e.tile_lo for e in s if e.task not in V.CONTROL_SENTINELS)
             for s in sched.lane_streams]
    assert max(loads) == 2
    vmref.execute_schedule(V.serialize(prog, sched),
                           [np.zeros(8 * ts, np.float32)] * 2 + [np.zeros(2 * ts, np.float32)] * 2,
                           ew_ts=ts)


def test_equal_cost_even_split():
    ts = 4096
    prog = two_adds(4 * ts, 4 * ts)
    sched = S.schedule_program(prog, S.DeviceConfig(nlanes=8, ew_ts=ts))
    n0 = sum(1 for s in sched.lane_streams for e in s if e.task == 0)
    n1 = sum(1 for s in sched.lane_streams for e in s if e.task == 1)
    assert n0 == n1 == 4


def test_device_config_from_env(tmp_path):
    cost = tmp_path / "cost.json"
    cost.write_text(json.dumps({"ew_tile_us": 2.5, "mma_tile_us": 40.0,
                                "gather_tile_us": 3.0, "reduce_tile_us": 5.0}))
    cfg = S.DeviceConfig.from_env({"PJRT_OCL_NLANES": "16", "PJRT_OCL_EW_TS": "8192",
                                   "PJRT_OCL_MMA_T": "256",
                                   "PJRT_OCL_COST_TABLE": str(cost)})
    assert (cfg.nlanes, cfg.ew_ts, cfg.mma_t) == (16, 8192, 256)
    assert cfg.costs["mma_tile_us"] == 40.0
    d = S.DeviceConfig.from_env({})
    assert d.nlanes == S.DEFAULT_NLANES and d.costs == {}
    m = S.DeviceConfig.from_env({"PJRT_OCL_COST_TABLE": str(tmp_path / "none.json")})
    assert m.costs == {}


def test_while_control_entry_and_root_len():
    prog = V.VMProgram(
        arena_bytes=128, buffers=[V.Buffer(0, 4), V.Buffer(64, 4)],
        inputs=[], outputs=[0], input_shapes=[], output_shapes=[()],
        consts=[(1, np.float32(0.0).tobytes())],
        instrs=[V.Instr(V.OP_WHILE, dst=1, a=1, b=0, n=1, imm=0)], main_len=1)
    sched = S.schedule_program(prog, S.DeviceConfig(nlanes=8))
    for lane, s in enumerate(sched.lane_streams):
        root = s[:sched.root_lens[lane]]
        w = [e for e in root if e.task == V.ENT_WHILE]
        assert len(w) == 1
        assert w[0].tile_lo >= sched.root_lens[lane]
        assert w[0].wait_flag >= sched.root_lens[lane]
        assert w[0].signal_flag == 1


def test_mma_autotile_picks_parallel_tile():
    g = G.Graph()
    a, b = g.input((4096, 4096), "bf16"), g.input((4096, 4096), "bf16")
    g.output(g.dot(a, b))
    prog = g.build()
    sched = S.schedule_program(prog, S.DeviceConfig(nlanes=256, mma_t=128))
    t = sched.tasks[0]
    assert t.tile_op == V.TOP_MMA and (t.p3 >> 24) == V.MMA_TILE_CODES[256]
    assert S.n_tiles(t, S.DeviceConfig(nlanes=256)) == 256
    g = G.Graph()
    a, b = g.input((512, 768)), g.input((768, 768))
    g.output(g.dot(a, b))
    sched = S.schedule_program(g.build(), S.DeviceConfig(nlanes=256, mma_t=128))
    assert (sched.tasks[0].p3 >> 24) & 0xF == V.MMA_TILE_CODES[64]


def test_mma_autotile_prefers_fast_16bit_tile():
    """16-bit matmuls the 256-wide fast tile takes keep 256 down to an eighth of
    the lanes (36 tiles of 256 for 1536^3 on 256 lanes); f32, views, K or N not a
    multiple of 8, and too few tiles fall back to the count rule."""
    def tile(M, K, N, dt, view=False):
        g = G.Graph()
        a = g.input((M, K), dt)
        if view:
            b = g.transpose_view(g.input((N, K), dt), (1, 0))
        else:
            b = g.input((K, N), dt)
        g.output(g.dot(a, b))
        t = S.schedule_program(g.build(), S.DeviceConfig(nlanes=256, mma_t=128)).tasks[0]
        return V.MMA_CODE_TILE[(t.p3 >> 24) & 0xF]
    assert tile(1536, 1536, 1536, "bf16") == 256
    assert tile(3000, 3000, 3000, "f16") == 256
    assert tile(1536, 1536, 1536, "f32") == 64          # 6 x 6 tiles of 256, 144 of 128: the count rule
    assert tile(1024, 1024, 1024, "bf16") == 64         # 16 tiles of 256: too few
    assert tile(1536, 1536, 1532, "bf16") != 256        # N not a multiple of 8
    assert tile(1536, 1536, 1536, "bf16", view=True) != 256


def test_mma_autotile_long_k_skinny_takes_split_128():
    """A long K (>= 4096) with few 256-wide tiles (fewer than a sixth of the
    lanes) takes 128-wide tiles, which the K split spreads over the lanes, or
    64-wide ones where those fit the lanes in one round; 48 or more 256-wide
    tiles, or a shorter K, keep the other rules."""
    def task(M, K, N, dt="bf16"):
        g = G.Graph()
        g.output(g.dot(g.input((M, K), dt), g.input((K, N), dt)))
        return S.schedule_program(g.build(), S.DeviceConfig(nlanes=256, mma_t=128)).tasks[0]
    edge = lambda t: V.MMA_CODE_TILE[(t.p3 >> 24) & 0xF]
    split = lambda t: 1 << (t.p3 >> 28)
    for M, K, N in ((512, 4096, 4096), (512, 11008, 4096)):
        t = task(M, K, N)
        assert edge(t) == 128, (M, K, N)
        tiles = -(-M // 128) * -(-N // 128)
        assert split(t) > 1 and tiles * split(t) <= 256, (M, K, N, split(t))
    for M, K, N in ((256, 4096, 4096), (512, 4096, 2048), (128, 4096, 4096)):   # 256, 256, 128 tiles of 64
        t = task(M, K, N)
        assert edge(t) == 64, (M, K, N)
        tiles = -(-M // 64) * -(-N // 64)
        assert tiles * split(t) <= 256 and (split(t) > 1) == (tiles * 2 <= 256), (M, K, N, split(t))
    assert edge(task(768, 4096, 4096)) == 256           # 48 tiles of 256
    assert edge(task(384, 4096, 8192)) == 256           # 64 tiles of 256
    assert edge(task(256, 3072, 768)) != 128            # K below 4096
    assert edge(task(256, 4096, 4096, "f32")) == 64     # f32: the count rule (256 tiles of 64)


# --- K-split matmuls (extension) -----------------------------------------------------

def test_mma_split_k_choice():
    """Config 1's matmuls on 128 lanes: [256,128]x[128,512] as 32 tiles of 64 x 64
    split 4 ways (two 16-deep slabs each), [256,512]x[512,64] as 4 tiles split 16
    ways; never a split for big outputs, shallow K, or with the switch off."""
    cfg = S.DeviceConfig(nlanes=128)
    assert S.mma_split_log2(256, 512, 128, 1, 64, V.DT_F32, cfg) == 2
    assert S.mma_split_log2(256, 64, 512, 1, 64, V.DT_F32, cfg) == 4
    assert S.mma_split_log2(256, 64, 512, 1, 64, V.DT_BF16, cfg) == 3      # 32-deep 16-bit slabs
    assert S.mma_split_log2(4096, 4096, 4096, 1, 256, V.DT_BF16, cfg) == 0
    assert S.mma_split_log2(256, 64, 48, 1, 64, V.DT_F32, cfg) == 0
    assert S.mma_split_log2(64, 64, 1 << 20, 1, 64, V.DT_F32, cfg) == V.MMA_MAX_SPLIT_LOG2
    off = S.DeviceConfig.from_env({"PJRT_AMD_MMA_SPLITK": "0", "PJRT_OCL_NLANES": "128"})
    assert S.mma_split_log2(256, 64, 512, 1, 64, V.DT_F32, off) == 0
    g = G.Graph()
    x, w = g.input((256, 512)), g.input((512, 64))
    g.output(g.dot(x, w))
    t = S.schedule_program(g.build(), S.DeviceConfig(nlanes=128, fit_lanes=False)).tasks[0]
    assert t.p3 >> V.MMA_SPLIT_SHIFT == 4
    assert S.n_tiles(t, S.DeviceConfig(nlanes=128)) == 4 * 16


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("Gb,M,K,N", [(1, 256, 512, 64), (2, 100, 300, 70), (1, 64, 1000, 128)])
def test_mma_split_k_tiles_exact(dt, Gb, M, K, N):
    """Integer-valued operands give an exact product however K is cut: the lane
    simulator (tiles in forward and reverse lane order, each output tile written
    once all its splits have run) gives the float64 product bit for bit, with a
    bias + relu epilogue on the combined sum."""
    from oracle import vmref
    rng = np.random.default_rng(8)
    a = rng.integers(-3, 4, (Gb, M, K)).astype(np.float32)
    b = rng.integers(-3, 4, (Gb, K, N)).astype(np.float32)
    bias = rng.integers(-9, 10, N).astype(np.float32)
    g = G.Graph()
    x, y, bb = g.input(a.shape, dt), g.input(b.shape, dt), g.input(bias.shape)
    g.output(g.dot(x, y, residual=bb, epilogue=[(V.SUB_ADD, 2, 0.0, 0.0), (V.SUB_MAX, 3, 0.0, 0.0)]))
    prog = g.build()
    sched = S.schedule_program(prog, S.DeviceConfig(nlanes=128, fit_lanes=False))
    assert sched.tasks[0].p3 >> V.MMA_SPLIT_SHIFT >= 1
    blob = V.serialize(prog, sched)
    got = vmref.execute_schedule(blob, [a, b, bias])[0]
    want = np.maximum(np.matmul(a.astype(np.float64), b.astype(np.float64)) + bias, 0.0)
    np.testing.assert_array_equal(got, want.astype(np.float32))


# --- skinny matmuls as split-K TOP_GEMV tasks ----------------------------------------

@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("Gb,M,K,N", [(1, 1, 5, 8), (1, 3, 64, 264), (3, 8, 300, 1000), (1, 1, 3072, 768)])
def test_gemv_split_k_tiles_exact(dt, Gb, M, K, N):
    """Integer-valued operands: every partial sum is exact, so the lane simulator
    (tiles in forward and reverse lane order) must give the float64 product bit
    for bit."""
    from oracle import vmref
    rng = np.random.default_rng(7)
    a = rng.integers(-3, 4, (Gb, M, K)).astype(np.float32)
    b = rng.integers(-3, 4, (Gb, K, N)).astype(np.float32)
    g = G.Graph()
    x, y = g.input(a.shape, dt), g.input(b.shape, dt)
    g.output(g.dot(x, y))
    prog = g.build()
    cfg = S.DeviceConfig(nlanes=16)
    sched = S.schedule_program(prog, cfg)
    gemv = [t for t in sched.tasks if t.tile_op == V.TOP_GEMV]
    assert len(gemv) == 1 and gemv[0].p4 % 8 == 0
    blob = V.serialize(prog, sched)
    got = vmref.execute_schedule(blob, [a, b])[0]
    np.testing.assert_array_equal(got, np.matmul(a.astype(np.float64), b.astype(np.float64)))


def test_gemv_epilogue_matches_tensor_semantics():
    from oracle import vmref
    rng = np.random.default_rng(8)
    M, K, N = 2, 96, 520
    a = rng.standard_normal((M, K)).astype(np.float32)
    b = rng.standard_normal((K, N)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    g = G.Graph()
    x, y, bb = g.input(a.shape), g.input(b.shape), g.input(bias.shape)
    g.output(g.dot(x, y, residual=bb, epilogue=[(V.SUB_ADD, 2, 0.0, 0.0), (V.SUB_GELU, 0, 0.0, 0.0)]))
    prog = g.build()
    blob = V.serialize(prog, S.schedule_program(prog, S.DeviceConfig(nlanes=32)))
    got = vmref.execute_schedule(blob, [a, b, bias])[0]
    want = vmref.execute(blob, [a, b, bias])[0]            # tensor level: one matmul
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)


def test_gemv_strips_cover_lanes():
    for N, G_, want in [(2304, 1, 16), (32000, 1, 128), (768, 1, 8), (640, 12, 32), (64, 12, 8),
                        (8, 1, 8), (4096, 16, 256)]:
        cw = S.gemv_strip(N, G_, 256)
        assert cw == want and G_ * -(-N // cw) <= max(256, G_)
    assert S.gemv_strip(768, 1, 256, min_strip=16) == 16 and S.gemv_strip(3072, 1, 256, min_strip=16) == 16


def test_gemv_lds_bound_falls_back_to_mma():
    g = G.Graph()
    x, w = g.input((8, 3072), "bf16"), g.input((3072, 64), "bf16")
    g.output(g.dot(x, w))
    sched = S.schedule_program(g.build(), S.DeviceConfig(nlanes=16))
    assert [t.tile_op for t in sched.tasks] == [V.TOP_MMA]


def test_gemv_not_chosen_for_views_or_wide_m():
    g = G.Graph()
    x, w = g.input((16, 64), "bf16"), g.input((64, 128), "bf16")
    wt = g.input((128, 64), "bf16")
    g.output(g.dot(x, w), g.dot(g.slice(x, (0, 0), (1, 64)), g.transpose_view(wt, (1, 0))))
    sched = S.schedule_program(g.build(), S.DeviceConfig(nlanes=16))
    assert all(t.tile_op != V.TOP_GEMV for t in sched.tasks)


def test_alias_shares_memory_and_orders_like_its_parent():
    """An alias is a buffer placed inside its parent's bytes (no arena of its
    own), and the scheduler separates a write of the parent from a read of the
    alias by a barrier, like two accesses to one buffer."""
    g = G.Graph()
    x = g.input((4, 96))
    w = g.input((96, 96))
    y = g.dot(x, w)                                   # writes y on several lanes
    hi = g.alias(y, 2 * 96, (2, 96))                  # rows 2..3 of y, in place
    z = g.reduce_last(hi, V.RED_SUM)                  # reads the alias
    g.output(z)
    prog = g.build()
    assert prog.buffers[hi.buf].arena_byte_offset == prog.buffers[y.buf].arena_byte_offset + 2 * 96 * 4
    assert prog.buffers[hi.buf].size_bytes == 2 * 96 * 4
    grp = S.overlap_groups(prog)
    assert grp[hi.buf] == grp[y.buf] and grp[x.buf] != grp[y.buf]
    sched = S.schedule_program(prog, S.DeviceConfig(nlanes=8, mma_t=64))
    assert len(phases(sched)) == 2
    rng = np.random.default_rng(1007)
    a = rng.integers(-4, 5, (4, 96)).astype(np.float32)
    b = rng.integers(-4, 5, (96, 96)).astype(np.float32)
    out = vmref.execute_schedule(V.serialize(prog, sched), [a, b])
    np.testing.assert_array_equal(out[0], (a @ b)[2:].sum(-1))


def test_alias_rejects_unaligned_or_outside():
    g = G.Graph()
    y = g.input((10,), "bf16")
    with pytest.raises(G.GraphError):
        g.alias(y, 3, (2,))                           # 6-byte offset
    with pytest.raises(G.GraphError):
        g.alias(y, 8, (4,))                           # past the end


def test_decode_attention_task_and_cache_update_overlap():
    """OP_DECODE_ATTN lowers to one TOP_DECODE_ATTN tile per head; the cache
    update that follows it (write after read of the caches) starts the next
    phase and shares it with the output projection, which reads neither cache."""
    H, hd, C, D = 4, 16, 32, 64
    g = G.Graph()
    qkv = g.input((1, 3 * D), "bf16")
    ck, cv = g.fill((H, hd, C), 0.0, "bf16"), g.fill((H, C, hd), 0.0, "bf16")
    pos = g.fill((), 5, "i32")
    zero = g.scalar(0, "i32")
    w = g.input((D, D), "bf16")
    q, k, v = (g.alias(qkv, s * D, (H, hd)) for s in range(3))
    att = g.decode_attention(q, k, v, ck, cv, pos, 0.25)
    g.dynamic_update_slice(ck, g.reshape(k, (H, hd, 1)), [zero, zero, pos])
    g.dynamic_update_slice(cv, g.reshape(v, (H, 1, hd)), [zero, pos, zero])
    g.output(g.dot(g.reshape(att, (1, D)), w))
    prog = g.build()
    sched = S.schedule_program(prog, S.DeviceConfig(nlanes=8))
    da = [i for i, t in enumerate(sched.tasks) if t.tile_op == V.TOP_DECODE_ATTN]
    assert len(da) == 1
    t = sched.tasks[da[0]]
    assert (t.p4 & 0xFFFF, t.p5, t.p6) == (H, hd, C)
    assert S.n_tiles(t, S.DeviceConfig(nlanes=8)) == H * max(1, t.p4 >> 16)
    ph = phases(sched)
    at = next(i for i, p in enumerate(ph) if da[0] in p)
    later = {sched.tasks[x].tile_op for x in ph[at + 1]}
    assert V.TOP_DYN_SCATTER in later and (V.TOP_GEMV in later or V.TOP_MMA in later)


def test_decode_attention_rejects_bad_shapes():
    g = G.Graph()
    q = g.input((2, 8))
    pos = g.input((), "i32")
    with pytest.raises(G.GraphError):      # C not a multiple of 8
        g.decode_attention(q, q, q, g.input((2, 8, 12)), g.input((2, 12, 8)), pos, 1.0)
    with pytest.raises(G.GraphError):      # V cache shape
        g.decode_attention(q, q, q, g.input((2, 8, 16)), g.input((2, 8, 16)), pos, 1.0)
    with pytest.raises(G.GraphError):      # mixed dtypes
        g.decode_attention(q, q, q, g.input((2, 8, 16), "bf16"), g.input((2, 16, 8), "bf16"), pos, 1.0)
    with pytest.raises(G.GraphError):      # pos must be i32
        g.decode_attention(q, q, q, g.input((2, 8, 16)), g.input((2, 16, 8)), g.input(()), 1.0)


def test_gpt_decode_phases_per_layer():
    """The C5 decode body: 5 barrier-separated phases per layer (QKV with its
    layernorm staged inside and the attention-residual add, attention, cache
    update with the output projection, FC with its layernorm and the
    MLP-residual add, projection)."""
    import dataclasses
    from pjrt_amd import configs as CF
    counts = {}
    for layers in (1, 2):
        c = dataclasses.replace(CF.C5, layers=layers, steps=4, vocab=512)
        prog = CF.gpt_c5(c, trips=4)
        fo = next(x for x in prog.instrs if x.op == V.OP_FOR)
        sc = S._Scheduler(prog, S.DeviceConfig(nlanes=256))
        counts[layers] = len(sc.levels(list(range(fo.n, fo.n + fo.imm))))
    assert counts[2] - counts[1] == 5


def _ln_dot(extra=None):
    g = G.Graph()
    x = g.input((1, 64))
    gam, bet = g.input((64,)), g.input((64,))
    w = g.input((64, 32), "bf16")
    h = g.layernorm(x, gam, bet, 1e-5, out_dtype="bf16")
    if extra:
        extra(g, x, h)
    g.output(g.dot(h, w))
    return g.build()


def test_ln_gemv_prologue_fuses_single_reader():
    """A layernorm read only by a GEMV runs inside it: the GEMV task's p5 names
    the layernorm task, which no lane runs, and the program has one phase."""
    prog = _ln_dot()
    cfg = S.DeviceConfig(nlanes=8)
    sched = S.schedule_program(prog, cfg)
    gv = [t for t in sched.tasks if t.tile_op == V.TOP_GEMV]
    assert len(gv) == 1 and gv[0].p5
    ln = gv[0].p5 - 1
    assert sched.tasks[ln].tile_op == V.TOP_LAYERNORM_SEG
    assert all(e.task != ln for st in sched.lane_streams for e in st)
    assert len(phases(sched)) == 1
    off = S.schedule_program(prog, S.DeviceConfig(nlanes=8, ln_gemv=False))
    assert len(phases(off)) == 2 and not any(t.p5 for t in off.tasks if t.tile_op == V.TOP_GEMV)


@pytest.mark.parametrize("case", ["second_reader", "input_written", "output"])
def test_ln_gemv_prologue_not_fused(case):
    def second_reader(g, x, h):
        g.output(g.convert(h, "f32"))

    def input_written(g, x, h):
        g.copy_into(x, g.add(x, x))

    def output(g, x, h):
        g.output(h)

    prog = _ln_dot({"second_reader": second_reader, "input_written": input_written, "output": output}[case])
    assert S.ln_gemv_pairs(prog, S.DeviceConfig(nlanes=8)) == {}


def test_decode_splits():
    cfg = S.DeviceConfig(nlanes=256)
    assert S.decode_splits(12, 640, cfg) == 10          # 64 keys each
    assert S.decode_splits(12, 4096, cfg) == 64
    assert S.decode_splits(300, 72, cfg) == 2
    assert S.decode_splits(2, 16, cfg) == 1


def test_layernorm_row_interleave():
    """LAYERNORM_SEG p5: set when the rows are a multiple of the lanes; the
    lane simulator (which applies it) still equals the tensor interpreter."""
    assert S.row_interleave(8192, S.DeviceConfig(nlanes=256)) == 32
    assert S.row_interleave(8191, S.DeviceConfig(nlanes=256)) == 0
    assert S.row_interleave(256, S.DeviceConfig(nlanes=256)) == 0
    g = G.Graph()
    x = g.input((32, 24))
    ga, be = g.input((24,)), g.input((24,))
    g.output(g.layernorm(x, ga, be, 1e-5, gelu=True))
    prog = g.build()
    blob = V.serialize(prog, S.schedule_program(prog, S.DeviceConfig(nlanes=4)))
    assert any(t.top == V.TOP_LAYERNORM_SEG and t.p[5] == 8 for t in vmref.parse(blob).tasks)
    rng = np.random.default_rng(3)
    args = [rng.standard_normal((32, 24)).astype(np.float32), rng.uniform(0.5, 1.5, 24).astype(np.float32),
            rng.normal(0, 0.1, 24).astype(np.float32)]
    np.testing.assert_array_equal(vmref.execute_schedule(blob, args)[0], vmref.execute(blob, args)[0])


def test_lane_fit():
    """A program of many small phases (the decode loop, scheduled with grid
    barriers only) runs on half the lanes; bandwidth- and MFMA-bound programs
    keep every lane."""
    import dataclasses
    from pjrt_amd import configs as CF
    cfg = S.DeviceConfig(nlanes=256, counters=False)
    dec = CF.gpt_c5(dataclasses.replace(CF.C5, layers=2, steps=8))
    assert S.lane_fit(dec, cfg) == 128
    assert S.schedule_program(dec, cfg).n_lanes == 128
    assert S.schedule_program(dec, dataclasses.replace(cfg, fit_lanes=False)).n_lanes == 256
    assert S.lane_fit(dec, S.DeviceConfig(nlanes=7)) == 7
    g = G.Graph()
    x = g.input((8192, 4096))
    ga, be = g.input((4096,)), g.input((4096,))
    g.output(g.layernorm(x, ga, be, 1e-5, gelu=True, out_dtype="bf16"))
    assert S.lane_fit(g.build(), cfg) == 256
    g = G.Graph()
    a, b = g.input((4096, 4096), "bf16"), g.input((4096, 4096), "bf16")
    g.output(g.dot(a, b))
    assert S.lane_fit(g.build(), cfg) == 256
    # the FOR body's phases count once per trip
    one = S._schedule(dec, dataclasses.replace(cfg, fit_lanes=False)).est
    dec16 = CF.gpt_c5(dataclasses.replace(CF.C5, layers=2, steps=16))
    assert S._schedule(dec16, dataclasses.replace(cfg, fit_lanes=False)).est > 1.5 * one


def test_lane_count_defaults():
    """Strip floor and idle master follow the lane count unless set."""
    assert S.gemv_strip_floor(S.DeviceConfig(nlanes=256)) == 8
    assert S.gemv_strip_floor(S.DeviceConfig(nlanes=128)) == 16
    assert S.gemv_strip_floor(S.DeviceConfig(nlanes=128, gemv_min_strip=8)) == 8
    assert S.gemv_strip_floor(S.DeviceConfig(nlanes=256, gemv_min_strip=3)) == 8
    assert S.master_idle(S.DeviceConfig(nlanes=256)) is True
    assert S.master_idle(S.DeviceConfig(nlanes=128)) is False
    assert S.master_idle(S.DeviceConfig(nlanes=128, idle_master=True)) is True
    env = S.DeviceConfig.from_env({"PJRT_AMD_GEMV_STRIP": "8", "PJRT_AMD_IDLE_MASTER": "1"})
    assert env.gemv_min_strip == 8 and env.idle_master is True
    env = S.DeviceConfig.from_env({})
    assert env.gemv_min_strip == 0 and env.idle_master is None


def test_viewed_operand_is_a_cross_lane_dependency():
    """y = 2 x, then z = transpose(y) + w with the transpose folded into z's
    operand view: same element count, but z's tile t reads y elements other lanes
    write, so a barrier must separate them.  The oracle's lane simulator runs the
    lanes forward and in reverse and catches the race if it is scheduled
    lane-local."""
    n = 64
    g = G.Graph()
    x, w = g.input((n, n)), g.input((n, n))
    y = g.affine(x, 2.0, 0.0)
    z = g.add(g.transpose_view(y, (1, 0)), w)
    g.output(z)
    prog = g.build()
    cfg = S.DeviceConfig(nlanes=4, ew_ts=256, mma_t=64)
    blob = V.serialize(prog, S.schedule_program(prog, cfg))
    sched = vmref.parse(blob)
    assert sum(e[0] == V.ENT_BARRIER for e in sched.streams[0]) >= 1
    rng = np.random.default_rng(3)
    xv, wv = rng.standard_normal((n, n)).astype(np.float32), rng.standard_normal((n, n)).astype(np.float32)
    (got,) = vmref.execute_schedule(blob, [xv, wv], ew_ts=256, mma_t=64)
    np.testing.assert_array_equal(got, (2 * xv).T + wv)


def test_cost_table_forms_and_model_terms(tmp_path):
    """PJRT_OCL_COST_TABLE as a file path (the reference's form) or inline JSON;
    the measured terms replace the work model's constants, unknown keys and
    non-positive values are ignored."""
    table = {"ew_tile_us": 2.5, "tile_us": 1.25, "lane_gbs": 20.0, "barrier_us": 3.0,
             "barrier_us_per_lane": 0.01, "lane_mma_tflops": 8.0, "bogus": 1.0, "gather_tile_us": -1}
    p = tmp_path / "costs.json"
    p.write_text(json.dumps(table))
    for spec in (str(p), json.dumps(table)):
        cfg = S.DeviceConfig.from_env({"PJRT_OCL_COST_TABLE": spec})
        assert cfg.costs == {k: v for k, v in table.items() if k not in ("bogus", "gather_tile_us")}
        assert S.model_terms(cfg) == (1.25, 20.0, 8.0, 3.0, 0.01)
    assert S.DeviceConfig.from_env({"PJRT_OCL_COST_TABLE": "/nonexistent.json"}).costs == {}


def test_lane_fit_follows_the_measured_barrier_cost():
    """A barrier-heavy program (a FOR loop of one small EW per trip) moves to
    half the lanes when barriers cost more per lane, and stays when they cost
    nothing."""
    g = G.Graph()
    x = g.input((4096,))
    a = g.fill((4096,), 0.0)
    g.copy_into(a, x)
    g.begin()
    g.copy_into(a, g.add(a, g.broadcast_view(g.scalar(1.0), (4096,), ())))
    g.for_loop(64, g.end())
    g.output(a)
    prog = g.build()
    cheap = S.DeviceConfig(nlanes=256, costs={"barrier_us": 0.01, "barrier_us_per_lane": 0.0})
    dear = S.DeviceConfig(nlanes=256, costs={"barrier_us": 1.0, "barrier_us_per_lane": 0.5})
    assert S.lane_fit(prog, cheap) == 256
    assert S.lane_fit(prog, dear) == 128


def test_residual_buffer_zero_is_a_read():
    """A matmul epilogue's residual that is buffer 0 (the first input) is read:
    the id is no 'no residual' marker, the epilogue's sources say so."""
    g = G.Graph()
    x = g.input((1, 16))
    w = g.input((16, 16))
    y = g.dot(x, w, residual=x, epilogue=[(V.SUB_ADD, 1, 0.0, 0.0)])
    g.output(y)
    prog = g.build()
    (dot,) = [i for i in prog.instrs if i.op == V.OP_DOT]
    assert x.buf == 0 and 0 in S.instr_reads(dot, prog)
    g2 = G.Graph()
    x2, w2 = g2.input((1, 16)), g2.input((16, 16))
    g2.output(g2.dot(x2, w2))
    (dot2,) = [i for i in g2.build().instrs if i.op == V.OP_DOT]
    assert S.instr_reads(dot2, g2.build()) == {0, 1}


# --- completion flags (extension of the WAIT / SIGNAL entry fields) -------------------

def _decoder(counters, nlanes=16):
    import dataclasses
    from pjrt_amd import configs as CF
    c = CF.GptConfig(layers=2, d=128, heads=4, mlp=256, vocab=300, prompt=32, steps=3)
    prog = CF.gpt_c5(c, emit_logits=True)
    cfg = S.DeviceConfig(nlanes=nlanes, counters=counters, fit_lanes=False)
    sched = S.schedule_program(prog, cfg)
    return c, prog, sched, cfg


def _segments(stream):
    """The lane's entries split at its barriers (one list per phase)."""
    out = [[]]
    for e in stream:
        if e.task == V.ENT_BARRIER:
            out.append([])
        elif e.task not in V.CONTROL_SENTINELS:
            out[-1].append(e)
    return out


def test_counters_join_decode_attention_to_its_qkv_phase():
    """With completion flags each layer's decode attention runs in its QKV
    GEMV's phase (one grid barrier fewer per layer, per decode step); every
    attention entry waits for exactly the flags of the strips that write its
    heads' q, k and v (recomputed here from the arena byte ranges), every
    signaling entry comes before any waiting entry of its lane and phase, and
    the schedule computes what the barrier-only one computes, in both lane
    orders of the oracle's simulator."""
    from pjrt_amd import configs as CF
    c, prog, on, cfg = _decoder(True)
    _, _, off, _ = _decoder(False)
    nbar = lambda sc: sum(1 for e in sc.lane_streams[0] if e.task == V.ENT_BARRIER)
    assert nbar(off) - nbar(on) == c.layers            # the FOR body is scheduled once
    assert on.n_flags > 0 and off.n_flags == 0
    bufs = prog.buffers
    # who signals what, and the bytes each signaling GEMV entry writes
    signal = {}
    for s in on.lane_streams:
        for e in s:
            if e.task not in V.CONTROL_SENTINELS and e.signal_flag != V.FLAG_NONE:
                assert e.signal_flag not in signal
                t = on.tasks[e.task]
                assert t.tile_op == V.TOP_GEMV
                dst = next(b for b in range(len(bufs)) if bufs[b].arena_byte_offset == bufs[t.dst].arena_byte_offset
                           and bufs[b].size_bytes == bufs[t.dst].size_bytes)
                es = V.DT_SIZE[bufs[dst].dtype]
                lo = bufs[dst].arena_byte_offset + e.tile_lo * t.p4 * es
                hi = bufs[dst].arena_byte_offset + min(e.tile_hi * t.p4, t.p1) * es
                signal[e.signal_flag] = (e.task, lo, hi)
    assert sorted(signal) == list(range(on.n_flags))
    waits = 0
    for s in on.lane_streams:
        for seg in _segments(s):
            seen_wait = False
            for e in seg:
                if e.wait_count:
                    seen_wait = True
                    waits += 1
                    t = on.tasks[e.task]
                    assert t.tile_op == V.TOP_DECODE_ATTN
                    H, Sp = t.p4 & 0xFFFF, max(1, t.p4 >> 16)
                    hd = t.p5 & 0xFFFF
                    es = V.DT_SIZE[bufs[t.a].dtype]
                    heads = range(e.tile_lo // Sp, (e.tile_hi - 1) // Sp + 1)
                    need = set()
                    for f, (_, lo, hi) in signal.items():
                        for b in (t.a, t.p1, t.p2):           # q, k, v
                            o = bufs[b].arena_byte_offset
                            if any(lo < o + (h + 1) * hd * es and o + h * hd * es < hi for h in heads):
                                need.add(f)
                    assert set(range(e.wait_flag, e.wait_flag + e.wait_count)) == need
                elif e.signal_flag != V.FLAG_NONE:
                    assert not seen_wait
    assert waits >= c.layers
    args = CF.gpt_inputs(c, seed=11)
    a = vmref.execute_schedule(V.serialize(prog, on), args)
    b = vmref.execute_schedule(V.serialize(prog, off), args)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)
    want_tok, want_logits = CF.gpt_reference(c, args)
    np.testing.assert_array_equal(np.concatenate(a[:2]), want_tok)


def test_counters_off_by_switch_and_for_other_consumers():
    """PJRT_AMD_COUNTERS=0 keeps every barrier; a phase whose consumer is not a
    decode attention fed by GEMV strips is never joined."""
    cfg = S.DeviceConfig.from_env({"PJRT_AMD_COUNTERS": "0"})
    assert not cfg.counters
    g = G.Graph()
    x, w = g.input((1, 256)), g.input((256, 512))
    y = g.dot(x, w)
    g.output(g.reduce_last(y, V.RED_SUM))
    sched = S.schedule_program(g.build(), S.DeviceConfig(nlanes=16, fit_lanes=False))
    assert sched.n_flags == 0
    assert all(e.wait_count == 0 and e.signal_flag == V.FLAG_NONE
               for s in sched.lane_streams for e in s if e.task not in V.CONTROL_SENTINELS)


def test_oracle_rejects_bad_completion_flags():
    """The oracle's parser rejects a flag signaled twice or a wait outside
    n_flags, and its simulator reports a wait no entry of the phase signals."""
    import dataclasses
    c, prog, on, cfg = _decoder(True)
    args = None

    def mutate(fn):
        streams = [[dataclasses.replace(e) for e in s] for s in on.lane_streams]
        fn(streams)
        return V.serialize(prog, V.Schedule(on.n_lanes, on.tasks, streams, on.root_lens, on.n_flags))

    sig = [(l, k) for l, s in enumerate(on.lane_streams) for k, e in enumerate(s)
           if e.task not in V.CONTROL_SENTINELS and e.signal_flag != V.FLAG_NONE]
    wt = [(l, k) for l, s in enumerate(on.lane_streams) for k, e in enumerate(s)
          if e.task not in V.CONTROL_SENTINELS and e.wait_count]

    def twice(st):
        (l0, k0), (l1, k1) = sig[0], sig[1]
        st[l1][k1].signal_flag = st[l0][k0].signal_flag

    def outside(st):
        l, k = wt[0]
        st[l][k].wait_count = on.n_flags + 1 - st[l][k].wait_flag

    for fn in (twice, outside):
        with pytest.raises(vmref.FormatError):
            vmref.parse(mutate(fn))

    def unsignaled(st):          # the first producer of a waited range stops signaling
        l, k = wt[0]
        f = st[l][k].wait_flag
        for ls, ks in sig:
            if st[ls][ks].signal_flag == f:
                st[ls][ks].signal_flag = V.FLAG_NONE
    from pjrt_amd import configs as CF
    with pytest.raises(AssertionError, match="completion flags"):
        vmref.execute_schedule(mutate(unsignaled), CF.gpt_inputs(c, seed=11))
