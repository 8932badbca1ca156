"""The allocation-free entry point (vmrt_run_noalloc, through the C ABI) gives the
results of vmrt_load + vmrt_execute on the same program and device buffers, on two
calls in a row -- the second a smaller program, so the static array still holds
the first call's contents -- and rejects a program larger than its array.

The programs use task scratch: a split argmax (rows of 8192 or more elements are
cut into runs on separate CUs, combined by the last arriving split through
arrival counters) and a split decode attention (64 cache keys per split), so a
counter or partial left over from the previous call would show."""
import numpy as np
import pytest

from gpu_util import blob_for, runtime
from oracle import vmref
from pjrt_amd import graph as G
from pjrt_amd import vmprogram as V
from pjrt_amd.runtime import RESOURCE_EXHAUSTED, VmrtError

pytestmark = pytest.mark.gpu


def _program(rows, seg, H, hd, C, seed):
    rng = np.random.default_rng(seed)
    g = G.Graph()
    X = g.input((rows, seg))
    Q, K, Vv = (g.input((H, hd), "bf16") for _ in range(3))
    CK, CV = g.input((H, hd, C), "bf16"), g.input((H, C, hd), "bf16")
    POS = g.input((), "i32")
    val, idx = g.argmax_last(X)
    att = g.decode_attention(Q, K, Vv, CK, CV, POS, 1.0 / np.sqrt(hd))
    g.output(idx, val, att)
    x = rng.standard_normal((rows, seg)).astype(np.float32)
    x[:, rng.integers(0, seg, rows)] = 7.0               # ties: the first index wins
    args = [x] + [V.f32_to_bf16(rng.standard_normal(s).astype(np.float32))
                  for s in ((H, hd), (H, hd), (H, hd), (H, hd, C), (H, C, hd))]
    args.append(np.array(C - 3, np.int32))
    return g.build(), args


def _device(rt, arrays):
    return [rt.to_device(np.ascontiguousarray(a)) for a in arrays]


@pytest.mark.parametrize("order", ["big_then_small"])
def test_noalloc_matches_execute_twice(order):
    rt = runtime()
    cases = [_program(6, 32000, 12, 64, 640, 1), _program(3, 9000, 4, 64, 128, 2)]
    for k, (prog, args) in enumerate(cases):
        blob, cfg = blob_for(prog)
        tasks = vmref.parse(blob).tasks
        assert any(t.top == V.TOP_ARGMAX_SEG and t.p[3] > 1 for t in tasks), "argmax not split"
        assert any(t.top == V.TOP_DECODE_ATTN and (t.p[4] >> 16) > 1 for t in tasks), "attention not split"
        dev_in = _device(rt, args)
        lp = rt.load(blob, ew_ts=cfg.ew_ts, mma_t=cfg.mma_t)
        want_bufs = lp.execute(dev_in)
        got_bufs = lp.alloc_outputs()
        rt.run_noalloc(blob, dev_in, got_bufs, ew_ts=cfg.ew_ts, mma_t=cfg.mma_t)
        for o, (w, gbuf) in enumerate(zip(want_bufs, got_bufs)):
            wv, gv = w.to_host(), gbuf.to_host()
            assert np.array_equal(wv, gv), f"case {k} output {o} differs from vmrt_execute"
        # the argmax indices are the oracle's too (exact integer results)
        want = vmref.execute(blob, args, ew_ts=cfg.ew_ts, mma_t=cfg.mma_t)
        assert np.array_equal(got_bufs[0].to_host(np.int32), want[0].reshape(-1))
        lp.close()
        for b in dev_in + want_bufs + got_bufs:
            b.free()


def test_noalloc_rejects_a_program_beyond_its_array():
    g = G.Graph()
    x = g.input((5 << 20,))                 # 20 MiB in, 20 MiB each for two temporaries
    y = g.add(x, x)
    z = g.mul(y, y)
    g.output(g.sub(z, x))
    blob, cfg = blob_for(g.build())
    rt = runtime()
    xin = rt.alloc(5 << 22)
    out = rt.alloc(5 << 22)
    with pytest.raises(VmrtError) as e:
        rt.run_noalloc(blob, [xin], [out], ew_ts=cfg.ew_ts, mma_t=cfg.mma_t)
    assert e.value.code == RESOURCE_EXHAUSTED and "at most" in e.value.message
    xin.free()
    out.free()
