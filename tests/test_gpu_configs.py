"""Configs 1 and 5 end to end on the GPU, against the CPU oracle.

Greedy decoding compares tokens step by step while the oracle's choice is
unambiguous: at each step the logits must agree within the tolerance, and the
tokens must be equal unless the oracle's top-two logits are closer than twice
that tolerance (then either token is a correct greedy choice and the two runs
may diverge from there on, as the reference's own JAX comparison would).  The
logit tolerance is 5e-3 of the largest logit: bf16 activations through 12
layers, f32 accumulation."""
import dataclasses
import sys

import numpy as np
import pytest

from gpu_util import assert_rel, blob_for, check_decoder, run_both, run_gpu, runtime
from oracle import vmref
from pjrt_amd import configs as CF

pytestmark = pytest.mark.gpu


def test_mlp_c1_full_size():
    args = CF.mlp_c1_inputs()
    got, want = run_both(CF.mlp_c1(), args, oracle="tensor")
    assert_rel(got[0], want[0], 1e-3, 1e-5, "config 1")
    x, w1, b1, w2, b2 = (a.astype(np.float64) for a in args)
    assert_rel(got[0], np.maximum(x @ w1 + b1, 0) @ w2 + b2, 1e-3, 1e-5, "config 1 vs numpy")


def test_gpt_c5_small():
    c = CF.GptConfig(layers=2, d=128, heads=2, mlp=512, vocab=1000, prompt=128, steps=16)
    args = CF.gpt_inputs(c, seed=11)
    got, want = run_both(CF.gpt_c5(c, emit_logits=True), args, oracle="tensor")
    check_decoder(got, want, 5e-3, pinned=17, what="small decoder")


def test_gpt_c5_full_size_first_steps():
    """The full config-5 model (12 layers, d 768, vocab 32000, 512-token prompt)
    for the prefill and the first three decode steps."""
    c = dataclasses.replace(CF.C5, steps=3)
    args = CF.gpt_inputs(c)
    got, want = run_both(CF.gpt_c5(c, emit_logits=True), args, oracle="tensor")
    check_decoder(got, want, 5e-3, pinned=4, what="config-5 decoder, 3 steps")


def test_gpt_c5_full_program_deterministic():
    """The benchmarked program (128 decode steps): two executions give identical
    tokens, all inside the vocabulary."""
    args = CF.gpt_inputs(CF.C5)
    blob, _ = blob_for(CF.gpt_c5(CF.C5))
    lp = runtime().load(blob)
    try:
        a = lp(*args)
        b = lp(*args)
    finally:
        lp.close()
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)
    toks = np.concatenate(a)
    assert toks.shape == (CF.C5.steps + 1,) and toks.min() >= 0 and toks.max() < CF.C5.vocab


def test_gpt_c5_lane_fit_matches_every_lane():
    """The decode program scheduled on half the lanes (lane_fit, with its
    lane-count defaults) gives the tokens of the same program on every lane
    (16 steps: with fewer, the prefill dominates and every lane is kept)."""
    c = dataclasses.replace(CF.C5, steps=16)
    prog = CF.gpt_c5(c, emit_logits=True)
    args = CF.gpt_inputs(c)
    # barrier-only schedules: the work model's lane choice was fitted on them
    fit, _ = blob_for(prog, counters=False)
    full, _ = blob_for(prog, fit_lanes=False, counters=False)
    lanes = vmref.parse(fit).n_lanes, vmref.parse(full).n_lanes
    print(f"[gpu] lane fit: {lanes[0]} lanes against {lanes[1]}", file=sys.stderr, flush=True)
    if runtime().info["n_lanes"] >= 128:
        assert lanes[0] == lanes[1] // 2
    got = run_gpu(fit, args)
    want = run_gpu(full, args)
    # the strip width, and with it the summation order of the bf16 GEMVs,
    # differs between the two schedules: the bf16 decoder tolerance applies
    check_decoder(got, want, 5e-3, pinned=17, what="half-lane vs all-lane decoder")


def _lowered_decoder(c):
    from pjrt_amd import lowering as L
    from pjrt_amd import stablehlo_configs as SC
    return L.lower_text(SC.gpt_decode(c, emit_logits=True))


def test_lowered_gpt_decode_small():
    """Config 5 as the JAX program, through the lowering (decode attention
    fused, caches updated in place): the GPU against the oracle."""
    c = CF.GptConfig(layers=2, d=128, heads=2, mlp=512, vocab=1000, prompt=128, steps=16)
    args = CF.gpt_inputs(c, seed=11)
    got, want = run_both(_lowered_decoder(c), args, oracle="tensor")
    check_decoder(got, want, 5e-3, pinned=17, what="lowered small decoder")


def test_lowered_gpt_decode_full_size_first_steps():
    """The lowered full config-5 program (12 layers, d 768, vocab 32000,
    512-token prompt) for the prefill and three decode steps, and beside it the
    hand-built program on the same inputs."""
    c = dataclasses.replace(CF.C5, steps=3)
    args = CF.gpt_inputs(c)
    prog = _lowered_decoder(c)
    got, want = run_both(prog, args, oracle="tensor")
    check_decoder(got, want, 5e-3, pinned=4, what="lowered decoder, 3 steps")
    hand, _ = blob_for(CF.gpt_c5(c, emit_logits=True))
    check_decoder(got, run_gpu(hand, args), 5e-3, pinned=4, what="lowered vs hand-built decoder")


@pytest.mark.parametrize("name", ["small", "base"])
def test_reference_decode_step(name):
    """One token of the reference's decode benchmark (tools/bench_decode.py,
    f32, keys and values appended by concatenate), lowered: the GPU against
    the oracle and against the float64 numpy statement of the step."""
    import hlo_programs as HP
    from pjrt_amd import lowering as L
    from pjrt_amd import stablehlo_configs as SC
    cfg = SC.DECODE_STEP_CONFIGS[name]
    args = SC.decode_step_inputs(cfg, seed=1)
    got, want = run_both(L.lower_text(SC.decode_step(cfg)), args, oracle="tensor")
    ref = HP.decode_step_reference(cfg, args)
    atol = 1e-4 * float(np.abs(ref).max())          # f32 GEMVs: summation order differs
    assert_rel(got[0], want[0], 1e-4, atol, f"decode step {name} vs oracle")
    assert_rel(got[0], ref, 1e-4, atol, f"decode step {name} vs numpy")


@pytest.mark.parametrize("full", [False, True])
def test_decoder_completion_flags_match_barriers(full):
    """The decoder scheduled with completion flags (each layer's decode
    attention in its QKV GEMV's phase, waiting for its head's strips) gives
    bit-identical tokens and logits to the same program scheduled with grid
    barriers only: the tiles and their summation orders are the same, only the
    synchronisation differs."""
    c = dataclasses.replace(CF.C5, steps=16) if full else CF.GptConfig(layers=2, d=128, heads=2, mlp=512,
                                                                      vocab=1000, prompt=128, steps=16)
    prog = CF.gpt_c5(c, emit_logits=True)
    args = CF.gpt_inputs(c, seed=11)
    # one lane count for both (the strip widths, and so the summation orders,
    # follow it): half the device's, as the benchmarked decoder runs
    lanes = max(1, runtime().info["n_lanes"] // 2)
    on, _ = blob_for(prog, nlanes=lanes, fit_lanes=False, counters=True)
    off, _ = blob_for(prog, nlanes=lanes, fit_lanes=False, counters=False)
    assert vmref.parse(on).n_flags > 0 and vmref.parse(off).n_flags == 0
    a, b = run_gpu(on, args), run_gpu(off, args)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)
    if not full:
        _, want = run_both(on, args, oracle="tensor")
        check_decoder(a, want, 5e-3, pinned=17, what="small decoder with completion flags")
