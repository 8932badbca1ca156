"""The benchmark-configuration programs (pjrt_amd.configs) on the CPU oracle,
against independent numpy statements of the same models."""
import dataclasses

import numpy as np
import pytest

from oracle import vmref
from pjrt_amd import configs as CF
from pjrt_amd import scheduler as S
from pjrt_amd import vmprogram as V

TINY = CF.GptConfig(layers=2, d=64, heads=2, mlp=128, vocab=97, prompt=8, steps=4)


def _blob(prog, nlanes=8):
    return V.serialize(prog, S.schedule_program(prog, S.DeviceConfig(nlanes=nlanes)))


def test_mlp_c1_oracle_matches_numpy():
    args = CF.mlp_c1_inputs(batch=16, d_in=32, d_hidden=48, d_out=8)
    got = vmref.execute(_blob(CF.mlp_c1(16, 32, 48, 8)), args)[0]
    x, w1, b1, w2, b2 = (a.astype(np.float64) for a in args)
    want = np.maximum(x @ w1 + b1, 0) @ w2 + b2
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)


def test_gpt_c5_oracle_matches_numpy_decoder():
    """Prefill + greedy decode: same tokens, logits within bf16 rounding of the
    independent numpy decoder (configs.gpt_reference)."""
    args = CF.gpt_inputs(TINY, seed=5)
    first, toks, logits = vmref.execute(_blob(CF.gpt_c5(TINY, emit_logits=True)), args)
    ref_toks, ref_logits = CF.gpt_reference(TINY, args)
    assert np.abs(logits - ref_logits).max() <= 1e-2 * np.abs(ref_logits).max()
    np.testing.assert_array_equal(np.concatenate([first, toks]), ref_toks)


def test_gpt_c5_planted_position_mistake_is_caught():
    """A decoder that feeds the wrong position embedding changes the tokens: the
    comparison above can tell."""
    args = CF.gpt_inputs(TINY, seed=5)
    bad = list(args)
    names = ["ids"] + [n for n, _, _ in CF.gpt_param_shapes(TINY)]
    i = names.index("wpe")
    bad[i] = np.roll(args[i], 1, axis=0)
    ref_toks, ref_logits = CF.gpt_reference(TINY, args)
    bad_toks, bad_logits = CF.gpt_reference(TINY, bad)
    assert np.abs(bad_logits - ref_logits).max() > 1e-2 * np.abs(ref_logits).max()


def test_gpt_c5_program_shape_at_full_size():
    """The full config-5 program builds, schedules for 256 lanes and keeps every
    weight a zero-copy port (at most 256 ports)."""
    prog = CF.gpt_c5(dataclasses.replace(CF.C5, steps=2))
    assert len(prog.inputs) == 1 + len(CF.gpt_param_shapes(CF.C5)) <= 256
    blob = _blob(prog, nlanes=256)
    p = vmref.parse(blob)
    assert p.n_lanes == 256
