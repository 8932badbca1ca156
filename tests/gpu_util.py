"""Helpers of the GPU parity tests: one Runtime per session, programs scheduled for
the device and checked against the CPU oracle (oracle/vmref.py)."""
from __future__ import annotations

import sys

import numpy as np

from oracle import vmref
from pjrt_amd import scheduler as S
from pjrt_amd import vmprogram as V

_RT = None


def runtime():
    """The session's Runtime (device 0).  Raises when no MI355X / libvmrt.so."""
    global _RT
    if _RT is None:
        from pjrt_amd.runtime import Runtime
        _RT = Runtime()
        print(f"[gpu] {_RT.info['name']} {_RT.info['arch']} lanes={_RT.info['n_lanes']}"
              f"/{_RT.info['max_lanes']} lds={_RT.info['lds_bytes']}", file=sys.stderr, flush=True)
    return _RT


def blob_for(prog: V.VMProgram, nlanes=None, ew_ts=4096, mma_t=128, **kw) -> tuple:
    rt = runtime()
    cfg = S.DeviceConfig(nlanes=nlanes or rt.info["n_lanes"], ew_ts=ew_ts, mma_t=mma_t, **kw)
    return V.serialize(prog, S.schedule_program(prog, cfg)), cfg


def run_gpu(blob: bytes, args, ew_ts=4096, mma_t=128):
    rt = runtime()
    lp = rt.load(blob, ew_ts=ew_ts, mma_t=mma_t)
    try:
        return lp(*args)
    finally:
        lp.close()


def run_both(prog, args, nlanes=None, ew_ts=4096, mma_t=128, oracle="schedule", **kw):
    """(gpu outputs, oracle outputs) for a tensor program scheduled for the device."""
    if isinstance(prog, bytes):
        blob = prog
    else:
        blob, _ = blob_for(prog, nlanes=nlanes, ew_ts=ew_ts, mma_t=mma_t, **kw)
    print(f"[gpu] case: {len(blob)} bytes, lanes={vmref.parse(blob).n_lanes}, ew_ts={ew_ts}, mma_t={mma_t}",
          file=sys.stderr, flush=True)
    got = run_gpu(blob, args, ew_ts=ew_ts, mma_t=mma_t)
    if oracle == "schedule":
        want = vmref.execute_schedule(blob, args, ew_ts=ew_ts, mma_t=mma_t, check_order=False)
    elif oracle == "tensor":
        want = vmref.execute(blob, args, ew_ts=ew_ts, mma_t=mma_t)
    else:
        want = None
    return got, want


def as_f32(x, dt):
    return vmref.bf16_to_f32(x) if dt == V.DT_BF16 else np.asarray(x, np.float32)


def assert_rel(got, want, rtol, atol=0.0, what=""):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    bad = ~(np.abs(got - want) <= atol + rtol * np.abs(want))
    both_nan = np.isnan(got) & np.isnan(want)
    bad &= ~both_nan & ~(got == want)        # equal infinities count as equal
    if bad.any():
        idx = np.argwhere(bad)[:5]
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} outside rtol={rtol} atol={atol}; "
                             f"first {[(tuple(i), float(got[tuple(i)]), float(want[tuple(i)])) for i in idx]}")


def close_runtime():
    """Close the session's Runtime (its programs first), so no HIP call is left
    for interpreter shutdown."""
    global _RT
    if _RT is not None:
        _RT.close()
        _RT = None


def assert_product_elementwise(got, want, scale, rtol, what=""):
    """Elementwise check of a matmul or attention output: |got - want| <= rtol *
    scale, with ``scale`` the same product taken over absolute values (|A| |B|
    for a GEMM, P |V| for attention).  A dot product's rounding error is bounded
    by a multiple of that sum, so this is the north star's per-element relative
    bar without a tolerance that blows up where the result cancels to ~0."""
    got = np.asarray(got, np.float64).reshape(np.shape(want))
    bad = ~(np.abs(got - want) <= rtol * scale)
    if bad.any():
        idx = np.argwhere(bad)[:5]
        raise AssertionError(f"{what}: {int(bad.sum())} elements outside rtol {rtol} of their |.| product scale; "
                             f"first {[tuple(i) for i in idx]}: got {[got[tuple(i)] for i in idx]} "
                             f"want {[want[tuple(i)] for i in idx]} scale {[scale[tuple(i)] for i in idx]}")


def attention_abs_scale(q, kt, v, scale, causal):
    """P |V| in float64 for attention(q [H,T,hd], kt [H,hd,C], v [H,C,hd])."""
    H, T, hd = q.shape
    C = kt.shape[2]
    s = np.einsum("htd,hdc->htc", q.astype(np.float64), kt.astype(np.float64)) * scale
    if causal:
        s = np.where(np.arange(C)[None, :] > np.arange(T)[:, None] + (C - T), -np.inf, s)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    return np.einsum("htc,hcd->htd", p, np.abs(v.astype(np.float64)))


def check_decoder(got, want, rel, pinned, what="decoder"):
    """Greedy decoding, step by step: the logits of every step agree within
    ``rel`` of the oracle's largest logit, and the tokens are equal until a step
    where the oracle's top two logits lie within twice that tolerance (a
    near-tie: either token is a correct greedy choice, and the two runs diverge
    from there).  Inputs and kernels are deterministic, so the count of
    token-exact steps is a fixed property of the case: it must reach ``pinned``,
    the count measured on the MI355X (all steps where nothing diverges).
    Returns (verified steps, steps, step of the near-tie or None)."""
    (g_first, g_toks, g_logits), (w_first, w_toks, w_logits) = got, want
    tg, tw = np.concatenate([g_first, g_toks]), np.concatenate([w_first, w_toks])
    tol = rel * float(np.abs(w_logits).max())
    verified, tie = 0, None
    for s in range(len(tw)):
        err = float(np.abs(g_logits[s] - w_logits[s]).max())
        assert err <= tol, f"{what}: step {s}: logits differ by {err} > {tol}"
        top = np.sort(w_logits[s])[-2:]
        if tg[s] != tw[s]:
            gap = float(top[1] - top[0])
            assert gap <= 2 * tol, f"{what}: step {s}: token {tg[s]} != {tw[s]} (top-two gap {gap} > {2 * tol})"
            tie = s
            print(f"[gpu] {what}: step {s} is a near-tie (top-two gap {gap:.3g} <= {2 * tol:.3g}); the runs "
                  f"diverge there", file=sys.stderr, flush=True)
            break
        verified += 1
    print(f"[gpu] {what}: {verified} of {len(tw)} steps verified token-exact", file=sys.stderr, flush=True)
    assert verified >= min(pinned, len(tw)), f"{what}: {verified} token-exact steps, {pinned} measured"
    return verified, len(tw), tie
