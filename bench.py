"""Benchmark of the MI355X megakernel VM on BASELINE.json's configurations.

Headline (one JSON line on stdout): config 2, fused layernorm(eps 1e-5, affine) +
tanh-GELU + f32->bf16 on x[8192, 4096] f32 (the HBM-bound
configuration the metric's "elementwise GB/s as % of roofline" is quoted on).  A
step is one execution of the program on device-resident inputs; value = algorithmic
bytes per step / wall time per step, with three input/output sets in rotation so
that every step reads from HBM (576 MiB, more than the 256 MB memory-side cache
holds); the rate of one cache-resident set is reported beside it ("warm_cache").

Also reported under "extra" (same JSON line): config 1 (f32 MLP), config 3
dot_general 4096^3 (bf16 and f32 operands, f32 accumulate) and config 4 causal
flash attention (B4 H16 S2048 d128, bf16) as TFLOP/s against their MFMA roofline,
and config 5 (GPT decoder, greedy decode) as tokens/s against the per-token HBM
bytes.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workloads c1,c2,c3,c3_bf16,c3_f32,c4,attn_variants,c5,copy]
                    [--no-cpu] [--skip-c2] [--c2-cache both|cold|warm] [--no-vendor]

"copy" adds a plain device-to-device copy of 128 MiB, the calibration kernel for
the HBM byte counters.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "pjrt-ocl_amd", "python"), ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402

METRIC = "decode tokens/s; GEMM/attn TFLOP/s and elementwise GB/s as % of MI355X roofline"
HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = {"bf16": 2500.0, "f16": 2500.0, "f32": 157.3}

C2_ROWS, C2_D = 8192, 4096
# algorithmic bytes of config 2: read x (f32), write y (bf16), read gamma + beta
C2_BYTES = C2_ROWS * C2_D * 4 + C2_ROWS * C2_D * 2 + 2 * C2_D * 4


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def build_c2():
    from pjrt_amd import graph as G
    g = G.Graph()
    x, ga, be = g.input((C2_ROWS, C2_D)), g.input((C2_D,)), g.input((C2_D,))
    g.output(g.layernorm(x, ga, be, 1e-5, gelu=True, out_dtype="bf16"))
    return g.build()


def c2_inputs():
    rng = np.random.default_rng(1002)
    x = rng.standard_normal((C2_ROWS, C2_D), dtype=np.float32)
    gamma = rng.uniform(0.5, 1.5, C2_D).astype(np.float32)
    beta = (rng.standard_normal(C2_D) * 0.1).astype(np.float32)
    return x, gamma, beta


def time_program(rt, lp, dev_in, dev_out, steps, warmup, min_warm_s=0.3, sets=None):
    """Warm up (at least `warmup` executions and `min_warm_s` seconds, so the GPU
    clocks have ramped up), then time exactly `steps` back-to-back executions:
    wall clock around the whole region and HIP events on the launch stream.
    `sets`, a list of (inputs, outputs), rotates the buffers step by step (a
    working set larger than the 256 MB memory-side cache: a cold-cache rate)."""
    sets = sets or [(dev_in, dev_out)]
    t_warm = time.perf_counter()
    n = 0
    while n < warmup or time.perf_counter() - t_warm < min_warm_s:
        lp.enqueue(*sets[n % len(sets)])
        n += 1
        if n % 8 == 0:
            rt.synchronize()
    rt.synchronize()
    lp.status()
    e0, e1 = rt.event(), rt.event()
    rt.synchronize()
    t0 = time.perf_counter()
    e0.record()
    for i in range(steps):
        lp.enqueue(*sets[i % len(sets)])
    e1.record()
    rt.synchronize()
    wall = time.perf_counter() - t0
    lp.status()
    return wall * 1e3 / steps, e0.elapsed_ms(e1) / steps


def load_traffic(name):
    path = os.path.join(ROOT, "profiles", f"traffic_{name}.json")
    try:
        with open(path) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


def cpu_info():
    """Host threads the CPU baseline uses and the host's CPU model.  The GPU box
    gives one GPU's job a share of 16 host cores (its OMP_NUM_THREADS), whatever
    nproc reports, so the baseline uses min(16, available cores)."""
    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    share = int(os.environ.get("OMP_NUM_THREADS", "16") or 16)
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return max(1, min(avail, share, 16)), os.cpu_count() or 1, model


def time_cpu(call, budget_s=10.0, min_round_s=0.1, min_rounds=5):
    """Median seconds per call: one warm-up call, then rounds of adaptive length
    (at least `min_round_s` each), at least `min_rounds` of them and as many more
    as fit `budget_s` (the reference's tools/bench_cpu.py:35-50 methodology)."""
    t0 = time.perf_counter()
    call()
    per = max(time.perf_counter() - t0, 1e-6)
    reps = max(1, int(math.ceil(min_round_s / per)))
    rounds, t_start = [], time.perf_counter()
    while len(rounds) < min_rounds or (time.perf_counter() - t_start < budget_s and len(rounds) < 50):
        t = time.perf_counter()
        for _ in range(reps):
            call()
        rounds.append((time.perf_counter() - t) / reps)
    return float(np.median(rounds)), len(rounds), reps


def _refcpu():
    lib = ctypes.CDLL(os.path.join(ROOT, "oracle", "librefcpu.so"))
    lib.refcpu_ln_gelu_bf16.restype = ctypes.c_int
    lib.refcpu_ln_gelu_bf16.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int64, ctypes.c_int64, ctypes.c_float,
                                                               ctypes.c_void_p, ctypes.c_int]
    lib.refcpu_mlp_f32.restype = ctypes.c_int
    lib.refcpu_mlp_f32.argtypes = [ctypes.c_void_p] * 8 + [ctypes.c_int64] * 4 + [ctypes.c_int]
    lib.refcpu_sgemm_packed.restype = ctypes.c_int
    lib.refcpu_sgemm_packed.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int64] * 3 + [ctypes.c_void_p, ctypes.c_int]
    lib.refcpu_attention_f32.restype = ctypes.c_int
    lib.refcpu_attention_f32.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int64] * 3 + [
        ctypes.c_float, ctypes.c_int, ctypes.c_void_p, ctypes.c_int]
    lib.refcpu_gpt_f32.restype = ctypes.c_int
    lib.refcpu_gpt_f32.argtypes = [ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_int64] * 7 + [
        ctypes.c_float, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
    return lib


def cpu_baseline_c2(x, gamma, beta, budget_s=10.0):
    """The reference's CPU engine path for config 2 (decomposed phases), restated in
    C (oracle/refcpu.c), on the host cores, over the full workload."""
    lib = _refcpu()
    cores, nproc, model = cpu_info()
    out = np.empty((C2_ROWS, C2_D), np.uint16)
    scratch = np.empty(2 * C2_ROWS * C2_D + 2 * C2_ROWS, np.float32)

    def call():
        lib.refcpu_ln_gelu_bf16(x.ctypes.data, gamma.ctypes.data, beta.ctypes.data, out.ctypes.data, C2_ROWS, C2_D,
                                1e-5, scratch.ctypes.data, cores)

    dt, rounds, reps = time_cpu(call, budget_s)
    return {"value": round(C2_BYTES / dt / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "nproc": nproc, "cpu_model": model,
            "sample": f"full config-2 workload [8192,4096]; median of {rounds} rounds of {reps} call(s) after a "
                      f"warm-up call, {dt * 1e3:.1f} ms/call; C restatement of the reference's decomposed "
                      f"CPU-engine phases (oracle/refcpu.c)"}, out


def cpu_baseline_c1(args, budget_s=3.0):
    """Config 1 on the reference's CPU path (its configs[0] names the PoCL CPU
    path): two SGEMM phases plus bias / relu phases (oracle/refcpu.c)."""
    lib = _refcpu()
    cores, nproc, model = cpu_info()
    x, w1, b1, w2, b2 = args
    M, D = x.shape
    H, O = w1.shape[1], w2.shape[1]
    y = np.empty((M, O), np.float32)
    h = np.empty((M, H), np.float32)
    bp = np.empty(max(D * H, H * O), np.float32)

    def call():
        if lib.refcpu_mlp_f32(x.ctypes.data, w1.ctypes.data, b1.ctypes.data, w2.ctypes.data, b2.ctypes.data,
                              y.ctypes.data, h.ctypes.data, bp.ctypes.data, M, D, H, O, cores):
            raise SystemExit("bench: CPU baseline MLP rejected its shapes")

    dt, rounds, reps = time_cpu(call, budget_s)
    flops = 2.0 * M * D * H + 2.0 * M * H * O
    return {"value": round(flops / dt / 1e9, 3), "unit": "GFLOP/s", "cores": cores, "kind": "port",
            "nproc": nproc, "cpu_model": model, "ms_per_forward": round(dt * 1e3, 4),
            "sample": f"full config-1 forward; median of {rounds} rounds of {reps} call(s); C restatement of the "
                      f"reference's CPU-engine path: packed SGEMM (mm2_pack + mm2p_epi, bias in the store) and a "
                      f"relu phase (oracle/refcpu.c)"}, y


def cpu_baseline_gemm_f32(a, b, budget_s=6.0):
    """Config 3 in f32 on the reference's CPU path: the 4096^3 matmul on its
    packed SGEMM (mm2_pack + mm2p, KC = 1024 sweeps; oracle/refcpu.c), full size.
    Returns (baseline record, C)."""
    lib = _refcpu()
    cores, nproc, model = cpu_info()
    M, K = a.shape
    N = b.shape[1]
    c = np.empty((M, N), np.float32)
    bp = np.empty(K * N, np.float32)

    def call():
        if lib.refcpu_sgemm_packed(a.ctypes.data, b.ctypes.data, c.ctypes.data, M, N, K, bp.ctypes.data, cores):
            raise SystemExit("bench: CPU baseline SGEMM rejected its shapes")

    dt, rounds, reps = time_cpu(call, budget_s, min_rounds=3)
    return {"value": round(2.0 * M * N * K / dt / 1e12, 4), "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "nproc": nproc, "cpu_model": model, "ms_per_call": round(dt * 1e3, 2),
            "sample": f"full {M}x{K}x{N} f32 matmul; median of {rounds} rounds of {reps} call(s) after a warm-up "
                      f"call; C restatement of the reference's CPU-engine packed SGEMM (oracle/refcpu.c)"}, c


def cpu_baseline_attention(q, k, v, D, heads=8, budget_s=6.0):
    """Config 4 is unsupported on the reference (bf16 causal flash attention).
    Times its f32-widened computation in the reference's decomposed style
    (per head: scores on the packed SGEMM, scale + mask, row softmax passes, p v
    on the packed SGEMM; oracle/refcpu.c) on the first `heads` heads, and reports
    the causal algorithmic FLOP rate of that sample."""
    from pjrt_amd import vmprogram as V
    lib = _refcpu()
    cores, nproc, model = cpu_info()
    G, S, _ = q.shape
    qs, ks, vs = (np.ascontiguousarray(V.bf16_to_f32(t[:heads]), np.float32) for t in (q, k, v))
    o = np.empty_like(qs)
    scratch = np.empty(S * S + S * D, np.float32)

    def call():
        if lib.refcpu_attention_f32(qs.ctypes.data, ks.ctypes.data, vs.ctypes.data, o.ctypes.data, heads, S, D,
                                    1.0 / math.sqrt(D), 1, scratch.ctypes.data, cores):
            raise SystemExit("bench: CPU baseline attention rejected its shapes")

    dt, rounds, reps = time_cpu(call, budget_s, min_rounds=3)
    flops = 4.0 * heads * D * S * (S + 1) / 2
    return {"value": round(flops / dt / 1e12, 4), "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "nproc": nproc, "cpu_model": model, "reference_support": "unsupported (f32-widened equivalent timed)",
            "ms_per_head": round(dt * 1e3 / heads, 2),
            "sample": f"{heads} of {G} heads [S {S}, d {D}], causal, f32 (the bf16 inputs widened); median of "
                      f"{rounds} rounds of {reps} call(s); the full S x S scores are computed, as the decomposed "
                      f"chain does; rate = causal algorithmic FLOP of the sample / time (oracle/refcpu.c)"}, o


def cpu_baseline_c5(c, args, steps=16):
    """Config 5 is unsupported on the reference (the argmax is a variadic reduce;
    bf16 matmuls).  Times its f32-widened computation (oracle/refcpu.c
    refcpu_gpt_f32: prefill on the packed SGEMM, decode steps as row GEMVs over
    f32 weights) for the prompt and `steps` greedy tokens; reports decode
    tokens/s and the prefill time.  Returns (record, tokens)."""
    from pjrt_amd import vmprogram as V
    lib = _refcpu()
    cores, nproc, model = cpu_info()
    ids = np.ascontiguousarray(args[0], np.int32)
    params = [np.ascontiguousarray(V.bf16_to_f32(a) if a.dtype == np.uint16 else a, np.float32) for a in args[1:]]
    ptrs = (ctypes.c_void_p * len(params))(*[p.ctypes.data for p in params])
    toks = np.empty(steps + 1, np.int32)
    best = None
    for _ in range(2):            # the second run is timed warm (weights paged in)
        times = np.zeros(2, np.float64)
        if lib.refcpu_gpt_f32(ids.ctypes.data, ptrs, c.layers, c.d, c.heads, c.mlp, c.vocab, c.prompt, steps, c.eps,
                              toks.ctypes.data, None, times.ctypes.data, cores):
            raise SystemExit("bench: CPU baseline decoder failed")
        best = times if best is None or times[1] < best[1] else best
    return {"value": round(steps / best[1], 2), "unit": "tokens/s", "cores": cores, "kind": "port",
            "nproc": nproc, "cpu_model": model, "reference_support": "unsupported (f32-widened equivalent timed)",
            "prefill_ms": round(best[0] * 1e3, 1), "ms_per_token": round(best[1] * 1e3 / steps, 2),
            "sample": f"prompt {c.prompt} then {steps} of the {c.steps} greedy steps, f32 weights and activations; "
                      f"better of 2 runs (oracle/refcpu.c)"}, toks


def bench_c2(rt, steps, warmup, with_cpu, cache="both"):
    """Config 2.  The headline is the cold-cache rate: three input/output sets
    (3 x 192 MiB) in rotation, more than the 256 MB memory-side cache holds, so
    every step reads its inputs from HBM.  Beside it, the warm rate of one set
    (192 MiB, which the memory-side cache keeps between steps: a cache-resident
    figure, not an HBM fraction).  `cache` = "cold" or "warm" measures only one
    (profiling runs, where every dispatch must be of the reported kind)."""
    prog = build_c2()
    lp = rt.compile(prog)
    x, gamma, beta = c2_inputs()
    dev_in = [rt.to_device(x), rt.to_device(gamma), rt.to_device(beta)]
    dev_out = lp.alloc_outputs()
    cold_step = cold_kernel = warm_step = warm_kernel = None
    sets = [(dev_in, dev_out)]
    if cache in ("both", "cold"):
        extra_sets = [([rt.to_device(x), dev_in[1], dev_in[2]], lp.alloc_outputs()) for _ in range(2)]
        sets += extra_sets
        cold_step, cold_kernel = time_program(rt, lp, None, None, steps, warmup, sets=sets)
        for ins, outs in extra_sets:
            for b in [ins[0]] + outs:
                b.free()
    if cache in ("both", "warm"):
        warm_step, warm_kernel = time_program(rt, lp, dev_in, dev_out, steps, warmup)
    got = dev_out[0].to_host(np.uint16, (C2_ROWS, C2_D))
    # spot check against float64 math on a slice of rows
    rows = slice(0, 256)
    x64 = x[rows].astype(np.float64)
    mu = x64.mean(1, keepdims=True)
    z = (x64 - mu) / np.sqrt(((x64 - mu) ** 2).mean(1, keepdims=True) + 1e-5) * gamma + beta
    want = 0.5 * z * (1 + np.tanh(0.7978845608 * (z + 0.044715 * z ** 3)))
    gotf = (got[rows].astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    err = float(np.max(np.abs(gotf - want) / (np.abs(want) + 1e-6)))
    if err > 2.0 ** -7 + 1e-6:       # one bf16 ulp of the float64 result
        raise SystemExit(f"bench: config-2 result check failed (max rel err {err:.3g})")
    cpu = None
    if with_cpu:
        cpu, cout = cpu_baseline_c2(x, gamma, beta)
        diff = np.abs((cout.astype(np.uint32) << 16).view(np.float32).astype(np.float64) -
                      (got.astype(np.uint32) << 16).view(np.float32).astype(np.float64))
        cpu["max_abs_diff_vs_gpu"] = float(diff.max())
    traffic = load_traffic("c2")
    head_step, head_kernel = (cold_step, cold_kernel) if cold_step is not None else (warm_step, warm_kernel)
    achieved = C2_BYTES / (head_kernel * 1e-3) / 1e9
    res = {
        "value": C2_BYTES / (head_step * 1e-3) / 1e9, "unit": "GB/s", "ms_per_step": head_step,
        "kernel_ms": head_kernel,
        "cache": (f"cold: {len(sets)} input/output sets in rotation, {len(sets) * C2_ROWS * C2_D * 6} B, more "
                  f"than the 256 MB memory-side cache" if cold_step is not None else
                  "warm: one set of 201 MB, resident in the 256 MB memory-side cache (not an HBM rate)"),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic.get("bytes_per_launch") if traffic else None},
        "warm": None if warm_step is None or cold_step is None else {
            "working_set_bytes": C2_ROWS * C2_D * 6, "value": round(C2_BYTES / (warm_step * 1e-3) / 1e9, 2),
            "ms_per_step": round(warm_step, 5), "kernel_ms": round(warm_kernel, 5),
            "achieved": round(C2_BYTES / (warm_kernel * 1e-3) / 1e9, 2),
            "frac": round(C2_BYTES / (warm_kernel * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "note": "one 192 MiB set, kept in the 256 MB memory-side cache between steps: a cache-resident rate"},
        "cpu_baseline": cpu, "max_rel_err_first_256_rows": err,
    }
    for b in dev_in + dev_out:
        b.free()
    lp.close()
    return res


def bench_gemm(rt, dt, steps, warmup, M=4096, N=4096, K=4096, with_cpu=False):
    from pjrt_amd import graph as G
    from pjrt_amd import vmprogram as V
    rng = np.random.default_rng(1003)
    a = (rng.standard_normal((M, K), dtype=np.float32) * 0.125)
    b = (rng.standard_normal((K, N), dtype=np.float32) * 0.125)
    g = G.Graph()
    x, y = g.input((M, K), dt), g.input((K, N), dt)
    g.output(g.dot(x, y))
    lp = rt.compile(g.build())
    if dt == "bf16":
        a_dev, b_dev = V.f32_to_bf16(a), V.f32_to_bf16(b)
        a, b = V.bf16_to_f32(a_dev), V.bf16_to_f32(b_dev)
    else:
        a_dev, b_dev = a, b
    dev_in = [rt.to_device(a_dev), rt.to_device(b_dev)]
    dev_out = lp.alloc_outputs()
    ms_step, ms_kernel = time_program(rt, lp, dev_in, dev_out, steps, warmup)
    c = dev_out[0].to_host(np.float32, (M, N))
    idx = np.random.default_rng(0).integers(0, M, 64)
    want = a[idx].astype(np.float64) @ b.astype(np.float64)
    err = float(np.abs(c[idx] - want).max() / np.abs(want).max())
    flops = 2.0 * M * N * K
    tf = flops / (ms_kernel * 1e-3) / 1e12
    for buf in dev_in + dev_out:
        buf.free()
    lp.close()
    res = {"workload": f"C3 dot_general {M}x{K}x{N} {dt} -> f32", "tflops": round(flops / (ms_step * 1e-3) / 1e12, 2),
           "ms_per_step": ms_step, "kernel_ms": ms_kernel,
           "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": MFMA_PEAK_TFLOPS[dt], "unit": "TFLOP/s",
                        "frac": round(tf / MFMA_PEAK_TFLOPS[dt], 4)},
           "max_rel_err_64_rows": err, "vendor_library_tflops": library_gemm_tflops(dt, M, N, K)}
    if with_cpu and dt == "f32":
        log("C3 f32 CPU baseline")
        cpu, ccpu = cpu_baseline_gemm_f32(a, b)
        cpu["max_rel_diff_vs_gpu"] = float(np.abs(ccpu - c).max() / np.abs(c).max())
        res["cpu_baseline"] = cpu
    return res


def library_gemm_tflops(dt, M, N, K, steps=20):
    """torch.matmul on the same shape and operand dtype (the vendor BLAS:
    hipBLASLt / rocBLAS), timed with events on torch's stream in a child
    process of its own: what AMD's own library reaches on this box, for
    comparison only.  Its output is in the operand dtype (bf16 writes half the
    bytes of this build's f32 output).  Skipped with --no-vendor (profiling
    runs: torch's own kernels under a tracer are not ours to measure)."""
    if os.environ.get("PJRT_AMD_BENCH_NO_VENDOR") == "1":
        return None
    code = f"""
import torch
tdt = torch.bfloat16 if {dt!r} == "bf16" else torch.float32
torch.backends.cuda.matmul.allow_tf32 = False
a = torch.randn({M}, {K}, device="cuda", dtype=tdt)
b = torch.randn({K}, {N}, device="cuda", dtype=tdt)
for _ in range(5):
    c = a @ b
torch.cuda.synchronize()
e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
e0.record()
for _ in range({steps}):
    c = a @ b
e1.record()
torch.cuda.synchronize()
print(2.0 * {M} * {N} * {K} / (e0.elapsed_time(e1) / {steps} * 1e-3) / 1e12)
"""
    import subprocess
    try:
        r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
        if r.returncode != 0:
            log(f"vendor GEMM not measured: exit {r.returncode}")
            return None
        return round(float(r.stdout.strip().splitlines()[-1]), 1)
    except (subprocess.SubprocessError, ValueError, IndexError) as e:
        log(f"vendor GEMM not measured: {e}")
        return None


def bench_attention(rt, steps, warmup, B=4, H=16, S=2048, D=128, with_cpu=False, dt="bf16"):
    """Causal flash attention [B*H, S, D] in `dt` (config 4: bf16, d 128; the
    f32 and d-256 entries are the same shape on the f32 and wide-head kernels,
    informational, not BASELINE configs)."""
    from pjrt_amd import graph as G
    from pjrt_amd import vmprogram as V
    rng = np.random.default_rng(1004)
    shape = (B * H, S, D)
    if dt == "f32":
        q, k, v = (rng.standard_normal(shape, dtype=np.float32) for _ in range(3))
        as_f32 = lambda t: t
    else:
        q, k, v = (V.f32_to_bf16(rng.standard_normal(shape, dtype=np.float32)) for _ in range(3))
        as_f32 = V.bf16_to_f32
    g = G.Graph()
    Q, K, Vv = g.input(shape, dt), g.input(shape, dt), g.input(shape, dt)
    g.output(g.flash_attention(Q, K, Vv, 1.0 / math.sqrt(D), True, out_dtype=dt))
    lp = rt.compile(g.build())
    dev_in = [rt.to_device(q), rt.to_device(k), rt.to_device(v)]
    dev_out = lp.alloc_outputs()
    ms_step, ms_kernel = time_program(rt, lp, dev_in, dev_out, steps, warmup)
    o = dev_out[0].to_host(np.float32, shape) if dt == "f32" else V.bf16_to_f32(dev_out[0].to_host(np.uint16, shape))
    # check two heads against float64 math: softmax(scale * q k^T, causal) v
    errs = []
    for h in (0, B * H - 1):
        qh, kh, vh = (as_f32(t[h]).astype(np.float64) for t in (q, k, v))
        s = (qh @ kh.T) / math.sqrt(D)
        s[np.triu_indices(S, 1)] = -np.inf
        p = np.exp(s - s.max(1, keepdims=True))
        want = (p / p.sum(1, keepdims=True)) @ vh
        errs.append(float(np.abs(o[h] - want).max() / np.abs(want).max()))
    flops = 4.0 * B * H * D * S * (S + 1) / 2
    tf = flops / (ms_kernel * 1e-3) / 1e12
    for buf in dev_in + dev_out:
        buf.free()
    lp.close()
    res = {"workload": f"{'C4 ' if dt == 'bf16' and D == 128 else ''}causal flash attention B{B} H{H} S{S} d{D} {dt}",
           "tflops": round(flops / (ms_step * 1e-3) / 1e12, 2), "ms_per_step": ms_step, "kernel_ms": ms_kernel,
           "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": MFMA_PEAK_TFLOPS[dt],
                        "unit": "TFLOP/s", "frac": round(tf / MFMA_PEAK_TFLOPS[dt], 4)},
           "max_rel_err_2_heads": max(errs)}
    if with_cpu:
        log("C4 CPU baseline")
        cpu, ocpu = cpu_baseline_attention(q, k, v, D)
        n = ocpu.shape[0]
        cpu["max_rel_diff_vs_gpu"] = float(np.abs(ocpu - o[:n]).max() / np.abs(o[:n]).max())
        res["cpu_baseline"] = cpu
    return res


def bench_lowered(rt, steps):
    """The drop-in path: configs 1-5 as the StableHLO text a JAX program lowers
    to (pjrt_amd.stablehlo_configs), through the lowering and its fusion passes
    (what the plugin's Compile runs), timed beside the hand-built program of the
    same config on the same inputs (config 5: bench_c5_lowered).  Reports both kernel times, their ratio,
    the lowered program's tile ops and the largest difference between the two
    outputs."""
    from pjrt_amd import configs as CF
    from pjrt_amd import graph as G
    from pjrt_amd import lowering as L
    from pjrt_amd import stablehlo_configs as H
    from pjrt_amd import vmprogram as V
    rng = np.random.default_rng(1005)

    def bf16(shape):
        return V.f32_to_bf16((rng.standard_normal(shape) * 0.125).astype(np.float32))

    def hand_c3():
        g = G.Graph()
        x, y = g.input((4096, 4096), "bf16"), g.input((4096, 4096), "bf16")
        g.output(g.dot(x, y))
        return g.build()

    def hand_c4():
        g = G.Graph()
        shape = (64, 2048, 128)
        q, k, v = (g.input(shape, "bf16") for _ in range(3))
        g.output(g.flash_attention(q, k, v, 1.0 / math.sqrt(128), True, out_dtype="bf16"))
        return g.build()

    x2, g2, b2 = c2_inputs()
    cases = {
        "c1": (H.mlp(), CF.mlp_c1(), list(CF.mlp_c1_inputs())),
        "c2": (H.ln_gelu(C2_ROWS, C2_D), build_c2(), [x2, g2, b2]),
        "c3_bf16": (H.matmul(4096, 4096, 4096, "bf16", "f32"), hand_c3(), [bf16((4096, 4096)), bf16((4096, 4096))]),
        "c4": (H.attention(4, 16, 2048, 128, "bf16", True), hand_c4(), [bf16((4, 16, 2048, 128)) for _ in range(3)]),
    }
    names = {v: k for k, v in vars(V).items() if k.startswith("TOP_") and k != "TOP_MAX"}
    out = {"c5": bench_c5_lowered(rt), "reference_decode_step": bench_reference_decode(rt, steps)}
    for name, (text, hand, args) in cases.items():
        t0 = time.perf_counter()
        low = L.lower_text(text)
        lower_s = time.perf_counter() - t0
        res = {}
        for kind, prog, reuse in (("lowered", low, False), ("hand_built", hand, True)):
            lp = rt.compile(prog, arena_reuse=reuse)
            dev_in = [rt.to_device(a) for a in args]
            dev_out = lp.alloc_outputs()
            _, ms = time_program(rt, lp, dev_in, dev_out, steps, 3, min_warm_s=0.1)
            spec = lp.outputs[0]
            res[kind] = (ms, dev_out[0].to_host(spec.np_dtype, spec.shape))
            for b in dev_in + dev_out:
                b.free()
            lp.close()
        (ml, ol), (mh, oh) = res["lowered"], res["hand_built"]
        f = (lambda a: V.bf16_to_f32(a).astype(np.float64)) if ol.dtype == np.uint16 else (lambda a: a.astype(np.float64))
        diff = float(np.abs(f(ol).reshape(-1) - f(oh).reshape(-1)).max())
        from pjrt_amd import scheduler as S
        ops = sorted({names.get(t.tile_op, str(t.tile_op)) for t in
                      S.schedule_program(low, rt.scheduler_config()).tasks})
        out[name] = {"lowered_kernel_ms": round(ml, 5), "hand_built_kernel_ms": round(mh, 5),
                     "lowered_over_hand_built": round(ml / mh, 3), "lower_s": round(lower_s, 2),
                     "lowered_tile_ops": ops, "max_abs_diff_vs_hand_built": diff}
        log(f"lowered {name}: {ml * 1e3:.1f} us vs hand-built {mh * 1e3:.1f} us ({', '.join(ops)})")
    return out


def bench_c5_lowered(rt, reps=3):
    """Config 5 as the JAX program (pjrt_amd.stablehlo_configs.gpt_decode:
    prefill, then a fori_loop decode with dynamic_update_slice KV caches, masked
    attention and argmax) through the lowering, timed as bench_c5 times the
    hand-built decoder: the full program against the same program cut to 8 loop
    trips.  Also reports how many of the 129 tokens equal the hand-built
    program's on the same inputs."""
    from pjrt_amd import configs as CF
    from pjrt_amd import lowering as L
    from pjrt_amd import scheduler as S
    from pjrt_amd import stablehlo_configs as H
    c = CF.C5
    args = CF.gpt_inputs(c)
    dev_in = [rt.to_device(a) for a in args]
    times, toks, lower_s, lanes = {}, {}, 0.0, None
    saved = os.environ.get("PJRT_OCL_WHILE")
    os.environ["PJRT_OCL_WHILE"] = "for"           # 8 trips would otherwise be unrolled
    try:
        for trips in (c.steps, 8):
            t0 = time.perf_counter()
            prog = L.lower_text(H.gpt_decode(c, trips=trips))
            lower_s = max(lower_s, time.perf_counter() - t0)
            if lanes is None:          # the full program's lane count, for both (see bench_c5)
                lanes = S.lane_fit(prog, rt.scheduler_config())
            lp = rt.compile(prog, arena_reuse=False, nlanes=lanes, fit_lanes=False)
            dev_out = lp.alloc_outputs()
            _, times[trips] = time_program(rt, lp, dev_in, dev_out, reps, 1)
            if trips == c.steps:
                toks["lowered"] = np.concatenate([dev_out[0].to_host(np.int32, (1,)),
                                                  dev_out[1].to_host(np.int32, (c.steps,))])
            for b in dev_out:
                b.free()
            lp.close()
    finally:
        if saved is None:
            os.environ.pop("PJRT_OCL_WHILE", None)
        else:
            os.environ["PJRT_OCL_WHILE"] = saved
    lp = rt.compile(CF.gpt_c5(c))
    dev_out = lp.alloc_outputs()
    lp.execute(dev_in, dev_out)
    toks["hand_built"] = np.concatenate([dev_out[0].to_host(np.int32, (1,)), dev_out[1].to_host(np.int32, (c.steps,))])
    for b in dev_out + dev_in:
        b.free()
    lp.close()
    per_tok = (times[c.steps] - times[8]) / (c.steps - 8)
    same = toks["lowered"] == toks["hand_built"]
    log(f"lowered c5: {1e3 / per_tok:.1f} tokens/s, {int(same.sum())} of {same.size} tokens as hand-built")
    return {"decode_tokens_per_s": round(1e3 / per_tok, 1), "ms_per_token": round(per_tok, 4),
            "program_ms": round(times[c.steps], 3), "prefill_plus_8_steps_ms": round(times[8], 3),
            "lower_s": round(lower_s, 2), "tokens_equal_to_hand_built": int(same.sum()),
            "first_token_difference": int(np.argmin(same)) if not same.all() else None}


REF_DECODE_US = {"base": (5702.0, 3835.0)}     # RTX PRO 6000, docs/decisions.md:2249-2253, 2369-2372


def bench_reference_decode(rt, steps):
    """The reference's own decode benchmark program (tools/bench_decode.py: one
    f32 token through the layers, keys and values appended by concatenate), as
    the StableHLO its jit lowers to, through our lowering: microseconds per
    token (one program execution each) and the bytes a token must read (f32
    weights plus the two caches, tools/bench_decode.py:83-89) per second.  The
    reference published 5702 us/token for "base" on an RTX PRO 6000, 3835 with
    its epilogue fusion."""
    from pjrt_amd import lowering as L
    from pjrt_amd import stablehlo_configs as H
    out = {}
    for name, cfg in H.DECODE_STEP_CONFIGS.items():
        prog = L.lower_text(H.decode_step(cfg))
        lp = rt.compile(prog, arena_reuse=False)
        dev_in = [rt.to_device(a) for a in H.decode_step_inputs(cfg)]
        dev_out = lp.alloc_outputs()
        wall_ms, ms = time_program(rt, lp, dev_in, dev_out, max(20, steps), 5)
        for b in dev_in + dev_out:
            b.free()
        lp.close()
        nbytes = H.decode_step_bytes(cfg)
        res = {"config": dict(zip(("d_model", "heads", "d_ff", "layers", "context"), cfg)),
               "us_per_token": round(ms * 1e3, 2), "wall_us_per_token": round(wall_ms * 1e3, 2),
               "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1), "bytes_per_token": nbytes}
        if name in REF_DECODE_US:
            res["reference_us_per_token_rtx_pro_6000"] = REF_DECODE_US[name][1]
        out[name] = res
        log(f"reference decode step {name}: {ms * 1e3:.1f} us/token")
    return out


def bench_c1(rt, steps, with_cpu=False):
    """Config 1: the f32 two-layer MLP forward, on the GPU,
    beside the reference's CPU path for it (the path configs[0] names)."""
    from pjrt_amd import configs as CF
    args = CF.mlp_c1_inputs()
    lp = rt.compile(CF.mlp_c1())
    dev_in = [rt.to_device(a) for a in args]
    dev_out = lp.alloc_outputs()
    ms_step, ms_kernel = time_program(rt, lp, dev_in, dev_out, steps, 5)
    y = dev_out[0].to_host(np.float32, (256, 64))
    x, w1, b1, w2, b2 = (a.astype(np.float64) for a in args)
    want = np.maximum(x @ w1 + b1, 0) @ w2 + b2
    err = float(np.abs(y - want).max() / np.abs(want).max())
    flops = 2.0 * 256 * 128 * 512 + 2.0 * 256 * 512 * 64
    for b in dev_in + dev_out:
        b.free()
    lp.close()
    res = {"workload": "C1 f32 MLP x[256,128] @ W1[128,512] + b1, relu, @ W2[512,64] + b2",
           "ms_per_step": ms_step, "kernel_ms": ms_kernel,
           "gflops": round(flops / (ms_kernel * 1e-3) / 1e9, 2), "max_rel_err": err}
    if with_cpu:
        cpu, ycpu = cpu_baseline_c1(args)
        cpu["max_rel_diff_vs_gpu"] = float(np.abs(ycpu - y).max() / np.abs(y).max())
        res["cpu_baseline"] = cpu
    return res


def bench_c5(rt, reps=3, with_cpu=False):
    """Config 5: GPT decoder (12 layers, d 768, vocab 32000, bf16), 512-token
    prompt then 128 greedy decode steps in one FOR loop.  Decode tokens/s comes
    from the difference between the full program and the same program cut to 8
    loop trips (prefill and launch cancel).  Both run on the lane count the
    scheduler picks for the full program (lane_fit), so that their prefills
    are the same work on the same lanes."""
    import dataclasses
    from pjrt_amd import configs as CF
    from pjrt_amd import scheduler as S
    c = CF.C5
    args = CF.gpt_inputs(c)
    dev_in = [rt.to_device(a) for a in args]
    lanes = S.lane_fit(CF.gpt_c5(c), rt.scheduler_config())
    times = {}
    toks = None
    for trips in (c.steps, 8):
        lp = rt.compile(CF.gpt_c5(c, trips=trips), nlanes=lanes, fit_lanes=False)
        dev_out = lp.alloc_outputs()
        _, ms = time_program(rt, lp, dev_in, dev_out, reps, 1)
        times[trips] = ms
        if trips == c.steps:
            toks = np.concatenate([dev_out[0].to_host(np.int32, (1,)), dev_out[1].to_host(np.int32, (c.steps,))])
        for b in dev_out:
            b.free()
        lp.close()
    for b in dev_in:
        b.free()
    per_tok = (times[c.steps] - times[8]) / (c.steps - 8)
    ctx_avg = c.prompt + (c.steps - 1) / 2.0
    bytes_tok = 219021312 + 36864 * ctx_avg              # weights + LM head + KV read per token
    achieved = bytes_tok / (per_tok * 1e-3) / 1e9
    assert toks.min() >= 0 and toks.max() < c.vocab
    res = {"workload": "C5 GPT decoder 12L d768 H12 mlp3072 vocab32000 bf16, prompt 512, 128 greedy steps "
                       "in one FOR loop", "lanes": lanes,
           "decode_tokens_per_s": round(1e3 / per_tok, 1), "ms_per_token": round(per_tok, 4),
           "program_ms": round(times[c.steps], 3), "prefill_plus_8_steps_ms": round(times[8], 3),
           "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(achieved / HBM_PEAK_GBS, 4), "bytes_per_token": int(bytes_tok),
                        # measured FETCH_SIZE + WRITE_SIZE per decode token, calibrated against a copy
                        # (profiles/vm_main_c5_traffic.txt)
                        "traffic": (load_traffic("c5") or {}).get("bytes_per_token")}}
    if with_cpu:
        log("C5 CPU baseline")
        cpu, ctoks = cpu_baseline_c5(c, args)
        same = 0
        while same < len(ctoks) and ctoks[same] == toks[same]:
            same += 1
        cpu["leading_tokens_equal_to_gpu"] = same     # f32 against bf16 activations: informational
        res["cpu_baseline"] = cpu
    return res


def profile_c5(rt, steps=16):
    """--device-profile: where a C5 decode step spends its time, from the
    runtime's per-task device counters (the runtime is created with
    PJRT_AMD_PROFILE=1).  The per-step figures are the difference between the
    decoder with `steps` loop trips and the same program with none, divided by
    `steps`: the grid barriers each lane passes and its average wait in them,
    and per tile op the entries, the mean time of one entry and the lane-time."""
    import dataclasses
    from pjrt_amd import configs as CF
    from pjrt_amd import scheduler as S
    from pjrt_amd import vmprogram as V
    c = dataclasses.replace(CF.C5, steps=steps)
    args = CF.gpt_inputs(c)
    dev_in = [rt.to_device(a) for a in args]
    # both programs on the lane count of the benchmarked decoder (128 steps),
    # so that the difference holds the decode steps and nothing else
    cfg = rt.scheduler_config()
    cfg = dataclasses.replace(cfg, nlanes=S.lane_fit(CF.gpt_c5(CF.C5), cfg), fit_lanes=False)
    res = {}
    for trips in (0, steps):
        prog = CF.gpt_c5(c, trips=trips)
        sched = S.schedule_program(prog, cfg)
        lp = rt.load(V.serialize(prog, sched))
        outs = lp.alloc_outputs()
        lp.execute(dev_in, outs)
        lp.profile(reset=True)
        e0, e1 = rt.event(), rt.event()
        e0.record()
        lp.execute(dev_in, outs)
        e1.record()
        rt.synchronize()
        res[trips] = (e0.elapsed_ms(e1), lp.profile(), sched)
        for b in outs:
            b.free()
        lp.close()
    for b in dev_in:
        b.free()
    names = {v: k for k, v in vars(V).items() if k.startswith("TOP_") and k != "TOP_MAX"}
    (ms0, pr0, _), (ms1, pr1, sched) = res[0], res[steps]
    lanes = sched.n_lanes
    per_step_us = (ms1 - ms0) * 1e3 / steps
    bar_n = (pr1["barriers"] - pr0["barriers"]) / lanes / steps
    bar_us = (pr1["barrier_us"] - pr0["barrier_us"]) / lanes / steps
    span_us = (pr1["lane_us"] - pr0["lane_us"]) / lanes / steps
    flag_us = (pr1["flag_us"] - pr0["flag_us"]) / lanes / steps
    tile_us = (sum(t[1] for t in pr1["tasks"]) - sum(t[1] for t in pr0["tasks"])) / lanes / steps
    print(f"C5 decode step on {lanes} lanes: {per_step_us:.1f} us per step (events), "
          f"{bar_n:.1f} grid barriers per step, average lane wait in them {bar_us:.1f} us per step "
          f"({bar_us / max(bar_n, 1):.2f} us per barrier)")
    # where one lane's step goes: the lane's span (launch start to its end) is
    # its tiles, its barrier waits, its completion-flag waits and the rest
    # (entry loads, the frame walk, block barriers between entries, and the
    # profiling atomics themselves)
    print("per lane and decode step (us):")
    for name, v in (("tiles (entries, incl. their closing block barrier)", tile_us),
                    ("grid barrier waits", bar_us), ("completion-flag waits", flag_us),
                    ("rest: entry dispatch, frame walk, profiling", span_us - tile_us - bar_us - flag_us),
                    ("lane span (sum of the above)", span_us), ("kernel time per step (events)", per_step_us)):
        print(f"  {name:52s} {v:8.1f}")
    base = {i: (tot, cnt) for i, tot, _, cnt in pr0["tasks"]}
    by_op, rows = {}, []
    for i, tot, mx, cnt in pr1["tasks"]:
        t0, c0 = base.get(i, (0.0, 0))
        n = (cnt - c0) / steps
        if n <= 0:
            continue
        lane_us = (tot - t0) / steps
        t = sched.tasks[i]
        op = names.get(t.tile_op & 0xFF, str(t.tile_op & 0xFF))
        e = by_op.setdefault(op, [0.0, 0.0, 0])
        e[0] += n
        e[1] += lane_us
        e[2] += 1
        rows.append((lane_us, i, op, n, lane_us / n, mx))
    print(f"{'tile op':18s} {'tasks':>5s} {'entries/step':>12s} {'us/entry':>9s} {'lane-us/step':>12s} "
          f"{'us/step (/lanes)':>16s}")
    for op, (n, us, k) in sorted(by_op.items(), key=lambda kv: -kv[1][1]):
        print(f"{op:18s} {k:5d} {n:12.1f} {us / n:9.2f} {us:12.1f} {us / lanes:16.2f}")
    print("heaviest tasks: task, op, entries/step, us/entry, max us/entry, lane-us/step")
    for lane_us, i, op, n, avg, mx in sorted(rows, reverse=True)[:24]:
        print(f"{i:5d} {op:18s} {n:8.1f} {avg:9.2f} {mx:9.2f} {lane_us:10.1f}")


def bench_copy(rt, steps, nbytes=128 << 20):
    """A plain device-to-device copy of known size (the runtime's hipMemcpyAsync):
    the calibration kernel for the FETCH_SIZE / WRITE_SIZE counters."""
    a, b = rt.alloc(nbytes), rt.alloc(nbytes)
    rt.d2d(b.ptr, a.ptr, nbytes)
    rt.synchronize()
    e0, e1 = rt.event(), rt.event()
    e0.record()
    for _ in range(steps):
        rt.d2d(b.ptr, a.ptr, nbytes)
    e1.record()
    rt.synchronize()
    ms = e0.elapsed_ms(e1) / steps
    a.free()
    b.free()
    return {"workload": f"device-to-device copy of {nbytes} bytes", "bytes": nbytes, "ms_per_copy": ms,
            "gbs_read_plus_write": round(2 * nbytes / (ms * 1e-3) / 1e9, 2)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workloads", default="c1,c2,c3,c4,c5,lowered")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-vendor", action="store_true",
                    help="skip the vendor-library comparison figures (torch.matmul in a child process)")
    ap.add_argument("--device-profile", action="store_true",
                    help="profiling aid: print the per-task device profile of the C5 decode step and exit")
    ap.add_argument("--c2-cache", choices=("both", "cold", "warm"), default="both",
                    help="config 2: the cold-cache headline and the warm figure beside it (default), or only one "
                         "of them (profiling runs)")
    ap.add_argument("--skip-c2", action="store_true",
                    help="profiling aid: run only the --workloads extras and print them as one JSON line "
                         "(no headline C2 measurement)")
    args = ap.parse_args()
    if args.gpus != 1:
        raise SystemExit("bench.py measures one GPU: this build has no multi-GPU path "
                         "(each GPU would run its own shard of the same megakernel; see DESIGN.md)")
    if args.no_vendor:
        os.environ["PJRT_AMD_BENCH_NO_VENDOR"] = "1"
    if args.device_profile:
        os.environ["PJRT_AMD_PROFILE"] = "1"       # read when the runtime is created
    from pjrt_amd.runtime import Runtime
    with Runtime(device=0) as rt:      # closed (programs first) before interpreter exit
        if args.device_profile:
            profile_c5(rt)
        else:
            run(args, rt)


def run(args, rt):
    log(f"device {rt.info['name']} {rt.info['arch']} lanes={rt.info['n_lanes']}")
    wl = set(args.workloads.split(","))
    extra = {}
    for dt in ("bf16", "f32"):
        if "c3" in wl or f"c3_{dt}" in wl:
            log(f"C3 {dt}")
            extra[f"c3_{dt}"] = bench_gemm(rt, dt, max(5, args.steps // 5), 2, with_cpu=not args.no_cpu)
    if "c3_bf16" in extra and extra.get("c3_f32", {}).get("cpu_baseline"):
        # bf16 dot_general is unsupported on the reference (its matmul reads the
        # operands as f32, ops/dot.py:158): the f32 leg is the widened equivalent
        extra["c3_bf16"]["cpu_baseline"] = dict(extra["c3_f32"]["cpu_baseline"],
                                                reference_support="unsupported (f32-widened equivalent: the f32 leg)")
    if "c4" in wl:
        log("C4")
        extra["c4"] = bench_attention(rt, max(5, args.steps // 5), 2, with_cpu=not args.no_cpu)
    if "c4" in wl or "attn_variants" in wl:
        # the same causal shape on the f32 kernel and with 256-wide bf16 heads
        # (informational: not BASELINE configs)
        log("attention variants")
        extra["c4_f32"] = bench_attention(rt, max(3, args.steps // 10), 1, dt="f32")
        extra["c4_d256"] = bench_attention(rt, max(3, args.steps // 10), 1, D=256)
    if "c1" in wl:
        log("C1")
        extra["c1"] = bench_c1(rt, max(5, args.steps), not args.no_cpu)
    if "c5" in wl:
        log("C5")
        extra["c5"] = bench_c5(rt, with_cpu=not args.no_cpu)
    if "lowered" in wl:
        log("lowered")
        extra["lowered"] = bench_lowered(rt, max(5, args.steps // 5))
    if "copy" in wl:
        log("copy")
        extra["copy"] = bench_copy(rt, max(5, args.steps // 5))
    if args.skip_c2:
        print(json.dumps({"extra": extra}), flush=True)
        return
    log("C2")
    c2 = bench_c2(rt, args.steps, args.warmup, not args.no_cpu, cache=args.c2_cache)
    line = {
        "metric": METRIC, "value": round(c2["value"], 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(c2["ms_per_step"], 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "C2 fused layernorm(eps=1e-5, gamma/beta) + tanh-GELU + f32->bf16 on x[8192,4096] f32",
                   "rows": C2_ROWS, "d": C2_D, "bytes_per_step": C2_BYTES, "kernel_ms": round(c2["kernel_ms"], 5),
                   "cache": c2["cache"]},
        "roofline": c2["roofline"], "cpu_baseline": c2["cpu_baseline"], "warm_cache": c2["warm"],
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
