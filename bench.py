#!/usr/bin/env python3
"""Benchmark of the MI355X-native OxideForge compute core (one GPU).

Headline (BASELINE.json metric, configs[2]): f32 GEMM C = A * B at
M = N = K = 4096, TFLOP/s, with its fraction of the fp32-MFMA peak.  A "step"
is one GEMM launch over inputs already resident in HBM; the timed region is
bracketed by synchronisation and timed with HIP events on the stream the
kernel runs on, and every figure is the median over five groups of
back-to-back launches (time_launches).  Secondary figures in the same JSON
line: the 8192x1024x4096 GEMM, the [8192,4096] transpose, the C2 row and
elementwise kernels, the sum-reduce kernels and the column sums (GB/s,
rotating over >= 512 MiB of buffers so the 256 MiB MALL cannot serve them),
and the transformer executors when built.

The CPU baseline is the C mirror (oracle/oxforge_oracle.c: f64-accumulate
GEMM, row kernels) on bounded samples of the same workloads, one thread per
CPU the host grants this process (nproc and the share are both reported);
with the secondary figures, the transformer layer's host tokens/s (one C4
forward and one C5 training step of the C mirror) is reported beside the
GPU's.  Inputs come from
oxforge.synth; the oracle is imported only by the CPU legs.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
       [--no-secondary] [--sweep]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "oxide-forge_amd"))
sys.path.insert(0, ROOT)

from oxforge import synth  # noqa: E402  (seeded inputs; the package, not the oracle)

METRIC = "f32 GEMM TFLOP/s (% fp32-MFMA peak); transformer layer tokens/sec, 1 GPU"
PEAK_FP32_MFMA_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


SPIN_UP_S = 0.3


TIMING_GROUPS = 5


def time_launches(rt, fn, steps: int, warmup: int, stream=None) -> float:
    """Milliseconds per launch of fn(i): the median over TIMING_GROUPS groups
    of back-to-back launches (`steps` in all) of each group's mean, from HIP
    events on `stream` recorded only at the group boundaries.

    An event pair around every launch would add about 2.6 us of dispatch
    idle per launch (measured on MI355X: C2 softmax 6.3 us back to back,
    8.9 us event-bracketed; a 4096^3 GEMM 903 against 905 us), which is
    half of a C2 kernel's time, so launches are timed in groups and the
    median is taken over the groups.

    Warmup runs at least `warmup` launches and at least SPIN_UP_S seconds of
    the same work: the MI355X raises its clocks over the first tens of
    milliseconds of sustained load (a 4096^3 GEMM dispatch drops from about
    1.1-1.2 ms to 0.95 ms over its first ~20 launches, and to 0.90 ms in the
    steady state), and the timed steps should see the steady state."""
    t0 = time.perf_counter()
    i = 0
    while i < warmup or time.perf_counter() - t0 < SPIN_UP_S:
        fn(i)
        i += 1
        if i % 8 == 0:
            rt.sync(stream)
    rt.sync(stream)
    groups = max(1, min(TIMING_GROUPS, steps))
    bounds = [steps * g // groups for g in range(groups + 1)]
    evs = [rt.event() for _ in range(groups + 1)]
    rt.record(evs[0], stream)
    for g in range(groups):
        for i in range(bounds[g], bounds[g + 1]):
            fn(i)
        rt.record(evs[g + 1], stream)
    rt.sync(stream)
    per = sorted(rt.elapsed_ms(evs[g], evs[g + 1]) / (bounds[g + 1] - bounds[g])
                 for g in range(groups))
    for e in evs:
        rt.event_destroy(e)
    mid = groups // 2
    return per[mid] if groups % 2 else 0.5 * (per[mid - 1] + per[mid])


def load_traffic(kernel: str):
    """HBM-side bytes per launch of `kernel` from the committed rocprofv3
    --pmc summary (profiles/traffic.json): FETCH_SIZE and WRITE_SIZE (KiB per
    dispatch), each scaled by the factor a copy kernel of known size gives
    that counter.  None if the kernel has not been measured."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            data = json.load(f)
        k = data["kernels"][kernel]
        fetch = k["fetch_kib"] * 1024 * data["fetch_factor"]
        write = k["write_kib"] * 1024 * data["write_factor"]
        return int(round(fetch + write))
    except (OSError, KeyError, ValueError):
        return None


def gemm_tflops(rt, M, N, K, steps, warmup, seed=3):
    A = synth.uniform((M, K), seed)
    B = synth.uniform((K, N), seed + 1)
    dA, dB, dC = rt.array(A), rt.array(B), rt.empty((M, N))
    ms = time_launches(rt, lambda i: rt.gemm(dA, dB, dC, M, N, K), steps, warmup)
    for d in (dA, dB, dC):
        d.recycle()
    return 2.0 * M * N * K / (ms * 1e-3) / 1e12, ms


def rotating(rt, shape, sets, seed):
    base = rt.array(synth.normal(shape, seed))
    bufs = [base]
    for _ in range(sets - 1):
        b = rt.empty(shape)
        rt.copy(b, base)
        bufs.append(b)
    return bufs


def secondary(rt, steps, warmup, extended):
    out = {}
    log("gemm 8192x1024x4096")
    t, ms = gemm_tflops(rt, 8192, 1024, 4096, steps, warmup)
    out["gemm_8192x1024x4096"] = {"tflops": round(t, 2), "ms": round(ms, 4),
                                  "frac_mfma_peak": round(t / PEAK_FP32_MFMA_TFLOPS, 4)}

    log("transpose 8192x4096")
    R, C = 8192, 4096
    xs = rotating(rt, (R, C), 2, 21)
    ys = [rt.empty((C, R)) for _ in range(2)]
    ms = time_launches(rt, lambda i: rt.transpose(xs[i % 2], ys[i % 2], R, C), max(steps, 64),
                       warmup)
    gbs = 2 * R * C * 4 / (ms * 1e-3) / 1e9
    out["transpose_8192x4096"] = {"gbs": round(gbs, 1), "ms": round(ms, 4),
                                  "frac_hbm_peak": round(gbs / PEAK_HBM_GBS, 4)}
    for b in xs + ys:
        b.recycle()

    out.update(secondary_rows(rt, steps, warmup, extended))
    out.update(secondary_rows_at_scale(rt, steps, warmup))
    return out


def secondary_rows_at_scale(rt, steps, warmup, min_launches=32):
    """The same row and streaming kernels on X [65536, 1024] (256 MiB per
    operand, two rotating sets: 512 MiB, beyond the 256 MiB MALL).  At the
    C2 size a launch lasts 7-15 us and its ramp-up and drain are a large
    part of it; here the kernels run long enough to show the bandwidth they
    sustain."""
    import oxforge

    out = {}
    rows, cols, sets = 65536, 1024, 2
    X = 4 * rows * cols
    log("row ops 65536x1024")
    xs = rotating(rt, (rows, cols), sets, 2)
    gs = rotating(rt, (rows, cols), sets, 3)
    ds = [rt.empty((rows, cols)) for _ in range(sets)]
    gam = rt.array(synth.normal((cols,), 4, 1.0, 0.1))
    bet = rt.array(synth.normal((cols,), 5, 0.0, 0.1))
    dgam, dbet = rt.empty((cols,)), rt.empty((cols,))
    rvec = rt.array(synth.normal((cols,), 6))
    cases = {
        "softmax_fwd": (2 * X, lambda i: rt.softmax_rows(xs[i % sets], rows, cols)),
        "layer_norm_fwd": (2 * X, lambda i: rt.layer_norm(xs[i % sets], rows, cols, gam, bet)),
        "rms_norm_fwd": (2 * X, lambda i: rt.rms_norm(xs[i % sets], rows, cols, gam)),
        "softmax_bwd": (3 * X, lambda i: rt.softmax_rows_bwd(xs[i % sets], gs[i % sets],
                                                             ds[i % sets], rows, cols)),
        "layer_norm_bwd": (3 * X, lambda i: rt.layer_norm_bwd(xs[i % sets], gs[i % sets],
                                                              ds[i % sets], rows, cols, gam,
                                                              dgam, dbet)),
        "rms_norm_bwd": (3 * X, lambda i: rt.rms_norm_bwd(xs[i % sets], gs[i % sets],
                                                          ds[i % sets], rows, cols, gam, dgam)),
        "binary_add": (3 * X, lambda i: rt.binary(xs[i % sets], gs[i % sets], ds[i % sets],
                                                  oxforge.ADD)),
        "map_scale": (2 * X, lambda i: rt.map(ds[i % sets], oxforge.MAP_SCALE, 1.0)),
        "by_rows_add": (2 * X, lambda i: rt.binary_assign_by_rows(ds[i % sets], rvec, rows, cols,
                                                                  oxforge.ADD)),
    }
    for name, (nbytes, fn) in cases.items():
        ms = time_launches(rt, fn, max(steps, min_launches), warmup)
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[f"{name}_65536x1024"] = {"gbs": round(gbs, 1), "us": round(ms * 1e3, 1),
                                     "frac_hbm_peak": round(gbs / PEAK_HBM_GBS, 4)}
    for b in xs + gs + ds:
        b.recycle()
    return out


def secondary_rows(rt, steps, warmup, extended=True, min_launches=256):
    """C2 row / elementwise kernels on X [4096, 1024], 32 rotating buffer
    sets (512 MiB per operand) so the MALL cannot serve them."""
    import oxforge

    out = {}
    rows, cols, sets = 4096, 1024, 32
    X = 4 * rows * cols
    log("row ops 4096x1024")
    xs = rotating(rt, (rows, cols), sets, 2)
    gs = rotating(rt, (rows, cols), sets, 3)
    ds = [rt.empty((rows, cols)) for _ in range(sets)]
    gam = rt.array(synth.normal((cols,), 4, 1.0, 0.1))
    bet = rt.array(synth.normal((cols,), 5, 0.0, 0.1))
    dgam, dbet = rt.empty((cols,)), rt.empty((cols,))
    rvec = rt.array(synth.normal((cols,), 6))
    rsum = rt.empty((rows,))
    scalar = rt.empty((1,))
    cases = {
        "softmax_fwd": (2 * X, lambda i: rt.softmax_rows(xs[i % sets], rows, cols)),
        "layer_norm_fwd": (2 * X, lambda i: rt.layer_norm(xs[i % sets], rows, cols, gam, bet)),
        "rms_norm_fwd": (2 * X, lambda i: rt.rms_norm(xs[i % sets], rows, cols, gam)),
        "softmax_bwd": (3 * X, lambda i: rt.softmax_rows_bwd(xs[i % sets], gs[i % sets],
                                                             ds[i % sets], rows, cols)),
        "layer_norm_bwd": (3 * X, lambda i: rt.layer_norm_bwd(xs[i % sets], gs[i % sets],
                                                              ds[i % sets], rows, cols, gam,
                                                              dgam, dbet)),
        "rms_norm_bwd": (3 * X, lambda i: rt.rms_norm_bwd(xs[i % sets], gs[i % sets],
                                                          ds[i % sets], rows, cols, gam, dgam)),
        "binary_add": (3 * X, lambda i: rt.binary(xs[i % sets], gs[i % sets], ds[i % sets],
                                                  oxforge.ADD)),
        "map_scale": (2 * X, lambda i: rt.map(ds[i % sets], oxforge.MAP_SCALE, 1.0)),
        "by_rows_add": (2 * X, lambda i: rt.binary_assign_by_rows(ds[i % sets], rvec, rows, cols,
                                                                  oxforge.ADD)),
        "sum_rows": (X, lambda i: rt.sum_rows(xs[i % sets], rsum, rows, cols)),
        # The configs[1] sum-reduce kernels over the whole of X as one
        # vector (reduction.rs:4-130 via span.rs:301-411): sum, max and the
        # map_sum of a functor (0.5 x^2, the MSE loss's), each into one
        # device scalar; and the column sums of the bias gradients.
        "reduce_sum": (X, lambda i: rt.reduce_sum(xs[i % sets], scalar)),
        "reduce_max": (X, lambda i: rt.reduce_max(xs[i % sets], scalar)),
        "map_sum_half_sq": (X, lambda i: rt.map_sum(xs[i % sets], scalar, oxforge.MAP_HALF_SQ)),
        "sum_cols": (X, lambda i: rt.sum_cols(xs[i % sets], dgam, rows, cols)),
    }
    if extended:
        cases["map_gelu"] = (2 * X, lambda i: rt.map(ds[i % sets], oxforge.MAP_GELU))
    # Each launch is a few microseconds: time at least 256 of them (groups of
    # about 51), so the one-off idle gap before each group's first launch
    # reaches the emptied queue (host launch latency after the
    # synchronisation) and the group's boundary event are amortised.
    for name, (nbytes, fn) in cases.items():
        ms = time_launches(rt, fn, max(steps, min_launches), warmup)
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[f"{name}_4096x1024"] = {"gbs": round(gbs, 1), "us": round(ms * 1e3, 2),
                                    "frac_hbm_peak": round(gbs / PEAK_HBM_GBS, 4)}
    for b in xs + gs + ds + [scalar, rsum]:
        b.recycle()
    return out


def transformer_params(S, H, F, O, seed, affine):
    p = {"WQ": synth.xavier(H, H, seed), "WK": synth.xavier(H, H, seed + 1),
         "WV": synth.xavier(H, H, seed + 2), "POS": synth.xavier(S, H, seed + 3),
         "W1": synth.xavier(H, F, seed + 4), "W2": synth.xavier(F, H, seed + 5),
         "WO": synth.xavier(H, O, seed + 6)}
    import numpy as np

    for k, n in (("BQ", H), ("BK", H), ("BV", H), ("B1", F), ("B2", H), ("BO", O)):
        p[k] = np.zeros(n, np.float32)
    if affine:
        p["G1"] = synth.normal((H,), seed + 20, 1.0, 0.1)
        p["G2"] = synth.normal((H,), seed + 21, 1.0, 0.1)
        p["BE1"] = synth.normal((H,), seed + 22, 0.0, 0.1)
        p["BE2"] = synth.normal((H,), seed + 23, 0.0, 0.1)
    return p


def transformers(rt, steps, warmup):
    """C4 inference forward and C5 training step, tokens/s."""
    from oxforge import net

    out = {}
    # C4: seq 2048, hidden 1024, FFN 4096 GELU, out 1024, RMSNorm, inference.
    S, H, F, O = 2048, 1024, 4096, 1024
    log("transformer C4 inference")
    T = net.Transformer(rt, transformer_params(S, H, F, O, 4, False), S, H, F, O, net.RMS,
                        net.ENCODER_INFERENCE, qkv_streams=False)
    X = rt.array(synth.normal((S, H), 4))
    Y = rt.empty((S, O))
    ms = time_launches(rt, lambda i: T.forward(X, Y), steps, warmup)
    flops = 2.0 * S * H * H * 3 + 2.0 * S * S * H * 2 + 2.0 * S * H * F * 2 + 2.0 * S * H * O
    out["transformer_c4_inference"] = {
        "tokens_per_s": round(S / (ms * 1e-3), 1), "ms_per_forward": round(ms, 4),
        "tflops": round(flops / (ms * 1e-3) / 1e12, 2),
        "frac_mfma_peak": round(flops / (ms * 1e-3) / 1e12 / PEAK_FP32_MFMA_TFLOPS, 4)}
    T.close()
    X.recycle()
    Y.recycle()
    # C5: seq 4096, hidden 2048, FFN 8192 GELU, out 2048, LayerNorm, training.
    S, H, F, O = 4096, 2048, 8192, 2048
    log("transformer C5 training step")
    T = net.Transformer(rt, transformer_params(S, H, F, O, 5, True), S, H, F, O, net.LAYER,
                        net.ENCODER_TRAINING)
    X = rt.array(synth.normal((S, H), 5))
    dY = rt.array(synth.normal((S, O), 6))
    Y = rt.empty((S, O))
    dX = rt.empty((S, H))

    def step(i):
        T.forward(X, Y)
        T.backward(dY, 1e-3, dX)

    ms = time_launches(rt, step, max(3, steps // 2), 2)
    fwd = 2.0 * S * H * H * 3 + 2.0 * S * S * H * 2 + 2.0 * S * H * F * 2 + 2.0 * S * H * O
    flops = 3 * fwd
    out["transformer_c5_training"] = {
        "tokens_per_s": round(S / (ms * 1e-3), 1), "ms_per_step": round(ms, 3),
        "tflops_algorithmic": round(flops / (ms * 1e-3) / 1e12, 2),
        "frac_mfma_peak": round(flops / (ms * 1e-3) / 1e12 / PEAK_FP32_MFMA_TFLOPS, 4)}
    T.close()
    for d in (X, dY, Y, dX):
        d.recycle()
    return out


def host_cpus() -> dict:
    """CPUs of the host and the share this process may use: nproc
    (os.cpu_count), the affinity mask, and the cgroup v2 CPU quota
    (cpu.max) when one is set.  The baselines run one thread per usable CPU:
    min(affinity, quota)."""
    nproc = os.cpu_count() or 1
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = nproc
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, period = f.read().split()[:2]
        if q != "max":
            quota = float(q) / float(period)
    except (OSError, ValueError):
        pass
    usable = affinity if quota is None else max(1, min(affinity, int(quota + 0.5)))
    return {"nproc": nproc, "affinity_cpus": affinity, "cgroup_quota_cpus": quota,
            "threads": usable}


def cpu_transformer_baseline():
    """The transformer layer on the host, on the same synthetic inputs as the
    GPU runs, one thread per usable CPU: the C mirror (oracle/oxforge_oracle.c
    kernels composed in the reference's launch order, f32 with f64-accumulated
    products) for one C4 forward (oracle.transformer_forward) and one C5
    training step, forward, backward and every SGD step
    (oracle.transformer_training_step).  A reported baseline, not the
    optimisation target."""
    from oracle import oracle as orc

    cpus = host_cpus()
    threads = cpus["threads"]
    orc.set_threads(threads)
    out = {}
    S, H, F, O = 2048, 1024, 4096, 1024
    p = transformer_params(S, H, F, O, 4, False)
    X = synth.normal((S, H), 4)
    t0 = time.perf_counter()
    orc.transformer_forward(p, X, rms=True)
    c4 = time.perf_counter() - t0
    S, H, F, O = 4096, 2048, 8192, 2048
    p = transformer_params(S, H, F, O, 5, True)
    X, dY = synth.normal((S, H), 5), synth.normal((S, O), 6)
    t0 = time.perf_counter()
    orc.transformer_training_step(p, X, dY, 1e-3, rms=False)
    c5 = time.perf_counter() - t0
    out["c4_inference_tokens_per_s"] = round(2048 / c4, 1)
    out["c5_training_tokens_per_s"] = round(4096 / c5, 1)
    out.update({"cores": threads, "nproc": cpus["nproc"], "kind": "port",
                "sample": f"one C4 forward ({c4:.1f} s) and one C5 training step ({c5:.1f} s) "
                          f"of the C mirror, {threads} threads"})
    return out


def sweep(rt, steps, warmup):
    """Times every plain GEMM tile instance and the split-K candidates on the
    C3, C4 and C5 GEMM shapes."""
    import oxforge
    from oxforge import _lib

    lib = oxforge.load()
    res = {}
    for (M, N, K) in GEMM_SHAPES:
        A = synth.uniform((M, K), 3)
        B = synth.uniform((K, N), 4)
        dA, dB, dC = rt.array(A), rt.array(B), rt.empty((M, N))
        for tag in ["128x256x32_x", "128x128x32_x", "128x64x32_x", "128x64x32_x@2",
                    "64x128x32_x", "64x128x32_x@2", "64x128x32_x8", "64x64x32_x"]:
            key = f"{M}x{N}x{K}:{tag}"

            def fn(i, tag=tag.encode()):
                _lib.check(lib.forge_gemm_f32_tile(rt.handle, None, tag, dA.slice, dB.slice,
                                                   dC.slice, M, N, K), "forge_gemm_f32_tile")

            try:
                ms = time_launches(rt, fn, steps, warmup)
            except oxforge.ForgeError as e:
                res[key] = f"error: {e}"
                continue
            res[key] = round(2.0 * M * N * K / (ms * 1e-3) / 1e12, 2)
            log(f"sweep {key}: {res[key]}")
        # Split-K candidates for the shapes with few output tiles.
        for tag in ["128x128x32_x", "128x64x32_x", "64x128x32_x", "64x64x32_x"]:
            for splits in (2, 4):
                key = f"{M}x{N}x{K}:{tag}:split{splits}"
                try:
                    ms = time_launches(rt, lambda i, t=tag, sp=splits: rt.gemm_split(
                        t, sp, dA, dB, dC, M, N, K), steps, warmup)
                except oxforge.ForgeError as e:
                    res[key] = f"error: {e}"
                    continue
                res[key] = round(2.0 * M * N * K / (ms * 1e-3) / 1e12, 2)
                log(f"sweep {key}: {res[key]}")
        for d in (dA, dB, dC):
            d.recycle()
    return res


GEMM_SHAPES = [(4096, 4096, 4096), (8192, 1024, 4096),
               # C4 GEMMs: QKV/out, QK^T, AV, FFN1, FFN2
               (2048, 1024, 1024), (2048, 2048, 1024), (2048, 1024, 2048), (2048, 4096, 1024),
               (2048, 1024, 4096),
               # C5 GEMMs
               (4096, 2048, 2048), (4096, 4096, 2048), (4096, 2048, 4096), (4096, 8192, 2048),
               (4096, 2048, 8192)]


def vendor_gemm(steps, warmup):
    """The vendor library on the same plain products, for comparison only:
    torch.mm on the GPU (hipBLASLt / rocBLAS as PyTorch dispatches it) in
    strict fp32 (TF32 off), timed with events on torch's current stream over
    `steps` launches after a spin-up, as time_launches does."""
    import torch

    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False
    res = {}
    dev = torch.device("cuda:0")
    for (M, N, K) in GEMM_SHAPES:
        a = torch.from_numpy(synth.uniform((M, K), 3)).to(dev)
        b = torch.from_numpy(synth.uniform((K, N), 4)).to(dev)
        c = torch.empty((M, N), device=dev)
        t0 = time.perf_counter()
        i = 0
        while i < warmup or time.perf_counter() - t0 < SPIN_UP_S:
            torch.mm(a, b, out=c)
            i += 1
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            torch.mm(a, b, out=c)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        res[f"{M}x{N}x{K}"] = round(2.0 * M * N * K / (ms * 1e-3) / 1e12, 2)
        log(f"vendor {M}x{N}x{K}: {res[f'{M}x{N}x{K}']} TFLOP/s")
        del a, b, c
    return {"library": f"torch {torch.__version__} torch.mm, fp32 (TF32 off)", "tflops": res}


def profile_workload(rt, name, steps, warmup):
    """Runs one workload `steps` times (for rocprofv3 runs) and returns its
    average time.  copy: an identity map over 256 MiB (reads and writes
    exactly 256 MiB per launch), the calibration kernel for FETCH_SIZE and
    WRITE_SIZE."""
    import oxforge
    from oxforge import net

    if name in ("gemm4096", "gemm8192x1024"):
        M, N, K = (4096, 4096, 4096) if name == "gemm4096" else (8192, 1024, 4096)
        t, ms = gemm_tflops(rt, M, N, K, steps, warmup)
        return {"workload": name, "ms": round(ms, 5), "tflops": round(t, 3)}
    if name == "copy":
        # x = x * 1.0 with the scale a kernel argument: one read and one
        # write per element that the compiler cannot elide.
        n = 64 * 1024 * 1024
        x = rt.empty((n,))
        rt.fill(x, 1.0)
        ms = time_launches(rt, lambda i: rt.map(x, oxforge.MAP_SCALE, 1.0), steps, warmup)
        return {"workload": name, "ms": round(ms, 5), "bytes_per_launch": 2 * 4 * n,
                "gbs": round(2 * 4 * n / (ms * 1e-3) / 1e9, 1)}
    if name == "transpose":
        # Two rotating input/output pairs (512 MiB), as the bench line times it.
        R, C = 8192, 4096
        xs = rotating(rt, (R, C), 2, 21)
        ys = [rt.empty((C, R)) for _ in range(2)]
        ms = time_launches(rt, lambda i: rt.transpose(xs[i % 2], ys[i % 2], R, C), steps, warmup)
        return {"workload": name, "ms": round(ms, 5)}
    if name in ("c4", "c4streams", "c5"):
        if name in ("c4", "c4streams"):
            # c4streams: the same forward with Q, K and V on three forked
            # streams (attention.rs:65-102) instead of one batched launch.
            S, H, F, O = 2048, 1024, 4096, 1024
            T = net.Transformer(rt, transformer_params(S, H, F, O, 4, False), S, H, F, O,
                                net.RMS, net.ENCODER_INFERENCE,
                                qkv_streams=name == "c4streams")
            X, Y = rt.array(synth.normal((S, H), 4)), rt.empty((S, O))
            ms = time_launches(rt, lambda i: T.forward(X, Y), steps, warmup)
        else:
            S, H, F, O = 4096, 2048, 8192, 2048
            T = net.Transformer(rt, transformer_params(S, H, F, O, 5, True), S, H, F, O,
                                net.LAYER, net.ENCODER_TRAINING)
            X, dY = rt.array(synth.normal((S, H), 5)), rt.array(synth.normal((S, O), 6))
            Y, dX = rt.empty((S, O)), rt.empty((S, H))

            def step(i):
                T.forward(X, Y)
                T.backward(dY, 1e-3, dX)

            ms = time_launches(rt, step, steps, warmup)
        T.close()
        return {"workload": name, "ms": round(ms, 4)}
    if name == "gemms":
        ours = {}
        for (M, N, K) in GEMM_SHAPES:
            t, _ = gemm_tflops(rt, M, N, K, steps, warmup)
            ours[f"{M}x{N}x{K}"] = {"tflops": round(t, 2), "kernel": rt.gemm_kernel_name(M, N, K)}
        return {"workload": name, "results": ours}
    if name == "ksweep":
        return {"workload": name, "results": gemm_k_sweep(rt, steps, warmup)}
    if name == "rows":
        return {"workload": name, "results": secondary_rows(rt, steps, warmup, min_launches=1)}
    if name == "rows65536":
        return {"workload": name,
                "results": secondary_rows_at_scale(rt, steps, warmup, min_launches=1)}
    if name == "sumcols":
        # Column sums of the bias-gradient and norm-backward shapes, over
        # rotating copies (at least 512 MiB, or two) so the MALL cannot
        # serve them; the first-pass shape follows $OXFORGE_SUMCOL_LOADS and
        # $OXFORGE_SUMCOL_BLOCKS when they are set.
        res = {}
        for rows, cols in ((4096, 1024), (4096, 2048), (65536, 1024), (4096, 8192)):
            sets = max(2, min(32, (512 << 20) // (4 * rows * cols)))
            xs = rotating(rt, (rows, cols), sets, 2)
            out = rt.empty((cols,))
            ms = time_launches(rt, lambda i: rt.sum_cols(xs[i % sets], out, rows, cols), steps,
                               warmup)
            res[f"{rows}x{cols}"] = {"us": round(ms * 1e3, 2),
                                     "gbs": round(4 * rows * cols / (ms * 1e-3) / 1e9, 1)}
            for b in xs + [out]:
                b.recycle()
        return {"workload": name, "loads": os.environ.get("OXFORGE_SUMCOL_LOADS", "default"),
                "blocks": os.environ.get("OXFORGE_SUMCOL_BLOCKS", "default"), "results": res}
    if name == "dsfold":
        # The C5 attention backward's softmax step both ways, kernel by
        # kernel: the plain dP product, the softmax backward over P and dP,
        # and the LayerNorm backward (gamma/beta, their SGD steps) -- against
        # the dP product that stores dS in its epilogue and the LayerNorm
        # backward that also writes the row term.  P rotates over four
        # [S, S] matrices (256 MiB) so the MALL cannot serve it.
        S, H = 4096, 2048
        s = 1.0 / H ** 0.5
        R, V = rt.array(synth.normal((S, H), 1)), rt.array(synth.normal((S, H), 2))
        Ps = rotating(rt, (S, S), 4, 3)
        dP, dS = rt.empty((S, S)), rt.empty((S, S))
        X, dY, Xin = (rt.array(synth.normal((S, H), k)) for k in (9, 10, 12))
        dX, dot = rt.empty((S, H)), rt.empty((S,))
        g, b = rt.array(synth.normal((H,), 11, 1.0, 0.1)), rt.array(synth.normal((H,), 13))
        dg, db = rt.empty((H,)), rt.empty((H,))
        cases = {
            "dP product": lambda i: rt.gemm_ex(R, V, dP, S, S, H, trans_b=True),
            "softmax backward": lambda i: rt.softmax_rows_bwd_scaled(Ps[i % 4], dP, dS, S, S, s),
            "layer norm backward": lambda i: rt.layer_norm_bwd_sgd(
                X, dY, dX, S, H, 0.0, gamma=g, beta=b, dgamma=dg, dbeta=db),
            "dS product": lambda i: rt.gemm_ex(R, V, dS, S, S, H, trans_b=True, alpha=s,
                                               row_sub=dot, aux_mul=Ps[i % 4]),
            "layer norm backward + row dot": lambda i: rt.layer_norm_bwd_sgd_dot(
                X, dY, dX, Xin, dot, S, H, 0.0, dot_scale=s, gamma=g, beta=b, dgamma=dg,
                dbeta=db),
        }
        res = {k: round(time_launches(rt, fn, steps, warmup) * 1e3, 2) for k, fn in cases.items()}
        return {"workload": name, "us": res}
    raise SystemExit(f"unknown profile workload {name}")


KSWEEP_TILES = ("64x128x32_x", "64x128x32_x8", "128x64x32_x")
KSWEEP_KS = (32, 64, 128, 256, 512, 1024, 2048, 4096)


def gemm_k_sweep(rt, steps, warmup):
    """Plain 2048 x 1024 x K products (one tile per CU) for each tile in
    KSWEEP_TILES and K in KSWEEP_KS, `steps` launches each after the clock
    spin-up, with a 4096^3 product between groups so the device never idles
    (its clock would drop).  Under rocprofv3 --kernel-trace the dispatches
    give the per-launch cost and the per-slab rate, and `steps` 64-float
    fills at the end a minimal launch to compare with; the returned event
    timings are averages that include launch gaps at small K."""
    M, N, W = 2048, 1024, 4096
    wa, wb = rt.array(synth.uniform((W, W), 1)), rt.array(synth.uniform((W, W), 2))
    wc = rt.empty((W, W))
    ops = {K: (rt.array(synth.uniform((M, K), 5)), rt.array(synth.uniform((K, N), 6)))
           for K in KSWEEP_KS}
    C = rt.empty((M, N))
    time_launches(rt, lambda i: rt.gemm(wa, wb, wc, W, W, W), 1, warmup)
    res = {}
    e0, e1 = rt.event(), rt.event()
    for tag in KSWEEP_TILES:
        for K, (A, B) in ops.items():
            rt.gemm(wa, wb, wc, W, W, W)
            rt.record(e0)
            for _ in range(steps):
                rt.gemm_tile(tag, A, B, C, M, N, K)
            rt.record(e1)
            res[f"{tag}:K={K}"] = round(rt.elapsed_ms(e0, e1) / steps * 1e3, 2)
    # A minimal launch for comparison: a 64-float fill.
    f = rt.empty((64,))
    rt.gemm(wa, wb, wc, W, W, W)
    for _ in range(steps):
        rt.fill(f, 1.0)
    rt.sync()
    f.recycle()
    rt.event_destroy(e0)
    rt.event_destroy(e1)
    for d in [wa, wb, wc, C] + [x for ab in ops.values() for x in ab]:
        d.recycle()
    return res


def cpu_baseline(M, N, K):
    """The C mirror (oracle/oxforge_oracle.c) on the host, one thread per
    usable CPU (host_cpus), on bounded samples of the GPU's workloads:
      - headline: the f64-accumulate GEMM over consecutive 512-row blocks of
        the same M x N x K product (wrapping round) until about 10 s have
        been timed, scaled to TFLOP/s;
      - row ops: C2 softmax forward (2X bytes) and LayerNorm backward with
        dgamma/dbeta (3X bytes) on X [4096, 1024], each repeated for about
        3 s, in GB/s of the same algorithmic bytes the GPU figures use."""
    from oracle import oracle as orc

    cpus = host_cpus()
    threads = cpus["threads"]
    orc.set_threads(threads)
    rows = 512
    nblk = (M + rows - 1) // rows
    A = synth.uniform((M, K), 3)
    B = synth.uniform((K, N), 4)
    t0 = time.perf_counter()
    blocks = 0
    # Consecutive blocks, wrapping round to the first after the last, until
    # about 10 s have been timed: a partial pass on a slow host, one or more
    # whole passes on a fast one.
    while True:
        b = blocks % nblk
        orc.gemm(A[b * rows:(b + 1) * rows], B)
        blocks += 1
        if time.perf_counter() - t0 >= 10.0:
            break
    dt = time.perf_counter() - t0
    tflops = 2.0 * blocks * rows * N * K / dt / 1e12

    r, c = 4096, 1024
    X = 4 * r * c
    x = synth.normal((r, c), 2)
    dy = synth.normal((r, c), 3)
    gam = synth.normal((c,), 4, 1.0, 0.1)
    xs = x.copy()  # softmax runs in place, as on the GPU
    row_ops = {}
    for name, nbytes, fn in (
            ("softmax_fwd", 2 * X, lambda: orc.lib().orc_softmax_rows(orc._p(xs), r, c)),
            ("layer_norm_bwd", 3 * X, lambda: orc.layer_norm_backward(x, dy, gam, want_params=True))):
        t1 = time.perf_counter()
        reps = 0
        while True:
            fn()
            reps += 1
            el = time.perf_counter() - t1
            if el >= 3.0:
                break
        row_ops[f"{name}_4096x1024_gbs"] = round(nbytes * reps / el / 1e9, 2)
    return {"value": round(tflops, 5), "unit": "TFLOP/s", "cores": threads,
            "nproc": cpus["nproc"], "affinity_cpus": cpus["affinity_cpus"],
            "cgroup_quota_cpus": cpus["cgroup_quota_cpus"], "kind": "port",
            "sample": f"{blocks} 512-row blocks ({blocks / nblk:.2f} passes) of the "
                      f"{M}x{N}x{K} GEMM (C mirror, f64 accumulate, {threads} threads), "
                      f"{dt:.1f} s; row ops on [4096,1024] about 3 s each",
            "row_ops": row_ops}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--extended", action="store_true")
    ap.add_argument("--sweep", action="store_true")
    ap.add_argument("--profile", default=None,
                    help="run only one workload (gemm4096, gemm8192x1024, gemms, ksweep, copy, "
                         "transpose, rows, rows65536, sumcols, dsfold, c4, c4streams, c5) for "
                         "rocprofv3, "
                         "or vendor "
                         "(torch.mm "
                         "on the same GEMM shapes, in a process without this build's runtime)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE "
              f"{world}); this build has no multi-GPU path.", file=sys.stderr)
        return 2

    if args.profile == "vendor":
        # torch's own HIP runtime: in a process of its own (a second HIP
        # runtime beside this build's finds no device).
        print(json.dumps({"workload": "vendor", "results": vendor_gemm(args.steps, args.warmup)}),
              flush=True)
        return 0

    import oxforge

    rt = oxforge.Runtime(0)
    props = rt.props()
    log(f"device {props}")
    if args.profile:
        res = profile_workload(rt, args.profile, args.steps, args.warmup)
        rt.close()
        print(json.dumps(res), flush=True)
        return 0
    M = N = K = 4096
    log("gemm 4096^3")
    tflops, ms = gemm_tflops(rt, M, N, K, args.steps, args.warmup)
    kernel = rt.gemm_kernel_name(M, N, K)
    traffic = load_traffic(kernel)
    line = {
        "metric": METRIC,
        "value": round(tflops, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (SplitMix64 uniform(-1,1), seeds 3/4)",
        "config": {"workload": "f32 GEMM C=A*B, M=N=K=4096, row-major (BASELINE configs[2])",
                   "kernel": kernel, "device": props.get("arch")},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 3),
                     "peak": PEAK_FP32_MFMA_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / PEAK_FP32_MFMA_TFLOPS, 4), "traffic": traffic},
    }
    if not args.no_secondary:
        line["secondary"] = secondary(rt, args.steps, args.warmup, args.extended)
        line["secondary"].update(transformers(rt, args.steps, args.warmup))
    if args.sweep:
        line["sweep"] = sweep(rt, args.steps, args.warmup)
    if not args.no_cpu:
        log("cpu baseline")
        line["cpu_baseline"] = cpu_baseline(M, N, K)
        if "secondary" in line:
            log("cpu baseline: transformer layer")
            line["secondary"]["cpu_baseline_transformer"] = cpu_transformer_baseline()
    rt.close()
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
