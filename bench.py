#!/usr/bin/env python3
"""Benchmark of the HIP device on one MI355X; prints ONE JSON line.

Headline workload: the fused broadcast chain
  z = tanh((x + bias) * scale) * sigmoid(x) - 0.1 * x * x
with x (8192, 4096), bias (4096,), scale (8192, 1), fp32, seed 1. A step builds
the lazy graph and realizes it (one fused kernel). value = algorithmic HBM bytes
per step / step time (GB/s); inputs are resident in HBM before the timed region
and rotate over 3 copies (3 x 128 MiB > the 256 MB Infinity Cache).

roofline: the same kernel timed with HIP events on the library's stream over
back-to-back launches of pre-built graphs. cpu_baseline: the CPU oracle
(restatement of Ormi's CPU backend, one core) on a bounded row sample.
"extra" carries the other configs (C1, C3, C4, C5), each with its own roofline.
"""
from __future__ import annotations

import argparse
import collections
import contextlib
import csv
import ctypes
import gc
import json
import math
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP32_PEAK_TFLOPS = 157.3
# Untimed work before each timed measurement, in milliseconds of wall time.
# The card's clocks rise over the first tens of milliseconds of sustained
# work: in one process, sets of 30 bf16 4096^3 GEMMs timed one after another
# took 136, 127, 120, 118, 116, then 114 us per launch.
WARM_MS = 60.0
# C1 input sets the C1 figures rotate over: 24 x 12.6 MB = 302 MB, past the 256 MB Infinity Cache.
C1_SETS = 24
METRIC = json.loads((ROOT / "BASELINE.json").read_text())["metric"]


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Events:
    """HIP events on libormi_hip's stream (the null stream every launch uses)."""

    def __init__(self):
        self.lib = ctypes.CDLL(str(ROOT / "ormi_amd" / "lib" / "libormi_hip.so"))
        self.lib.ormi_hip_event_create.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.lib.ormi_hip_event_record.argtypes = [ctypes.c_void_p]
        self.lib.ormi_hip_event_elapsed_ms.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(ctypes.c_float)]
        self.lib.ormi_hip_synchronize.argtypes = []

    def new(self):
        e = ctypes.c_void_p()
        assert self.lib.ormi_hip_event_create(ctypes.byref(e)) == 0
        return e

    def record(self, e):
        assert self.lib.ormi_hip_event_record(e) == 0

    def elapsed_ms(self, a, b) -> float:
        ms = ctypes.c_float()
        assert self.lib.ormi_hip_event_elapsed_ms(a, b, ctypes.byref(ms)) == 0
        return ms.value

    def sync(self):
        assert self.lib.ormi_hip_synchronize() == 0


@contextlib.contextmanager
def gc_paused():
    """Timed GPU loops run with Python's cyclic collector off, as timeit runs its
    loops: a collection pause otherwise lands on whichever step it hits."""
    was = gc.isenabled()
    gc.disable()
    try:
        yield
    finally:
        if was:
            gc.enable()


def timed_launches(ev: Events, make, n: int, rounds: int = 3) -> float:
    """Median over `rounds` timed sets of the average ms per iteration, each set
    n back-to-back realizations of pre-built graphs (make(i) returns a Tensor
    or a list of Tensors to realize). Untimed sets come first: the first fills
    the allocator's pool with every output block a set needs (steady state, as
    in a training loop: the timed region issues launches, not hipMalloc calls),
    and more follow until this work has run for WARM_MS of wall time."""
    def as_list(g):
        return g if isinstance(g, (list, tuple)) else [g]

    def run_set(timed: bool):
        graphs = [as_list(make(i)) for i in range(n)]
        ev.sync()
        a, b = ev.new(), ev.new()
        with gc_paused():
            ev.record(a)
            for gs in graphs:
                for g in gs:
                    g.realize()
            ev.record(b)
        ms = ev.elapsed_ms(a, b) / n
        # Autograd graphs hold reference cycles until zero_grad_graph (the
        # reference's contract); objects that own one release it here.
        for gs in graphs:
            for g in gs:
                if hasattr(g, "release"):
                    g.release()
        return ms if timed else None

    t0 = time.perf_counter()
    run_set(False)
    while (time.perf_counter() - t0) * 1e3 < WARM_MS:
        run_set(False)
    times = sorted(run_set(True) for _ in range(rounds))
    return times[len(times) // 2]


# ------------------------------------------------------------------ workloads
def c2_arrays(rows=8192, cols=4096, seed=1):
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 1, (rows, cols)).astype(np.float32)
    bias = rng.normal(0, 0.1, (cols,)).astype(np.float32)
    scale = rng.uniform(0.5, 1.5, (rows, 1)).astype(np.float32)
    return x, bias, scale


def c2_graph(X, B, S):
    return ((X + B) * S).tanh() * X.sigmoid() - 0.1 * X * X


def c2_bytes(rows=8192, cols=4096):
    return 4 * (rows * cols * 2 + cols + rows)  # read x, bias, scale; write z


def host_cpu_model() -> str:
    """The host CPU's model name as /proc/cpuinfo gives it, or "unknown"."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline_c2(target_s: float = 10.0) -> dict:
    """Oracle on one core: per-node execute_graph (what Ormi's CPU backend does on
    .numpy()) over a row sample of the C2 workload, repeated to ~target_s."""
    import oracle
    from ormi_amd import Tensor

    oracle.load()
    rows, cols = 1024, 4096
    x, bias, scale = c2_arrays(8192, cols)
    x, scale = x[:rows], scale[:rows]
    X, B, S = Tensor(x, "cpu"), Tensor(bias, "cpu"), Tensor(scale, "cpu")
    t0 = time.perf_counter()
    c2_graph(X, B, S).numpy()
    one = time.perf_counter() - t0
    reps = max(1, min(100, int(target_s / max(one, 1e-3))))
    t0 = time.perf_counter()
    for _ in range(reps):
        c2_graph(X, B, S).realize()
    per = (time.perf_counter() - t0) / reps
    # The fused tape (execute_jit on the whole chain), the favourable CPU case.
    from ormi_amd import ormi_backend as ob

    t0 = time.perf_counter()
    z = c2_graph(X, B, S)
    ob.execute_jit(z._node)
    fused = time.perf_counter() - t0
    gbs = c2_bytes(rows, cols) / per / 1e9
    return {
        "value": round(gbs, 4), "unit": "GB/s", "cores": 1, "kind": "port",
        "sample": f"C2 rows 0..{rows} of (8192,4096) (1/8 of the workload), per-node execute_graph, "
                  f"{reps} reps, {per * 1e3:.1f} ms/rep; fused-tape execute_jit {fused * 1e3:.1f} ms "
                  f"({c2_bytes(rows, cols) / fused / 1e9:.4f} GB/s); host {os.cpu_count()} cpus visible "
                  f"({host_cpu_model()})",
    }


def cpu_baselines_extra() -> dict:
    """The reference's CPU path beside the other configs, each on a bounded sample
    of a few seconds: the oracle (restatement of Ormi's CPU backend, one core, as
    its loops are unthreaded) for C1 and the C3 reductions; where the
    reference's own CPU path is built (oracle/_ref), it too for the C3 sums; and
    numpy float32 matmul (its bundled OpenBLAS, all host threads) standing in for
    the reference's cblas_sgemm for the C4 GEMMs."""
    import oracle
    from ormi_amd import Tensor

    oracle.load()
    out = {}

    def timed(fn, reps):
        fn()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        return (time.perf_counter() - t0) / reps

    rng = np.random.default_rng(0)
    a, b, c = (rng.uniform(-1, 1, (1024, 1024)).astype(np.float32) for _ in range(3))
    A, B, C = (Tensor(v, "cpu", requires_grad=True) for v in (a, b, c))
    f = timed(lambda: ((A * B + C).relu() * 0.5).sum(1).realize(), 3)

    def grads():
        for t in (A, B, C):
            t.zero_grad()
        ((A * B + C).relu() * 0.5).sum(1).sum().backward()
        for g in (A.grad, B.grad, C.grad):
            g.realize()

    g = timed(grads, 2)
    out["C1"] = {"kind": "port", "cores": 1, "fwd_ms": round(f * 1e3, 2), "fwd_GB/s": round(12587008 / f / 1e9, 4),
                 "bwd_ms": round(g * 1e3, 2), "bwd_GB/s": round(50331648 / g / 1e9, 4),
                 "sample": "full (1024,1024), per-node execute_graph"}
    rows, cols = 256, 8192
    x = np.random.default_rng(2).normal(0, 2, (rows, cols)).astype(np.float32)
    X = Tensor(x, "cpu")
    M = X.max(1, keepdims=True).realize()
    nb = rows * cols * 4
    red = {"row_max": lambda: X.max(1).realize(), "row_sumexp": lambda: (X - M).exp().sum(1).realize(),
           "row_mean": lambda: X.mean(1).realize(), "row_argmax": lambda: X.argmax(1).realize(),
           "col_sum": lambda: X.sum(0).realize()}
    c3 = {"kind": "port", "cores": 1, "sample": f"rows 0..{rows} of (16384,8192) (1/64), per-node execute_graph"}
    for k, fn in red.items():
        t = timed(fn, 2)
        c3[k] = {"ms": round(t * 1e3, 2), "GB/s": round(nb / t / 1e9, 4)}
    out["C3"] = c3
    if oracle.ref_available():
        # The reference's own CPU path (oracle/_ref, built from its sources) on
        # the C3 ops it has: the row sum behind the mean, and the column sum.
        # Each call also copies the sample in and the result out (about 1% of it).
        ref = {"kind": "reference", "cores": 1, "sample": c3["sample"]}
        for k, axis in (("row_sum", 1), ("col_sum", 0)):
            t = timed(lambda axis=axis: oracle.ref_run([(x, False)], [("SUM", 0, -1, [axis], 0)], [1]), 2)
            ref[k] = {"ms": round(t * 1e3, 2), "GB/s": round(nb / t / 1e9, 4)}
        out["C3_reference"] = ref
    try:
        from threadpoolctl import threadpool_info

        blas = [i for i in threadpool_info() if i.get("user_api") == "blas"]
        threads = blas[0]["num_threads"] if blas else None
        lib = f"{blas[0].get('internal_api')} {blas[0].get('version')}" if blas else "unknown"
    except ImportError:
        threads, lib = None, "unknown"
    rng = np.random.default_rng(3)
    a16 = rng.normal(0, 1 / 64, (4096, 4096)).astype(np.float32)
    b16 = rng.normal(0, 1 / 64, (4096, 4096)).astype(np.float32)
    t16 = timed(lambda: a16 @ b16, 2)
    a32 = rng.normal(0, 1 / 64, (2048, 1024)).astype(np.float32)
    b32 = rng.normal(0, 1 / 64, (1024, 4096)).astype(np.float32)
    t32 = timed(lambda: a32 @ b32, 3)
    out["C4"] = {"kind": "stand-in: numpy float32 matmul for cblas_sgemm", "cores": threads, "blas": lib,
                 "sgemm_4096_ms": round(t16 * 1e3, 1), "sgemm_4096_TFLOP/s": round(2 * 4096 ** 3 / t16 / 1e12, 3),
                 "sgemm_2048x1024x4096_ms": round(t32 * 1e3, 1),
                 "sgemm_2048x1024x4096_TFLOP/s": round(2 * 2048 * 1024 * 4096 / t32 / 1e12, 3),
                 "sample": "full shapes; the bf16 config as sgemm on fp32 values"}
    out["C5"] = cpu_c5_step(threads, lib, timed)
    return out


def cpu_c5_step(threads, lib: str, timed) -> dict:
    """The C5 step in numpy float32 on the host: the same seed-4 inputs, the
    eight GEMMs (numpy matmul on its bundled OpenBLAS, all host threads, for the
    reference's cblas_sgemm), erf GELU and its derivative, the MSE and the SGD
    update, as whole-array numpy passes (the reference's CPU element-wise path
    is one unthreaded kernel per node, slower still)."""
    from scipy.special import erf

    rng = np.random.default_rng(4)
    dims = [1024, 4096, 4096, 1024]
    X = rng.normal(0, 1, (1024, 1024)).astype(np.float32)
    T = rng.normal(0, 1, (1024, 1024)).astype(np.float32)
    W = [rng.uniform(-math.sqrt(6 / i), math.sqrt(6 / i), (i, o)).astype(np.float32) for i, o in zip(dims, dims[1:])]
    r2, c = np.float32(1 / math.sqrt(2)), np.float32(1.0 / (1024 * 1024))
    inv_sqrt_2pi = np.float32(1 / math.sqrt(2 * math.pi))

    def gelu(z):
        return np.float32(0.5) * z * (np.float32(1) + erf(z * r2).astype(np.float32))

    def gelu_grad(z):
        return (np.float32(0.5) * (np.float32(1) + erf(z * r2).astype(np.float32))
                + z * inv_sqrt_2pi * np.exp(np.float32(-0.5) * z * z))

    def step():
        z1 = X @ W[0]
        h1 = gelu(z1)
        z2 = h1 @ W[1]
        h2 = gelu(z2)
        y = h2 @ W[2]
        d = y - T
        loss = float((d * d).sum()) * float(c)
        dy = c * d + c * d
        dw3 = h2.T @ dy
        dz2 = (dy @ W[2].T) * gelu_grad(z2)
        dw2 = h1.T @ dz2
        dz1 = (dz2 @ W[1].T) * gelu_grad(z1)
        dw1 = X.T @ dz1
        return loss, [w - dw * np.float32(1e-3) for w, dw in zip(W, (dw1, dw2, dw3))]

    t = timed(step, 2)
    flops = 146028888064
    return {"kind": "stand-in: numpy float32 (matmul on its OpenBLAS, element-wise as whole-array passes)",
            "cores": threads, "blas": lib, "step_ms": round(t * 1e3, 1),
            "gemm_TFLOP/s": round(flops / t / 1e12, 3), "sample": "full step, batch 1024, 1024-4096-4096-1024"}


def traffic_from_profile(label: str):
    """HBM bytes per launch (read + write) of the row `label` of the committed
    rocprofv3 --pmc summary (profiles/hbm_traffic.md, written by
    `bench.py --pmc-report`: columns kernel, fetch KiB, write KiB, read bytes,
    write bytes, ...), or None when the summary has no such row."""
    f = ROOT / "profiles" / "hbm_traffic.md"
    if not f.exists():
        return None
    for line in f.read_text().splitlines():
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) >= 5 and cells[0] == label:
            try:
                return int(cells[3]) + int(cells[4])
            except ValueError:
                return None
    return None


def bench_c2(args, ev: Events) -> dict:
    """Headline workload. A step = build the lazy graph + realize it (one fused
    kernel). Inputs rotate over 3 resident copies and the last 4 outputs stay
    alive, so each step reads and writes buffers the 256 MB Infinity Cache does
    not hold from the step before."""
    from ormi_amd import Tensor

    log("C2: generating inputs")
    x, bias, scale = c2_arrays()
    sets = []
    for k in range(3):
        xs = x if k == 0 else np.ascontiguousarray(np.roll(x, k, axis=0))
        sets.append((Tensor(xs, "hip"), Tensor(bias, "hip"), Tensor(scale, "hip")))
    ring = collections.deque(maxlen=4)
    # The first realize compiles the fused kernel (hipRTC, cached in memory for
    # the rest of the process): reported on its own, outside every timed region.
    ev.sync()
    t0 = time.perf_counter()
    first = c2_graph(*sets[0]).realize()
    ev.sync()
    first_ms = (time.perf_counter() - t0) * 1e3
    del first
    # Give the allocator pool the blocks the ring cycles through (the ring's 4
    # outputs plus the one being written), so no timed step calls hipMalloc.
    [c2_graph(*sets[i % 3]).realize() for i in range(ring.maxlen + 1)]
    # Untimed steps for WARM_MS of wall time, then the W warm-up steps.
    t0, i = time.perf_counter(), 0
    while (time.perf_counter() - t0) * 1e3 < WARM_MS:
        ring.append(c2_graph(*sets[i % 3]).realize())
        i += 1
        if i % 64 == 0:
            ev.sync()
    for i in range(args.warmup):
        ring.append(c2_graph(*sets[i % 3]).realize())
    ev.sync()
    log("C2: timed steps")
    with gc_paused():
        t0 = time.perf_counter()
        for i in range(args.steps):
            ring.append(c2_graph(*sets[i % 3]).realize())
        ev.sync()
        step_s = (time.perf_counter() - t0) / args.steps
    ring.clear()
    log("C2: kernel timing (HIP events)")
    n = max(args.steps, 20)
    kernel_ms = timed_launches(ev, lambda i: c2_graph(*sets[i % 3]), n)
    nbytes = c2_bytes()
    achieved = nbytes / (kernel_ms * 1e-3) / 1e9
    return {
        "step_s": step_s,
        "first_realize_ms": first_ms,
        "value": nbytes / step_s / 1e9,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_from_profile("C2 fused map"),
                     "kernel_us": round(kernel_ms * 1e3, 2), "bytes_per_launch": nbytes, "launches_timed": n},
    }


def bench_copy(args, ev: Events) -> dict:
    """Calibration kernel for the --pmc traffic figures: y = -x over (8192, 4096)
    fp32, a fused map that reads 128 MiB and writes 128 MiB."""
    from ormi_amd import Tensor

    x = np.random.default_rng(7).normal(0, 1, (8192, 4096)).astype(np.float32)
    X = [Tensor(x, "hip"), Tensor(x[::-1].copy(), "hip"), Tensor(x[:, ::-1].copy(), "hip")]
    (-X[0]).realize()
    ms = timed_launches(ev, lambda i: -X[i % 3], max(args.steps, 20))
    nbytes = 2 * x.nbytes
    return {"us": round(ms * 1e3, 2), "GB/s": round(nbytes / ms / 1e6, 1), "bytes": nbytes}


def bench_c3(ev: Events, n: int) -> dict:
    from ormi_amd import Tensor

    log("C3: generating inputs")
    x = np.random.default_rng(2).normal(0, 2, (16384, 8192)).astype(np.float32)
    X = [Tensor(x, "hip"), Tensor(np.ascontiguousarray(x[::-1]), "hip")]
    M = [t.max(1, keepdims=True).realize() for t in X]
    rows, cols = x.shape
    inb = rows * cols * 4
    work = {
        "row_max": (lambda i: X[i % 2].max(1), inb + rows * 4),
        "row_sumexp": (lambda i: (X[i % 2] - M[i % 2]).exp().sum(1), inb + rows * 4 + rows * 4),
        "row_mean": (lambda i: X[i % 2].mean(1), inb + rows * 4),
        "row_argmax": (lambda i: X[i % 2].argmax(1), inb + rows * 8),
        "col_sum": (lambda i: X[i % 2].sum(0), inb + cols * 4),
    }
    out = {}
    for name, (make, nbytes) in work.items():
        make(0).realize()
        ms = timed_launches(ev, make, n)
        out[name] = {"us": round(ms * 1e3, 2), "GB/s": round(nbytes / ms / 1e6, 1),
                     "frac_hbm": round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 4), "bytes": nbytes}
    return out


def bench_c1(ev: Events, n: int) -> dict:
    """C1: y = sum(relu(a*b + c) * 0.5, axis=1) and the gradients of sum(y) with
    respect to a, b, c. Kernel figures come from pre-built graphs that rotate
    over C1_SETS input sets (12.6 MB each, 302 MB in all, more than the 256 MB
    Infinity Cache holds), so every realize reads its inputs from HBM; the
    *_cached figures reuse one set, which the cache then serves. The step
    figure is the host-inclusive loop (graph build + backward + realize)."""
    from ormi_amd import Tensor, realize_all

    rng = np.random.default_rng(0)
    sets = []
    for k in range(C1_SETS):
        vals = [rng.uniform(-1, 1, (1024, 1024)).astype(np.float32) for _ in range(3)]
        sets.append(tuple(Tensor(v, "hip", requires_grad=True) for v in vals))

    def fwd_on(A, B, C):
        return ((A * B + C).relu() * 0.5).sum(1)

    def grads_on(A, B, C):
        for t in (A, B, C):
            t.zero_grad()
        loss = fwd_on(A, B, C).sum()
        loss.backward()
        return loss, [A.grad, B.grad, C.grad]

    def fwd(i):
        return fwd_on(*sets[i % C1_SETS])

    def grads(i):
        return grads_on(*sets[i % C1_SETS])

    # Sets of 200 realizes, as the step loop below: a C1 kernel runs 3-4 us, so
    # a set of 30 lasts about 100 us, and the start of a set (the launch
    # thread's first launch after the start event) adds about 0.2 us per
    # realize to it (one box: 3.3 us per realize in sets of 50, 3.1 in 400).
    n = max(n, 200)
    ms_f = timed_launches(ev, fwd, n)
    ms_b = timed_launches(ev, lambda i: _Grads(*grads(i), grouped=False), n)
    ms_g = timed_launches(ev, lambda i: _Grads(*grads(i), grouped=True), n)
    ms_fc = timed_launches(ev, lambda i: fwd_on(*sets[0]), n)
    ms_gc = timed_launches(ev, lambda i: _Grads(*grads_on(*sets[0]), grouped=True), n)

    def step(i):
        loss, gs = grads(i)
        realize_all(*gs)
        loss.zero_grad_graph()  # a training step releases its graph (reference contract)

    # Steady state: 20 untimed steps, then 200 timed ones (3 ms), so the
    # final synchronize and the first steps' cold caches do not weigh in.
    for i in range(20):
        step(i)
    ev.sync()
    n_step = 200
    with gc_paused():
        t0 = time.perf_counter()
        for i in range(n_step):
            step(i)
        ev.sync()
        step_ms = (time.perf_counter() - t0) / n_step * 1e3
    fb, bb, gb = 12587008, 50331648, 25165824
    return {"fwd_us": round(ms_f * 1e3, 2), "fwd_GB/s": round(fb / ms_f / 1e6, 1),
            "bwd_separate_us": round(ms_b * 1e3, 2), "bwd_separate_GB/s": round(bb / ms_b / 1e6, 1),
            "bwd_grouped_us": round(ms_g * 1e3, 2), "bwd_grouped_GB/s": round(gb / ms_g / 1e6, 1),
            "fwd_cached_us": round(ms_fc * 1e3, 2), "bwd_grouped_cached_us": round(ms_gc * 1e3, 2),
            "bwd_step_wall_us": round(step_ms * 1e3, 1),
            "note": f"per realize, HIP events over sets of 200 pre-built graphs rotating over {C1_SETS} input sets "
                    f"({C1_SETS * 3 * 4} MiB, past the 256 MB Infinity Cache: HBM figures); *_cached: one input set, "
                    "served by the Infinity Cache (latency figures, not HBM bandwidth); "
                    "fwd: one fused reduce kernel (12,587,008 B); bwd_separate: one fused kernel per gradient root "
                    "(3 x 16,777,216 B); bwd_grouped: realize_all, one multi-output kernel (25,165,824 B); "
                    "bwd_step_wall_us: host-inclusive loop (graph build + backward + realize_all + zero_grad_graph) "
                    "over the rotating sets"}


class _Grads:
    """One backward graph for timed_launches: realize() realizes its gradients
    (one multi-output kernel with realize_all when grouped, else one kernel per
    gradient); release() clears the graph's stored gradients
    (zero_grad_graph), which autograd's reference cycles otherwise keep alive
    with every buffer they hold."""

    def __init__(self, loss, tensors, grouped):
        self.loss, self.tensors, self.grouped = loss, tensors, grouped

    def realize(self):
        from ormi_amd import realize_all

        if self.grouped:
            realize_all(*self.tensors)
        else:
            for t in self.tensors:
                t.realize()

    def release(self):
        self.loss.zero_grad_graph()


def bench_c4(ev: Events, n: int) -> dict:
    from ormi_amd import Tensor

    log("C4: GEMMs")
    rng = np.random.default_rng(3)
    a = rng.normal(0, 1 / 64, (4096, 4096)).astype(np.float32)
    b = rng.normal(0, 1 / 64, (4096, 4096)).astype(np.float32)
    A, B = Tensor(a, "hip", dtype="bfloat16"), Tensor(b, "hip", dtype="bfloat16")
    (A @ B).realize()
    ms = timed_launches(ev, lambda i: A @ B, n)
    flops = 2 * 4096 ** 3
    out = {"bf16_4096": {"us": round(ms * 1e3, 2), "TFLOP/s": round(flops / ms / 1e9, 1),
                         "frac_mfma": round(flops / ms / 1e9 / BF16_PEAK_TFLOPS, 4)}}
    a32 = rng.normal(0, 1 / 64, (2048, 1024)).astype(np.float32)
    b32 = rng.normal(0, 1 / 64, (1024, 4096)).astype(np.float32)
    dc = rng.normal(0, 1, (2048, 4096)).astype(np.float32)
    A32, B32, DC = Tensor(a32, "hip"), Tensor(b32, "hip"), Tensor(dc, "hip")
    f32 = 2 * 2048 * 1024 * 4096
    for name, make in (("fp32_fwd_NN", lambda i: A32 @ B32),
                       ("fp32_dA_NT", lambda i: DC @ B32.transpose()),
                       ("fp32_dB_TN", lambda i: A32.transpose() @ DC)):
        make(0).realize()
        ms = timed_launches(ev, make, n)
        out[name] = {"us": round(ms * 1e3, 2), "TFLOP/s": round(f32 / ms / 1e9, 1),
                     "frac_mfma": round(f32 / ms / 1e9 / FP32_PEAK_TFLOPS, 4)}
    return out


class _GemmDesc(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int), ("M", ctypes.c_int), ("N", ctypes.c_int), ("K", ctypes.c_int),
                ("a", ctypes.c_void_p), ("a_stride_m", ctypes.c_int64), ("a_stride_k", ctypes.c_int64),
                ("b", ctypes.c_void_p), ("b_stride_k", ctypes.c_int64), ("b_stride_n", ctypes.c_int64),
                ("c", ctypes.c_void_p), ("batch_ndim", ctypes.c_int), ("batch_shape", ctypes.c_int * 4),
                ("a_batch_stride", ctypes.c_int64 * 4), ("b_batch_stride", ctypes.c_int64 * 4)]


def vendor_gemm(out_md: Path, cmd: str, rounds: int = 3, n: int = 20) -> None:
    """The C4 and C5 GEMM shapes through ormi_hip_gemm and through torch.matmul
    (hipBLASLt) on the same device buffers, in one process, alternating per
    shape; each side timed with HIP events over n back-to-back launches, best
    of `rounds`. Writes a markdown summary to out_md."""
    import torch

    ev = Events()
    lib = ev.lib
    lib.ormi_hip_gemm.argtypes = [ctypes.POINTER(_GemmDesc)]
    lib.ormi_hip_last_error.restype = ctypes.c_char_p
    assert lib.ormi_hip_init(0) == 0

    def t_torch(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(n):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / n * 1e3

    def t_ours(g):
        for _ in range(3):
            assert lib.ormi_hip_gemm(ctypes.byref(g)) == 0, lib.ormi_hip_last_error()
        ev.sync()
        e0, e1 = ev.new(), ev.new()
        ev.record(e0)
        for _ in range(n):
            lib.ormi_hip_gemm(ctypes.byref(g))
        ev.record(e1)
        ev.sync()
        return ev.elapsed_ms(e0, e1) / n * 1e3

    gen = torch.Generator(device="cuda")
    gen.manual_seed(3)
    cases = []
    for name, M, N, K, ta, tb, bf16 in [("C4 fp32 forward NN", 2048, 4096, 1024, False, False, False),
                                        ("C4 fp32 dA = dC B^T (NT)", 2048, 1024, 4096, False, True, False),
                                        ("C4 fp32 dB = A^T dC (TN)", 1024, 4096, 2048, True, False, False),
                                        ("C5 fp32 H1 W2 (NN)", 1024, 4096, 4096, False, False, False),
                                        ("C5 fp32 dW2 = H1^T dH2 (TN)", 4096, 4096, 1024, True, False, False),
                                        ("C5 fp32 dH1 = dH2 W2^T (NT)", 1024, 4096, 4096, False, True, False),
                                        ("C4 bf16 4096^3 (NN), fp32 out", 4096, 4096, 4096, False, False, True),
                                        ("bf16 4096^3 NT, fp32 out", 4096, 4096, 4096, False, True, True),
                                        ("bf16 4096^3 TN, fp32 out", 4096, 4096, 4096, True, False, True),
                                        ("bf16 8192^3 NN, fp32 out", 8192, 8192, 8192, False, False, True)]:
        dt = torch.bfloat16 if bf16 else torch.float32
        a_st = (torch.randn(K, M, device="cuda", generator=gen) / 64).to(dt) if ta else \
            (torch.randn(M, K, device="cuda", generator=gen) / 64).to(dt)
        b_st = (torch.randn(N, K, device="cuda", generator=gen) / 64).to(dt) if tb else \
            (torch.randn(K, N, device="cuda", generator=gen) / 64).to(dt)
        A = a_st.t() if ta else a_st
        B = b_st.t() if tb else b_st
        C = torch.empty(M, N, device="cuda")
        g = _GemmDesc(dtype=3 if bf16 else 0, M=M, N=N, K=K, a=a_st.data_ptr(), b=b_st.data_ptr(), c=C.data_ptr())
        g.a_stride_m, g.a_stride_k = (1, M) if ta else (K, 1)
        g.b_stride_k, g.b_stride_n = (1, K) if tb else (N, 1)
        fn = (lambda A=A, B=B: torch.mm(A, B, out_dtype=torch.float32)) if bf16 else (lambda A=A, B=B: A @ B)
        # hipBLASLt with a bf16 output (half the store) as a reference point.
        fn16 = (lambda A=A, B=B: torch.mm(A, B)) if bf16 else None
        cases.append((name, (fn, fn16), g, 2 * M * N * K, bf16, (a_st, b_st, C)))
    best = {}
    for _ in range(rounds):
        for name, (fn, fn16), g, fl, bf16, keep in cases:
            tt, to = t_torch(fn), t_ours(g)
            t16 = t_torch(fn16) if fn16 else math.inf
            b0 = best.get(name, (math.inf, math.inf, math.inf))
            best[name] = (min(b0[0], tt), min(b0[1], to), min(b0[2], t16))
    lines = ["# GEMM: ormi_hip_gemm against torch.matmul (hipBLASLt) on the same box", "",
             f"Command (from the repo root): `{cmd}`", "",
             f"torch {torch.__version__}; one process, the same device buffers, the two alternating per shape; "
             f"HIP events over {n} back-to-back launches, best of {rounds} rounds. Operands N(0, 1/64) "
             "(the C4 distribution); T = stored transposed (a view, as autograd passes it). The last column times "
             "hipBLASLt on the same bf16 product with a bf16 output, which stores half the bytes; the C4 config "
             "asks for an fp32 output.", "",
             "| GEMM | M x N x K | hipBLASLt us | TFLOP/s | ours us | TFLOP/s | ours / hipBLASLt time | "
             "hipBLASLt bf16-out us |",
             "|---|---|---|---|---|---|---|---|"]
    for name, fns, g, fl, bf16, keep in cases:
        tt, to, t16 = best[name]
        lines.append(f"| {name} | {g.M}x{g.N}x{g.K} | {tt:.1f} | {fl / tt / 1e6:.1f} | {to:.1f} | {fl / to / 1e6:.1f} | "
                     f"{to / tt:.3f} | {'—' if math.isinf(t16) else f'{t16:.1f}'} |")
    del cases
    # The C5 step both ways, alternating, each timed over sustained back-to-back
    # steps (the clock the GEMMs run at falls as the card heats under load).
    c5_steps = 20
    t_c5 = [], []
    for _ in range(rounds):
        t_c5[0].append(torch_c5_step_ms(torch, c5_steps))
        t_c5[1].append(bench_c5(ev, c5_steps)["step_ms"])
    lines += ["", f"C5 MLP training step (BASELINE config 5), {c5_steps} back-to-back steps after untimed ones, best of "
              f"{rounds} rounds, the two alternating: PyTorch (hipBLASLt GEMMs, torch autograd, erf GELU, one kernel "
              "per element-wise op) against this build's lazy graph (fused epilogues).", "",
              "| C5 step | PyTorch ms | ours ms | ours / PyTorch time |", "|---|---|---|---|",
              f"| 1024x(1024-4096-4096-1024) fp32 | {min(t_c5[0]):.3f} | {min(t_c5[1]):.3f} | "
              f"{min(t_c5[1]) / min(t_c5[0]):.3f} |"]
    out_md.write_text("\n".join(lines) + "\n")
    print(out_md.read_text())


# Register-only MFMA loops: the matrix cores' sustained rate with no memory
# work. Each wave keeps 4 independent accumulators and cycles through 8
# operand fragments loaded once from `vals` (vary = 0: all 8 hold the same
# values; 1: 8 different sets, so the operands change every instruction).
# Each lane stores one sum of its accumulators, so nothing is dead code.
MFMA_PROBE_SRC = r"""
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
extern "C" __global__ __launch_bounds__(256) void ormi_mfma_probe_bf16(float* out, const unsigned* vals, long long iters,
                                                                       long long vary) {
    const int lane = threadIdx.x & 63;
    u32x4 a[8], b[8];
    for (int s = 0; s < 8; ++s) {
        const int k = (vary ? s : 0) * 512 + lane * 4;
        a[s] = u32x4{vals[k], vals[k + 1], vals[k + 2], vals[k + 3]};
        b[s] = u32x4{vals[k + 256], vals[k + 257], vals[k + 258], vals[k + 259]};
    }
    f32x16 acc[4];
    for (int q = 0; q < 4; ++q) acc[q] = f32x16{};
    for (long long it = 0; it < iters; ++it) {
#pragma unroll
        for (int s = 0; s < 8; ++s)
            acc[s & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a[s]),
                                                                 __builtin_bit_cast(bf16x8, b[s]), acc[s & 3], 0, 0, 0);
    }
    float t = 0.0f;
    for (int q = 0; q < 4; ++q)
        for (int r = 0; r < 16; ++r) t += acc[q][r];
    out[blockIdx.x * blockDim.x + threadIdx.x] = t;
}
extern "C" __global__ __launch_bounds__(256) void ormi_mfma_probe_f32(float* out, const unsigned* vals, long long iters,
                                                                      long long vary) {
    const int lane = threadIdx.x & 63;
    float a[8], b[8];
    for (int s = 0; s < 8; ++s) {
        const int k = (vary ? s : 0) * 512 + lane;
        a[s] = __uint_as_float(vals[k]);
        b[s] = __uint_as_float(vals[k + 256]);
    }
    f32x16 acc[4];
    for (int q = 0; q < 4; ++q) acc[q] = f32x16{};
    for (long long it = 0; it < iters; ++it) {
#pragma unroll
        for (int s = 0; s < 8; ++s) acc[s & 3] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s], b[s], acc[s & 3], 0, 0, 0);
    }
    float t = 0.0f;
    for (int q = 0; q < 4; ++q)
        for (int r = 0; r < 16; ++r) t += acc[q][r];
    out[blockIdx.x * blockDim.x + threadIdx.x] = t;
}
"""


HBM_PROBE_SRC = r"""
typedef float f4 __attribute__((ext_vector_type(4)));
// Block b reads chunk b (ch float4), 4 loads per thread in flight.
extern "C" __global__ __launch_bounds__(256) void ormi_hbm_read_chunk(const f4* __restrict__ x, long long n4,
                                                                      long long ch, float* out) {
    float acc = 0.f;
    const long long base = (long long)blockIdx.x * ch;
    for (long long i = threadIdx.x; i < ch; i += 1024) {
        f4 v[4];
        for (int u = 0; u < 4; ++u) {
            const long long j = base + i + u * 256;
            v[u] = (i + u * 256 < ch && j < n4) ? x[j] : f4{0.f, 0.f, 0.f, 0.f};
        }
        for (int u = 0; u < 4; ++u) acc += v[u].x + v[u].y + v[u].z + v[u].w;
    }
    if (acc == 12345.678f) out[0] = acc;  // keeps the loads; never true for the zeroed input
}
// Grid stride, one load per thread per iteration.
extern "C" __global__ __launch_bounds__(256) void ormi_hbm_read_stride(const f4* __restrict__ x, long long n4,
                                                                       float* out) {
    float acc = 0.f;
    const long long n = (long long)gridDim.x * 256;
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n4; i += n) {
        const f4 v = x[i];
        acc += v.x + v.y + v.z + v.w;
    }
    if (acc == 12345.678f) out[0] = acc;
}
// The same with non-temporal loads.
extern "C" __global__ __launch_bounds__(256) void ormi_hbm_read_chunk_nt(const f4* __restrict__ x, long long n4,
                                                                         long long ch, float* out) {
    float acc = 0.f;
    const long long base = (long long)blockIdx.x * ch;
    for (long long i = threadIdx.x; i < ch; i += 1024) {
        f4 v[4];
        for (int u = 0; u < 4; ++u) {
            const long long j = base + i + u * 256;
            v[u] = (i + u * 256 < ch && j < n4) ? __builtin_nontemporal_load(x + j) : f4{0.f, 0.f, 0.f, 0.f};
        }
        for (int u = 0; u < 4; ++u) acc += v[u].x + v[u].y + v[u].z + v[u].w;
    }
    if (acc == 12345.678f) out[0] = acc;
}
// Grid stride copy with non-temporal stores (the element-wise kernels' stores).
extern "C" __global__ __launch_bounds__(256) void ormi_hbm_copy(f4* __restrict__ y, const f4* __restrict__ x,
                                                                long long n4) {
    const long long n = (long long)gridDim.x * 256;
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n4; i += n)
        __builtin_nontemporal_store(x[i], y + i);
}
// The same with non-temporal loads (the element-wise kernels' loads of large read-once operands).
extern "C" __global__ __launch_bounds__(256) void ormi_hbm_copy_nt(f4* __restrict__ y, const f4* __restrict__ x,
                                                                   long long n4) {
    const long long n = (long long)gridDim.x * 256;
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n4; i += n)
        __builtin_nontemporal_store(__builtin_nontemporal_load(x + i), y + i);
}
// Grid stride, non-temporal stores only.
extern "C" __global__ __launch_bounds__(256) void ormi_hbm_write(f4* __restrict__ y, long long n4) {
    const long long n = (long long)gridDim.x * 256;
    const f4 z = {1.f, 2.f, 3.f, 4.f};
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n4; i += n) __builtin_nontemporal_store(z, y + i);
}
// Grid stride, plain stores.
extern "C" __global__ __launch_bounds__(256) void ormi_hbm_write_plain(f4* __restrict__ y, long long n4) {
    const long long n = (long long)gridDim.x * 256;
    const f4 z = {1.f, 2.f, 3.f, 4.f};
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n4; i += n) y[i] = z;
}
"""


def hbm_ceiling(out_md: Path, cmd: str, rounds: int = 7, n: int = 10) -> None:
    """What HBM streams sustain on this card: plain read, copy and write kernels
    over memory the 256 MB Infinity Cache does not hold, compiled and launched
    through libormi_hip's hipRTC entry points, HIP events, median of `rounds`
    sets of n launches after 8 untimed. The ceilings C2 (a copy's traffic) and
    C3 (reads) are compared with. Writes a markdown table to out_md."""
    ev = Events()
    lib = ev.lib
    lib.ormi_hip_last_error.restype = ctypes.c_char_p
    lib.ormi_hip_rtc_compile.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p), ctypes.c_int,
                                         ctypes.POINTER(ctypes.c_uint64)]
    lib.ormi_hip_launch.argtypes = [ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_uint32),
                                    ctypes.c_uint32, ctypes.POINTER(ctypes.c_void_p)]
    lib.ormi_hip_malloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
    lib.ormi_hip_free.argtypes = [ctypes.c_void_p]
    lib.ormi_hip_memset_d32.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_size_t]
    assert lib.ormi_hip_init(0) == 0
    props = _Props()
    assert lib.ormi_hip_get_props(ctypes.byref(props)) == 0
    cus = props.compute_units
    # One 2 GiB buffer in eight 256 MiB slices; launches rotate over four slice
    # sets, so each touches memory last used 1.5 GiB of traffic earlier (the
    # Infinity Cache holds none of it).
    slice_b = 256 << 20
    base = ctypes.c_void_p()
    assert lib.ormi_hip_malloc(ctypes.byref(base), 8 * slice_b) == 0, lib.ormi_hip_last_error()
    assert lib.ormi_hip_memset_d32(base, 0, 8 * slice_b // 4) == 0
    out = ctypes.c_void_p()
    assert lib.ormi_hip_malloc(ctypes.byref(out), 4) == 0

    def at(k):
        return ctypes.c_void_p(base.value + k * slice_b)

    handles = {}
    for name in ("ormi_hbm_read_chunk", "ormi_hbm_read_chunk_nt", "ormi_hbm_read_stride", "ormi_hbm_copy",
                 "ormi_hbm_copy_nt", "ormi_hbm_write", "ormi_hbm_write_plain"):
        h = ctypes.c_uint64()
        if lib.ormi_hip_rtc_compile(HBM_PROBE_SRC.encode(), name.encode(), None, 0, ctypes.byref(h)) != 0:
            raise SystemExit("hbm probe: " + lib.ormi_hip_last_error().decode())
        handles[name] = h.value
    n4_two, n4_one = 2 * slice_b // 16, slice_b // 16
    chunk = 8192 // 16  # 8 KB per block: the row reductions' segment
    keep = []

    def argv(*vals):
        cs = [v if isinstance(v, ctypes.c_void_p) else ctypes.c_longlong(v) for v in vals]
        keep.append(cs)
        return (ctypes.c_void_p * len(cs))(*[ctypes.addressof(c) for c in cs])

    # (label, kernel, grid, one argument set per rotation step, bytes per launch)
    cases = [
        ("read 512 MiB, 8 KB per work-group, 4 loads in flight per thread", "ormi_hbm_read_chunk", n4_two // chunk,
         [argv(at(2 * r), n4_two, chunk, out) for r in range(4)], 2 * slice_b),
        ("the same, non-temporal loads", "ormi_hbm_read_chunk_nt", n4_two // chunk,
         [argv(at(2 * r), n4_two, chunk, out) for r in range(4)], 2 * slice_b),
        (f"read 512 MiB, grid stride over {16 * cus} work-groups", "ormi_hbm_read_stride", 16 * cus,
         [argv(at(2 * r), n4_two, out) for r in range(4)], 2 * slice_b),
        (f"copy 256 MiB to 256 MiB, non-temporal stores, {64 * cus} work-groups", "ormi_hbm_copy", 64 * cus,
         [argv(at(4 + r), at(r), n4_one) for r in range(4)], 2 * slice_b),
        ("the same, non-temporal loads too", "ormi_hbm_copy_nt", 64 * cus,
         [argv(at(4 + r), at(r), n4_one) for r in range(4)], 2 * slice_b),
        (f"write 512 MiB, non-temporal stores, {64 * cus} work-groups", "ormi_hbm_write", 64 * cus,
         [argv(at(2 * r), n4_two) for r in range(4)], 2 * slice_b),
        ("the same, plain stores", "ormi_hbm_write_plain", 64 * cus,
         [argv(at(2 * r), n4_two) for r in range(4)], 2 * slice_b),
    ]

    # The same kernels with at most w work-groups per CU: a launch-time LDS
    # reservation they do not touch (160 KB per CU; as the element-wise and
    # row-reduction kernels are launched).
    def capped(w):
        return (160 * 1024 // w - 1024) // 512 * 512

    for w in (5, 3):
        cases.append((f"non-temporal read, 8 KB per work-group, at most {w} per CU", "ormi_hbm_read_chunk_nt",
                      n4_two // chunk, cases[1][3], 2 * slice_b, capped(w)))
        cases.append((f"non-temporal copy, at most {w} work-groups per CU", "ormi_hbm_copy_nt", 64 * cus,
                      cases[4][3], 2 * slice_b, capped(w)))
    rows = []
    for case in cases:
        label, kname, grid_x, arg_sets, nbytes = case[:5]
        lds = case[5] if len(case) > 5 else 0
        grid = (ctypes.c_uint32 * 3)(grid_x, 1, 1)
        block = (ctypes.c_uint32 * 3)(256, 1, 1)
        for i in range(8):
            assert lib.ormi_hip_launch(handles[kname], grid, block, lds, arg_sets[i % 4]) == 0, lib.ormi_hip_last_error()
        ev.sync()
        times = []
        for _ in range(rounds):
            e0, e1 = ev.new(), ev.new()
            ev.record(e0)
            for i in range(n):
                lib.ormi_hip_launch(handles[kname], grid, block, lds, arg_sets[i % 4])
            ev.record(e1)
            ev.sync()
            times.append(ev.elapsed_ms(e0, e1) / n)
        t = sorted(times)[rounds // 2]
        tbs = nbytes / (t * 1e-3) / 1e12
        rows.append(f"| {label} | {nbytes / 2**20:.0f} | {t * 1e3:.1f} | {tbs:.2f} | {tbs / (HBM_PEAK_GBS / 1000):.1%} |")
        log(rows[-1])
    bufs = [base]
    for p in bufs + [out]:
        lib.ormi_hip_free(p)
    lines = ["# HBM stream ceilings (plain read, copy and write kernels)", "", f"Command (from the repo root): `{cmd}`", "",
             "Kernels (`HBM_PROBE_SRC` in bench.py) compiled and launched through libormi_hip's hipRTC entry points, "
             "128-bit accesses, 512 MiB moved per launch, launches rotating over four slice sets of one 2 GiB buffer "
             "(each launch touches memory last used 1.5 GiB of traffic earlier, so the 256 MB Infinity Cache serves "
             f"none of it), HIP events, median of {rounds} sets of {n} launches after 8 untimed. These are what the "
             "card's HBM streams sustain with plain kernels; the element-wise and reduction kernels are measured "
             "against them.", "",
             "| kernel | MiB moved | us | TB/s | of 8 TB/s |", "|---|---|---|---|---|"] + rows
    out_md.write_text("\n".join(lines) + "\n")
    print(out_md.read_text())


def mfma_probe_values(seed: int = 7) -> np.ndarray:
    """8 x 512 operand words, each two bf16 of N(0, 1/64) values (the statistics
    of the C4 inputs); read as fp32, a word is about its upper value."""
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 1 / 64, 2 * 8 * 512).astype(np.float32)
    bf = (x.view(np.uint32) >> 16).astype(np.uint32)
    return (bf[0::2] | (bf[1::2] << 16)).astype(np.uint32)


class _Props(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 64), ("compute_units", ctypes.c_int), ("clock_khz", ctypes.c_int),
                ("lds_bytes_per_block", ctypes.c_int), ("total_mem_bytes", ctypes.c_size_t)]


def mfma_ceiling(out_md: Path, cmd: str) -> None:
    """Sustained matrix-core rate of v_mfma_f32_32x32x16_bf16 and
    v_mfma_f32_32x32x2_f32 in register-only loops (one and two 4-wave blocks
    per compute unit; constant and changing operands), compiled and launched
    through libormi_hip's hipRTC entry points; best of 3 launches after a warm-up.
    Writes a markdown table to out_md."""
    ev = Events()
    lib = ev.lib
    lib.ormi_hip_last_error.restype = ctypes.c_char_p
    lib.ormi_hip_rtc_compile.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p), ctypes.c_int,
                                         ctypes.POINTER(ctypes.c_uint64)]
    lib.ormi_hip_launch.argtypes = [ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_uint32),
                                    ctypes.c_uint32, ctypes.POINTER(ctypes.c_void_p)]
    lib.ormi_hip_malloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
    lib.ormi_hip_memcpy_h2d.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]
    assert lib.ormi_hip_init(0) == 0
    props = _Props()
    assert lib.ormi_hip_get_props(ctypes.byref(props)) == 0
    cus = props.compute_units
    vals = mfma_probe_values()
    dv, dout = ctypes.c_void_p(), ctypes.c_void_p()
    assert lib.ormi_hip_malloc(ctypes.byref(dv), vals.nbytes) == 0
    assert lib.ormi_hip_memcpy_h2d(dv, vals.ctypes.data, vals.nbytes) == 0
    assert lib.ormi_hip_malloc(ctypes.byref(dout), 2 * cus * 256 * 4) == 0
    rows = []
    for name, inst, flops_per, iters in (("ormi_mfma_probe_bf16", "`v_mfma_f32_32x32x16_bf16`", 32 * 32 * 16 * 2, 60000),
                                         ("ormi_mfma_probe_f32", "`v_mfma_f32_32x32x2_f32`", 32 * 32 * 2 * 2, 45000)):
        h = ctypes.c_uint64()
        if lib.ormi_hip_rtc_compile(MFMA_PROBE_SRC.encode(), name.encode(), None, 0, ctypes.byref(h)) != 0:
            raise SystemExit("mfma probe: " + lib.ormi_hip_last_error().decode())
        for bpc in (1, 2):
            for vary in (0, 1):
                grid = (ctypes.c_uint32 * 3)(cus * bpc, 1, 1)
                block = (ctypes.c_uint32 * 3)(256, 1, 1)
                a_out, a_vals = ctypes.c_void_p(dout.value), ctypes.c_void_p(dv.value)
                a_it, a_vary = ctypes.c_longlong(iters * bpc), ctypes.c_longlong(vary)
                argv = (ctypes.c_void_p * 4)(ctypes.addressof(a_out), ctypes.addressof(a_vals), ctypes.addressof(a_it),
                                             ctypes.addressof(a_vary))
                assert lib.ormi_hip_launch(h.value, grid, block, 0, argv) == 0, lib.ormi_hip_last_error()
                ev.sync()
                best = 1e9
                for _ in range(3):
                    e0, e1 = ev.new(), ev.new()
                    ev.record(e0)
                    assert lib.ormi_hip_launch(h.value, grid, block, 0, argv) == 0
                    ev.record(e1)
                    ev.sync()
                    best = min(best, ev.elapsed_ms(e0, e1))
                waves = cus * bpc * 4
                tf = waves * iters * bpc * 8 * flops_per / (best * 1e-3) / 1e12
                peak = BF16_PEAK_TFLOPS if "bf16" in name else FP32_PEAK_TFLOPS
                rows.append(f"| {inst} | {'random N(0,1/64)' if vary else 'constant'} | {bpc} | {best:.3f} | "
                            f"{tf:.1f} | {100 * tf / peak:.1f}% |")
                log(rows[-1])
    lines = ["# Matrix-core ceilings (register-only MFMA loops)", "", f"Command (from the repo root): `{cmd}`", "",
             "4 independent accumulators per wave, 4 waves per 256-thread block, one or two blocks per compute unit "
             "(1 or 2 waves per SIMD); the kernel (`MFMA_PROBE_SRC` in bench.py) is compiled and launched through "
             "libormi_hip's hipRTC entry points and timed with HIP events, best of 3 launches after one untimed. "
             "Operands are loaded once into 8 fragment registers and cycled: either all 8 hold the same N(0, 1/64) "
             "values (constant) or 8 different sets (random, changing every instruction).", "",
             "| instruction | operands | waves/SIMD | ms | TFLOP/s | of datasheet dense peak |",
             "|---|---|---|---|---|---|"] + rows
    out_md.write_text("\n".join(lines) + "\n")
    print(out_md.read_text())


def gemm_k_sweep(out_md: Path, cmd: str, rounds: int = 3, n: int = 10) -> None:
    """Time of the fp32 GEMM against K at the C5 output shapes (1024x4096: one
    128x128 tile per compute unit; 4096x4096: four), per epilogue, through
    ormi_hip_gemm_ex. Every (K, epilogue) pair is timed in each of `rounds`
    interleaved rounds (the clock depends on what ran before) with HIP events
    over n launches; the best is kept. A line through K = 1024 and 4096 splits
    each time into a fixed part per launch (launch, first loads, epilogue
    stores, tail) and a part per 1024 of K (the main loop)."""
    ev = Events()
    lib = ev.lib

    class Epi(ctypes.Structure):
        _fields_ = [("kind", ctypes.c_int), ("fn", ctypes.c_int), ("form", ctypes.c_int), ("s", ctypes.c_void_p),
                    ("d", ctypes.c_void_p), ("d_stride_m", ctypes.c_int64), ("d_stride_n", ctypes.c_int64),
                    ("d_batch_stride", ctypes.c_int64 * 4), ("aux", ctypes.c_void_p)]

    lib.ormi_hip_malloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
    lib.ormi_hip_memcpy_h2d.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]
    lib.ormi_hip_free.argtypes = [ctypes.c_void_p]
    lib.ormi_hip_gemm_ex.argtypes = [ctypes.POINTER(_GemmDesc), ctypes.POINTER(Epi)]
    lib.ormi_hip_last_error.restype = ctypes.c_char_p
    rng = np.random.default_rng(0)
    held = []

    def put(a):
        p = ctypes.c_void_p()
        assert lib.ormi_hip_malloc(ctypes.byref(p), a.nbytes) == 0, lib.ormi_hip_last_error()
        assert lib.ormi_hip_memcpy_h2d(p, a.ctypes.data, a.nbytes) == 0, lib.ormi_hip_last_error()
        held.append(p)
        return p

    kmax, ks = 4096, (256, 1024, 4096)
    lines = ["# fp32 GEMM: time against K, fixed cost per launch", "", f"Command (from the repo root): `{cmd}`", "",
             f"NN layout, direct-load kernel (the default configuration), N(0, 1/64) operands. Best of {rounds} "
             f"interleaved rounds of {n} launches (HIP events). fixed = the line through K = 1024 and K = 4096 "
             "at K = 0; per 1024 K = its slope, against 2·M·N·1024 flop at 157.3 TFLOP/s. Epilogues: none; GELU "
             "storing the product too (the forward layers); the SGD update reading and writing D (the weight "
             "gradients).", "",
             "| M x N | epilogue | " + " | ".join(f"K {k} us" for k in ks) + " | fixed us | per 1024 K us | loop vs peak |",
             "|---|---|" + "---|" * (len(ks) + 3)]
    for M, N in ((1024, 4096), (4096, 4096)):
        A = put((rng.standard_normal((M, kmax)) / 64).astype(np.float32))
        B = put((rng.standard_normal((kmax, N)) / 64).astype(np.float32))
        C = put(np.zeros((M, N), np.float32))
        X = put(np.zeros((M, N), np.float32))
        D = put(np.ones((M, N), np.float32))
        S = put(np.array([1e-3], np.float32))
        epis = {"none": None, "GELU + product": Epi(kind=2, fn=7, form=0, aux=X),
                "SGD (D - p s)": Epi(kind=1, fn=0, form=1, s=S, d=D, d_stride_m=N, d_stride_n=1)}
        best = collections.defaultdict(lambda: math.inf)
        for r in range(rounds):
            for K in ks:
                order = list(epis.items()) if r % 2 == 0 else list(epis.items())[::-1]
                for name, e in order:
                    g = _GemmDesc(dtype=0, M=M, N=N, K=K, a=A, a_stride_m=kmax, a_stride_k=1, b=B, b_stride_k=N,
                                  b_stride_n=1, c=C)
                    ep = ctypes.byref(e) if e is not None else None
                    for _ in range(2):
                        assert lib.ormi_hip_gemm_ex(ctypes.byref(g), ep) == 0, lib.ormi_hip_last_error()
                    ev.sync()
                    e0, e1 = ev.new(), ev.new()
                    ev.record(e0)
                    for _ in range(n):
                        lib.ormi_hip_gemm_ex(ctypes.byref(g), ep)
                    ev.record(e1)
                    best[(K, name)] = min(best[(K, name)], ev.elapsed_ms(e0, e1) / n * 1e3)
        for name in epis:
            t1, t4 = best[(1024, name)], best[(4096, name)]
            slope = (t4 - t1) / 3.0
            fixed = t1 - slope
            ideal = 2.0 * M * N * 1024 / (FP32_PEAK_TFLOPS * 1e6)
            lines.append(f"| {M}x{N} | {name} | " + " | ".join(f"{best[(k, name)]:.1f}" for k in ks)
                         + f" | {fixed:.1f} | {slope:.1f} | {ideal / slope:.1%} |")
        for p in held:
            lib.ormi_hip_free(p)
        held.clear()
    out_md.write_text("\n".join(lines) + "\n")
    print(out_md.read_text())


def gemm_pair_sweep(out_md: Path, cmd: str, rounds: int = 5, n: int = 20) -> None:
    """Grouped against separate launches of a layer's backward products
    through ormi_hip_gemm_pair: dX = dZ W^T (both operands k-contiguous, the
    activation derivative gelu' in the store) and dW = X^T dZ (both
    mn-contiguous, the SGD update in place), at the C5 layer shapes over a range
    of depths and at C5's own layer-2 pair. ORMI_GEMM_PAIR=0 runs them as two
    launches, =2 as one whatever the depth; the default (1) groups pairs of at
    most 64 k-tiles per work-group. Best of `rounds` interleaved rounds of n
    calls (HIP events)."""
    ev = Events()
    lib = ev.lib

    class Epi(ctypes.Structure):
        _fields_ = [("kind", ctypes.c_int), ("fn", ctypes.c_int), ("form", ctypes.c_int), ("s", ctypes.c_void_p),
                    ("d", ctypes.c_void_p), ("d_stride_m", ctypes.c_int64), ("d_stride_n", ctypes.c_int64),
                    ("d_batch_stride", ctypes.c_int64 * 4), ("aux", ctypes.c_void_p)]

    lib.ormi_hip_malloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
    lib.ormi_hip_memcpy_h2d.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]
    lib.ormi_hip_free.argtypes = [ctypes.c_void_p]
    lib.ormi_hip_gemm_pair.argtypes = [ctypes.POINTER(_GemmDesc), ctypes.POINTER(Epi), ctypes.POINTER(_GemmDesc),
                                       ctypes.POINTER(Epi), ctypes.POINTER(ctypes.c_int)]
    lib.ormi_hip_last_error.restype = ctypes.c_char_p
    props = _Props()
    assert lib.ormi_hip_init(0) == 0 and lib.ormi_hip_get_props(ctypes.byref(props)) == 0
    cus = props.compute_units
    rng = np.random.default_rng(0)
    held = []

    def put(a):
        p = ctypes.c_void_p()
        assert lib.ormi_hip_malloc(ctypes.byref(p), max(a.nbytes, 4)) == 0, lib.ormi_hip_last_error()
        assert lib.ormi_hip_memcpy_h2d(p, a.ctypes.data, a.nbytes) == 0, lib.ormi_hip_last_error()
        held.append(p)
        return p

    def rand(*shape):
        return (rng.standard_normal(shape) / 8).astype(np.float32)

    scale = put(np.array([1e-3], np.float32))

    def dx(M, N, K):
        g = _GemmDesc(dtype=0, M=M, N=N, K=K, a=put(rand(M, K)), a_stride_m=K, a_stride_k=1, b=put(rand(N, K)),
                      b_stride_k=1, b_stride_n=K, c=put(np.zeros((M, N), np.float32)))
        return g, Epi(kind=3, fn=8, d=put(rand(M, N)), d_stride_m=N, d_stride_n=1)

    def dw(M, N, K):
        c = put(rand(M, N))
        g = _GemmDesc(dtype=0, M=M, N=N, K=K, a=put(rand(K, M)), a_stride_m=1, a_stride_k=M, b=put(rand(K, N)),
                      b_stride_k=N, b_stride_n=1, c=c)
        return g, Epi(kind=1, form=1, s=scale, d=c, d_stride_m=N, d_stride_n=1)

    cases = [(f"1024x4096 + 4096x1024, K {k}", (1024, 4096, k), (4096, 1024, k)) for k in (64, 128, 256, 512, 1024)]
    cases += [("1024x4096 + 4096x4096, K 256", (1024, 4096, 256), (4096, 4096, 256)),
              ("C5 layer 2: 1024x4096 K 4096 + 4096x4096 K 1024", (1024, 4096, 4096), (4096, 4096, 1024))]
    built = [(name, dx(*x), dw(*w), x, w) for name, x, w in cases]
    best = collections.defaultdict(lambda: math.inf)
    grouped_by = {}
    saved = os.environ.get("ORMI_GEMM_PAIR")
    try:
        for r in range(rounds):
            for name, (g0, e0), (g1, e1), _, _ in built:
                for mode in (("0", "2", "1") if r % 2 == 0 else ("1", "2", "0")):
                    os.environ["ORMI_GEMM_PAIR"] = mode
                    flag = ctypes.c_int()
                    args = (ctypes.byref(g0), ctypes.byref(e0), ctypes.byref(g1), ctypes.byref(e1), ctypes.byref(flag))
                    for _ in range(2):
                        assert lib.ormi_hip_gemm_pair(*args) == 0, lib.ormi_hip_last_error()
                    grouped_by[(name, mode)] = flag.value
                    ev.sync()
                    t0, t1 = ev.new(), ev.new()
                    ev.record(t0)
                    for _ in range(n):
                        lib.ormi_hip_gemm_pair(*args)
                    ev.record(t1)
                    best[(name, mode)] = min(best[(name, mode)], ev.elapsed_ms(t0, t1) / n * 1e3)
    finally:
        if saved is None:
            os.environ.pop("ORMI_GEMM_PAIR", None)
        else:
            os.environ["ORMI_GEMM_PAIR"] = saved
    # Stream length alone: one launch over twice the tiles (two column halves of
    # one product, so twice the tiles per work-group) against a launch per half.
    lib.ormi_hip_gemm_ex.argtypes = [ctypes.POINTER(_GemmDesc), ctypes.POINTER(Epi)]
    halves = []
    for name, form, M, N, K in (("X^T dZ (mn-contiguous), 4096 x 8192, K 1024", "dw", 4096, 8192, 1024),
                                ("dZ W^T (k-contiguous), 2048 x 4096, K 4096", "dx", 2048, 4096, 4096)):
        if form == "dw":  # halves split N: B and C columns
            A, B, C = put(rand(K, M)), put(rand(K, N)), put(np.zeros((M, N), np.float32))
            whole = _GemmDesc(dtype=0, M=M, N=N, K=K, a=A, a_stride_m=1, a_stride_k=M, b=B, b_stride_k=N, b_stride_n=1, c=C)
            parts = [_GemmDesc(dtype=0, M=M, N=N // 2, K=K, a=A, a_stride_m=1, a_stride_k=M,
                               b=ctypes.c_void_p(B.value + h * (N // 2) * 4), b_stride_k=N, b_stride_n=1,
                               c=put(np.zeros((M, N // 2), np.float32))) for h in (0, 1)]
        else:  # halves split M: A rows and C rows
            A, B, C = put(rand(M, K)), put(rand(N, K)), put(np.zeros((M, N), np.float32))
            whole = _GemmDesc(dtype=0, M=M, N=N, K=K, a=A, a_stride_m=K, a_stride_k=1, b=B, b_stride_k=1, b_stride_n=K, c=C)
            parts = [_GemmDesc(dtype=0, M=M // 2, N=N, K=K, a=ctypes.c_void_p(A.value + h * (M // 2) * K * 4),
                               a_stride_m=K, a_stride_k=1, b=B, b_stride_k=1, b_stride_n=K,
                               c=ctypes.c_void_p(C.value + h * (M // 2) * N * 4)) for h in (0, 1)]
        halves.append((name, whole, parts, (M // 128) * (N // 128), K // 32))
    hbest = collections.defaultdict(lambda: math.inf)
    for r in range(rounds):
        for name, whole, parts, _, _ in halves:
            for which in (("one", "two") if r % 2 == 0 else ("two", "one")):
                calls = [whole] if which == "one" else parts
                for g in calls:
                    assert lib.ormi_hip_gemm_ex(ctypes.byref(g), None) == 0, lib.ormi_hip_last_error()
                ev.sync()
                t0, t1 = ev.new(), ev.new()
                ev.record(t0)
                for _ in range(n):
                    for g in calls:
                        lib.ormi_hip_gemm_ex(ctypes.byref(g), None)
                ev.record(t1)
                hbest[(name, which)] = min(hbest[(name, which)], ev.elapsed_ms(t0, t1) / n * 1e3)
    lines = ["# Grouped GEMM pairs: one launch against two, by depth", "", f"Command (from the repo root): `{cmd}`", "",
             "ormi_hip_gemm_pair on dX = dZ W^T (k-contiguous operands, gelu' in the store) and dW = X^T dZ "
             "(mn-contiguous operands, SGD update in place), fp32. k-tiles/wg: the 32-deep k-tiles each of the "
             f"{cus} work-groups streams when grouped. two = ORMI_GEMM_PAIR=0, one = 2, default = 1 (grouped only "
             f"up to 64 k-tiles per work-group). Best of {rounds} interleaved rounds of {n} calls, HIP events.", "",
             "| products | k-tiles/wg | two launches us | one launch us | one vs two | default us (grouped) |",
             "|---|---|---|---|---|---|"]
    for name, _, _, x, w in built:
        tiles = (x[0] // 128) * (x[1] // 128) * (x[2] // 32) + (w[0] // 128) * (w[1] // 128) * (w[2] // 32)
        groups = min(cus, (x[0] // 128) * (x[1] // 128) + (w[0] // 128) * (w[1] // 128))
        two, one, dflt = best[(name, "0")], best[(name, "2")], best[(name, "1")]
        lines.append(f"| {name} | {-(-tiles // groups)} | {two:.1f} | {one:.1f} | {one / two - 1:+.1%} | "
                     f"{dflt:.1f} ({'yes' if grouped_by[(name, '1')] else 'no'}) |")
        log(lines[-1])
    lines += ["", "Stream length alone, no epilogue, through ormi_hip_gemm_ex: one product over 2T whole tiles in one "
              "launch (the persistent kernel, 2T / 256 tiles per work-group) against its two halves (T tiles each) in "
              "two launches. Same operands, same flops, same kernel code.", "",
              "| product | tiles | k-tiles per tile | one launch us | two launches us | one vs two |", "|---|---|---|---|---|---|"]
    for name, _, _, tiles, kt in halves:
        one, two = hbest[(name, "one")], hbest[(name, "two")]
        lines.append(f"| {name} | {tiles} | {kt} | {one:.1f} | {two:.1f} | {one / two - 1:+.1%} |")
        log(lines[-1])
    for p in held:
        lib.ormi_hip_free(p)
    out_md.write_text("\n".join(lines) + "\n")
    print(out_md.read_text())


def torch_c5_step_ms(torch, steps: int) -> float:
    """The C5 step written in PyTorch on the same inputs as bench_c5 (seed 4):
    fp32 matmuls (hipBLASLt), erf GELU, MSE, autograd, SGD lr 1e-3. For the
    vendor comparison only."""
    torch.backends.cuda.matmul.allow_tf32 = False
    F = torch.nn.functional
    rng = np.random.default_rng(4)
    dims = [1024, 4096, 4096, 1024]
    X = torch.from_numpy(rng.normal(0, 1, (1024, 1024)).astype(np.float32)).cuda()
    Y = torch.from_numpy(rng.normal(0, 1, (1024, 1024)).astype(np.float32)).cuda()
    ws = [torch.from_numpy(rng.uniform(-math.sqrt(6 / i), math.sqrt(6 / i), (i, o)).astype(np.float32)).cuda()
          .requires_grad_() for i, o in zip(dims, dims[1:])]

    def step(ws):
        h = X
        for i, w in enumerate(ws):
            h = h @ w
            if i < len(ws) - 1:
                h = F.gelu(h)
        d = h - Y
        loss = (d * d).sum() * (1.0 / (1024 * 1024))
        grads = torch.autograd.grad(loss, ws)
        with torch.no_grad():
            ws = [(w - g * 1e-3).requires_grad_() for w, g in zip(ws, grads)]
        return loss, ws

    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < WARM_MS:
        _, ws = step(ws)
        torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with gc_paused():
        a.record()
        for _ in range(steps):
            loss, ws = step(ws)
        b.record()
        torch.cuda.synchronize()
    return a.elapsed_time(b) / steps


def bench_c5(ev: Events, steps: int) -> dict:
    from ormi_amd import Tensor, realize_all
    from ormi_amd import ormi_backend as ob
    from ormi_amd.ormi_backend import Node

    log("C5: MLP step")
    rng = np.random.default_rng(4)
    dims = [1024, 4096, 4096, 1024]
    X = Tensor(rng.normal(0, 1, (1024, 1024)).astype(np.float32), "hip")
    Y = Tensor(rng.normal(0, 1, (1024, 1024)).astype(np.float32), "hip")
    W = [rng.uniform(-math.sqrt(6 / i), math.sqrt(6 / i), (i, o)).astype(np.float32) for i, o in zip(dims, dims[1:])]
    ws = [Tensor(w, "hip", requires_grad=True) for w in W]

    def step(ws):
        h = X
        for i, w in enumerate(ws):
            h = h @ w
            if i < len(ws) - 1:
                h = h.gelu()
        d = h - Y
        loss = (d * d).sum() * (1.0 / (1024 * 1024))
        loss.backward()
        # The SGD updates and the loss (the step reports it: the MSE reduction
        # is part of the timed work) realized together, so each layer's dX and
        # weight-gradient products can share one grouped GEMM launch.
        ups = [w - w.grad * 1e-3 for w in ws]
        realize_all(*ups, loss)
        # New leaves each step so graphs do not chain across steps.
        out = [Tensor(_node=Node(u._node.data, True, u._node.device), device="hip") for u in ups]
        # backward stored a gradient on every node and gradient graphs point at
        # forward nodes (reference csrc/core/autograd.cpp:24-47): clearing them
        # (zero_grad_graph, :49-58) lets the step's buffers return to the pool.
        loss.zero_grad_graph()
        return loss, out

    loss0, ws = step(ws)
    first = float(loss0.numpy())
    del loss0
    # Untimed steps (the pool holds a step's blocks after the second) for
    # WARM_MS of wall time.
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < WARM_MS:
        _, ws = step(ws)
        ev.sync()
    e0, e1 = ev.new(), ev.new()
    pairs0 = ob.gemm_pair_count()
    with gc_paused():
        ev.record(e0)
        t0 = time.perf_counter()
        for _ in range(steps):
            loss, ws = step(ws)
        ev.record(e1)
        ms = ev.elapsed_ms(e0, e1) / steps
        wall = (time.perf_counter() - t0) / steps
    pairs = (ob.gemm_pair_count() - pairs0) / steps
    last = float(loss.numpy())
    flops = 146028888064
    return {"step_ms": round(ms, 3), "wall_ms": round(wall * 1e3, 3), "gemm_TFLOP/s": round(flops / ms / 1e9, 1),
            "frac_fp32": round(flops / ms / 1e9 / FP32_PEAK_TFLOPS, 4), "grouped_gemm_launches": pairs,
            "loss_first": first, "loss_last": last}


def _pmc_rows(run_dir: Path, counter: str):
    """(kernel name, value) per dispatch from the rocprofv3 counter CSVs under run_dir."""
    rows = []
    for f in sorted(run_dir.rglob("*counter_collection.csv")):
        with open(f, newline="") as fh:
            for r in csv.DictReader(fh):
                if r.get("Counter_Name", "").strip() == counter:
                    rows.append((r.get("Kernel_Name", "").strip(), float(r.get("Counter_Value", "nan"))))
    return rows


def _pmc_kernel(run_dir: Path, counter: str):
    """Name, dispatch count and mean counter value of the most-dispatched ormi_ kernel."""
    by = collections.defaultdict(list)
    for name, v in _pmc_rows(run_dir, counter):
        if name.startswith("ormi_"):
            by[name].append(v)
    if not by:
        raise SystemExit(f"--pmc-report: no ormi_ kernel with counter {counter} under {run_dir}")
    name = max(by, key=lambda k: len(by[k]))
    return name, len(by[name]), sum(by[name]) / len(by[name])


def _pmc_by_kernel(run_dir: Path, counter: str):
    """{kernel name: (first dispatch id, [values])} for one counter of one run."""
    by = {}
    for f in sorted(run_dir.rglob("*counter_collection.csv")):
        with open(f, newline="") as fh:
            for r in csv.DictReader(fh):
                if r.get("Counter_Name", "").strip() != counter:
                    continue
                name = r.get("Kernel_Name", "").strip()
                did = int(r.get("Dispatch_Id", 0) or 0)
                first, vals = by.get(name, (did, []))
                vals.append(float(r.get("Counter_Value", "nan")))
                by[name] = (min(first, did), vals)
    return by


# Per workload label: the kernels of that run, in order of first dispatch, with
# their algorithmic (read, write) bytes per launch. A None entry is a kernel the
# report lists without an algorithmic figure of its own.
def _pmc_plan():
    rows, cols = 16384, 8192
    inb = rows * cols * 4
    return {
        "copy": [("copy y = -x", (2 ** 27, 2 ** 27))],
        "c2": [("C2 fused map", (c2_bytes() - 2 ** 27, 2 ** 27))],
        "c3": [("C3 row max", (inb, rows * 4)), ("C3 row sum(exp(x - max))", (inb + rows * 4, rows * 4)),
               ("C3 row mean (sum, its 2^-13 scale at the store)", (inb, rows * 4)),
               ("C3 row argmax", (inb, rows * 8)),
               ("C3 column sum, main", (inb, None)), ("C3 column sum, finish", (None, cols * 4))],
        "c4": [("C4 bf16 4096^3", (2 * 4096 * 4096 * 2, 4096 * 4096 * 4)),
               ("C4 fp32 NN 2048x1024x4096", ((2048 * 1024 + 1024 * 4096) * 4, 2048 * 4096 * 4)),
               ("C4 fp32 NT dA (128x64 tiles)", ((2048 * 4096 + 4096 * 1024) * 4, 2048 * 1024 * 4)),
               ("C4 fp32 TN dB", ((1024 * 2048 + 2048 * 4096) * 4, 1024 * 4096 * 4))],
    }


def pmc_report(pmc_dir: Path, out: Path, cmd: str) -> None:
    """Turn `rocprofv3 --pmc FETCH_SIZE` / `--pmc WRITE_SIZE` runs into bytes per
    launch. Runs live in pmc_dir/<label>_<COUNTER>/. Label "copy" is the
    calibration kernel (y = -x over 8192x4096 fp32: 128 MiB read, 128 MiB
    written), whose counters scale every other kernel's KiB figures to bytes; a
    run pmc_dir/copy_raw/ of TCC_EA0_RDREQ, TCC_EA0_RDREQ_32B and TCC_BUBBLE,
    when present, shows where the read factor comes from."""
    plan = _pmc_plan()
    got = {}
    for label in plan:
        f_dir, w_dir = pmc_dir / f"{label}_FETCH_SIZE", pmc_dir / f"{label}_WRITE_SIZE"
        if not f_dir.exists() or not w_dir.exists():
            continue
        fb, wb = _pmc_by_kernel(f_dir, "FETCH_SIZE"), _pmc_by_kernel(w_dir, "WRITE_SIZE")
        names = sorted((k for k in fb if k in wb and ("ormi_" in k or "gemm" in k)), key=lambda k: fb[k][0])
        got[label] = [(k, len(fb[k][1]), sum(fb[k][1]) / len(fb[k][1]), sum(wb[k][1]) / len(wb[k][1])) for k in names]
    copy = got["copy"][0]
    sf = plan["copy"][0][1][0] / (copy[2] * 1024)
    sw = plan["copy"][0][1][1] / (copy[3] * 1024)
    lines = [
        "# HBM traffic per launch (rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE, one run each)",
        "",
        f"Command: `{cmd}`",
        "",
        f"Scale factors from the copy kernel (y = -x, 8192x4096 fp32, 134217728 B read + 134217728 B written): "
        f"fetch {sf:.4f}, write {sw:.4f} (algorithmic bytes / (KiB x 1024)).",
    ]
    raw = pmc_dir / "copy_raw"
    if raw.exists():
        vals = {c: _pmc_by_kernel(raw, c) for c in ("TCC_EA0_RDREQ_sum", "TCC_EA0_RDREQ_32B_sum", "TCC_BUBBLE_sum")}
        k = copy[0]
        mean = {c: (sum(v[k][1]) / len(v[k][1]) if k in v else float("nan")) for c, v in vals.items()}
        rd, r32, bub = mean["TCC_EA0_RDREQ_sum"], mean["TCC_EA0_RDREQ_32B_sum"], mean["TCC_BUBBLE_sum"]
        lines += ["", f"Raw read requests of the copy kernel (L2 to fabric): TCC_EA0_RDREQ {rd:.0f}, of which 32-byte "
                  f"{r32:.0f}, TCC_BUBBLE (counted as 128-byte) {bub:.0f}; 134217728 B / RDREQ = "
                  f"{2 ** 27 / rd:.1f} bytes per request. FETCH_SIZE weighs a request that is neither 32-byte nor "
                  f"counted by TCC_BUBBLE as 64 bytes."]
    lines += ["", "| kernel | fetch KiB/dispatch | write KiB/dispatch | read bytes | write bytes | algorithmic read | "
              "algorithmic write | traffic / algorithmic | dispatches | name |",
              "|---|---|---|---|---|---|---|---|---|---|"]
    for label, rows in got.items():
        for i, (name, n, fk, wk) in enumerate(rows):
            desc, (ar, aw) = plan[label][i] if i < len(plan[label]) else (name, (None, None))
            rb, wbyt = int(round(fk * 1024 * sf)), int(round(wk * 1024 * sw))
            alg = (ar or 0) + (aw or 0)
            ratio = f"{(rb + wbyt) / alg:.3f}" if ar is not None and aw is not None else "—"
            lines.append(f"| {desc} | {fk:.1f} | {wk:.1f} | {rb} | {wbyt} | {ar if ar is not None else '—'} | "
                         f"{aw if aw is not None else '—'} | {ratio} | {n} | `{name[:60]}` |")
    lines += ["", "Fetch and write bytes count the L2's requests to the fabric, so they include reads the 256 MB "
              "Infinity Cache serves. A GEMM reads each operand panel once per XCD that needs it (8 L2s): the bf16 "
              "kernel's 4x8 tile group per XCD needs 8 MB of A and 16 MB of B, 192 MB over the chip against the "
              "64 MB of its operands, which stay resident in the Infinity Cache."]
    out.write_text("\n".join(lines) + "\n")
    print(out.read_text())


def trace_report(run_dir: Path, out: Path, title: str, cmd: str) -> None:
    """Per-kernel durations from a `rocprofv3 --kernel-trace` run (the
    *kernel_trace.csv under run_dir): calls, mean, median, min and max in
    microseconds, and the share of GPU time. The trace counts every dispatch of
    the run, warm-up launches included; the median is the steady-state figure."""
    by = collections.defaultdict(list)
    for f in sorted(run_dir.rglob("*kernel_trace.csv")):
        with open(f, newline="") as fh:
            for r in csv.DictReader(fh):
                by[r["Kernel_Name"].strip()].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    if not by:
        raise SystemExit(f"--trace-report: no kernel trace under {run_dir}")
    total = sum(sum(v) for v in by.values())
    lines = [f"# {title}", "", f"Command (from the repo root): `{cmd}`", "",
             "rocprofv3 kernel trace, durations in microseconds. Every dispatch of the run is counted, the untimed "
             "warm-up launches included; the median is the steady-state figure.", "",
             "| kernel | calls | mean us | median us | min us | max us | % of GPU time |", "|---|---|---|---|---|---|---|"]
    for name, v in sorted(by.items(), key=lambda kv: -sum(kv[1])):
        v = sorted(v)
        lines.append(f"| `{name[:110]}` | {len(v)} | {sum(v) / len(v):.2f} | {v[len(v) // 2]:.2f} | {v[0]:.2f} | "
                     f"{v[-1]:.2f} | {100 * sum(v) / total:.2f} |")
    out.write_text("\n".join(lines) + "\n")
    print(out.read_text())


def mfma_report(pmc_dir: Path, out: Path, cmd: str) -> None:
    """MFMA utilisation and shader clock per GEMM kernel from one `rocprofv3
    --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_MFMA SQ_LDS_BANK_CONFLICT
    GRBM_GUI_ACTIVE --kernel-trace` run: busy cycles summed over SIMDs / (SIMDs x
    the kernel's active cycles per XCC), the formula of rocprofv3's derived
    MfmaUtil; clock = active cycles per XCC / dispatch duration. Dispatches of
    one kernel are grouped by their MFMA count (one group per GEMM shape). SIMD
    and XCC counts come from the run's agent info."""
    agent = {}
    for f in sorted(pmc_dir.rglob("*agent_info.csv")):
        for r in csv.DictReader(open(f, newline="")):
            if r.get("Name", "").startswith("gfx"):
                agent = r
    simds, xcc = int(agent.get("Simd_Count", 1024)), int(agent.get("Num_Xcc", 8))
    disp = collections.defaultdict(dict)  # (name, dispatch) -> counters, duration
    for f in sorted(pmc_dir.rglob("*counter_collection.csv")):
        for r in csv.DictReader(open(f, newline="")):
            name = r.get("Kernel_Name", "").strip()
            if "gemm" not in name:
                continue
            d = disp[(name, r["Dispatch_Id"])]
            d[r["Counter_Name"].strip()] = float(r["Counter_Value"])
            if "End_Timestamp" in r:
                d["us"] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-3
    groups = collections.defaultdict(list)
    for (name, _), d in disp.items():
        if d.get("GRBM_GUI_ACTIVE") and "SQ_VALU_MFMA_BUSY_CYCLES" in d:
            groups[(name, d.get("SQ_INSTS_MFMA", 0.0))].append(d)
    lines = [
        "# GEMM MFMA utilisation and shader clock (rocprofv3 counters)", "",
        f"Command (from the repo root): `{cmd}`", "",
        f"Device: {agent.get('Name', '?')}, {simds} SIMDs, {xcc} XCCs, datasheet engine clock "
        f"{agent.get('Max_Engine_Clk_Fcompute', '?')} MHz. util = SQ_VALU_MFMA_BUSY_CYCLES / (SIMDs x "
        "GRBM_GUI_ACTIVE / XCCs), averaged over dispatches; clock = GRBM_GUI_ACTIVE / XCCs / duration. Counters "
        "serialize kernels, so these are the figures while the kernel runs. Dispatches are grouped by kernel and "
        "MFMA count (one row per GEMM shape); the clock range runs from the first dispatch to the last.", "",
        "| kernel | MFMA instructions / dispatch | dispatches | avg us | MFMA util | clock GHz (first - last, min) "
        "| LDS bank conflicts / dispatch |",
        "|---|---|---|---|---|---|---|",
    ]
    for (name, mf), ds in sorted(groups.items(), key=lambda kv: (kv[0][0], -kv[0][1])):
        if mf == 0:
            continue  # no matrix work (the split-K finish pass)
        util = sum(d["SQ_VALU_MFMA_BUSY_CYCLES"] / (simds * d["GRBM_GUI_ACTIVE"] / xcc) for d in ds) / len(ds)
        us = [d.get("us", float("nan")) for d in ds]
        clk = [d["GRBM_GUI_ACTIVE"] / xcc / (d["us"] * 1e3) for d in ds if d.get("us")]
        bc = sum(d.get("SQ_LDS_BANK_CONFLICT", 0.0) for d in ds) / len(ds)
        clk_s = f"{clk[0]:.2f} - {clk[-1]:.2f}, {min(clk):.2f}" if clk else "-"
        lines.append(f"| `{name[:110]}` | {mf:.4g} | {len(ds)} | {sum(us) / len(us):.1f} | {util * 100:.1f}% | "
                     f"{clk_s} | {bc:.4g} |")
    out.write_text("\n".join(lines) + "\n")
    print(out.read_text())


WAVE_COUNTERS = (
    "SQ_WAVE_CYCLES SQ_BUSY_CYCLES SQ_WAIT_ANY SQ_WAIT_INST_ANY SQ_WAIT_INST_LDS SQ_ACTIVE_INST_LDS "
    "SQ_ACTIVE_INST_ANY GRBM_GUI_ACTIVE",
    "SQ_LDS_IDX_ACTIVE SQ_LDS_DATA_FIFO_FULL SQ_LDS_CMD_FIFO_FULL SQ_LDS_ADDR_CONFLICT SQ_LDS_UNALIGNED_STALL "
    "SQ_INSTS_LDS SQ_ACTIVE_INST_VALU GRBM_GUI_ACTIVE",
)


def wave_report(pmc_dirs, out: Path, cmd: str) -> None:
    """Wave states, shader clock and LDS activity per GEMM kernel from the two
    rocprofv3 --pmc passes of WAVE_COUNTERS over `--only c4` (one run each).
    clock = GRBM_GUI_ACTIVE per XCC / kernel duration. SQ wave-cycle counters
    count 4-cycle units (SQ_WAVE_CYCLES x 4 matches waves x active cycles), so
    shares of SQ_WAVE_CYCLES are fractions of wave time and the LDS busy
    fraction is SQ_LDS_IDX_ACTIVE x 4 / (CUs x active cycles per XCC)."""
    agent = {}
    per = collections.defaultdict(lambda: collections.defaultdict(list))
    dur = collections.defaultdict(dict)
    for d in pmc_dirs:
        for f in sorted(Path(d).rglob("*agent_info.csv")):
            for r in csv.DictReader(open(f, newline="")):
                if r.get("Name", "").startswith("gfx"):
                    agent = r
        for f in sorted(Path(d).rglob("*counter_collection.csv")):
            for r in csv.DictReader(open(f, newline="")):
                name = r.get("Kernel_Name", "").strip()
                if "gemm" not in name:
                    continue
                per[name][r["Counter_Name"].strip()].append(float(r["Counter_Value"]))
                dur[name][(d, r["Dispatch_Id"])] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-3
    cus, xcc = int(agent.get("Cu_Count", 256)), int(agent.get("Num_Xcc", 8))

    def mean(cs, c):
        v = cs.get(c, [])
        return sum(v) / len(v) if v else float("nan")

    lines = [
        "# GEMM wave states, shader clock and LDS activity (rocprofv3 counters)", "",
        f"Command (from the repo root): `{cmd}`", "",
        f"Device: {agent.get('Name', '?')}, {cus} CUs, {xcc} XCCs, datasheet engine clock "
        f"{agent.get('Max_Engine_Clk_Fcompute', '?')} MHz. clock = GRBM_GUI_ACTIVE / XCCs / kernel duration. "
        "Shares are of SQ_WAVE_CYCLES (wave time): s_waitcnt = SQ_WAIT_ANY, waiting to issue = SQ_WAIT_INST_ANY. "
        "LDS busy = SQ_LDS_IDX_ACTIVE x 4 / (CUs x active cycles per XCC), taking the SQ counters' 4-cycle unit. "
        "Counters serialize kernels; the duration is that of the counted dispatches. Kernels under 20 us "
        "(the split-K finish pass) are left out: their GRBM count is mostly dispatch overhead.", "",
        "| kernel | dispatches (both passes) | avg us | clock GHz | s_waitcnt share | waiting-to-issue share | LDS instructions / dispatch "
        "| LDS busy | LDS FIFO-full (data / cmd) |",
        "|---|---|---|---|---|---|---|---|---|",
    ]
    for name, cs in sorted(per.items()):
        us = sum(dur[name].values()) / len(dur[name])
        if us < 20.0:
            continue  # a few-us kernel's GRBM count is mostly dispatch overhead
        cyc = mean(cs, "GRBM_GUI_ACTIVE") / xcc
        wc = mean(cs, "SQ_WAVE_CYCLES")
        lines.append(
            f"| `{name[:100]}` | {len(dur[name])} | {us:.1f} | {cyc / (us * 1e3):.2f} | {mean(cs, 'SQ_WAIT_ANY') / wc:.1%} "
            f"| {mean(cs, 'SQ_WAIT_INST_ANY') / wc:.1%} | {mean(cs, 'SQ_INSTS_LDS'):.4g} "
            f"| {mean(cs, 'SQ_LDS_IDX_ACTIVE') * 4 / (cus * cyc):.1%} "
            f"| {mean(cs, 'SQ_LDS_DATA_FIFO_FULL'):.4g} / {mean(cs, 'SQ_LDS_CMD_FIFO_FULL'):.4g} |")
    out.write_text("\n".join(lines) + "\n")
    print(out.read_text())


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-extra", action="store_true", help="only the headline workload")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", choices=["c1", "c3", "c4", "c5", "copy"],
                    help="run one non-headline workload and print its figures (profiling runs)")
    ap.add_argument("--pmc-report", nargs=2, metavar=("PMC_DIR", "OUT_MD"),
                    help="summarize rocprofv3 --pmc runs into a traffic table (no GPU needed)")
    ap.add_argument("--mfma-report", nargs=2, metavar=("PMC_DIR", "OUT_MD"),
                    help="summarize a rocprofv3 --pmc run of --only c4 into MFMA utilisation (no GPU needed)")
    ap.add_argument("--wave-report", nargs=3, metavar=("PMC_A", "PMC_B", "OUT_MD"),
                    help="summarize the two rocprofv3 --pmc passes of WAVE_COUNTERS over --only c4 (no GPU needed)")
    ap.add_argument("--gemm-k-sweep", metavar="OUT_MD",
                    help="fp32 GEMM time against K at the C5 output shapes: fixed cost per launch and loop rate")
    ap.add_argument("--trace-report", nargs=3, metavar=("RUN_DIR", "OUT_MD", "TITLE"),
                    help="summarize a rocprofv3 --kernel-trace run into per-kernel durations (no GPU needed); "
                         "--trace-cmd gives the command that made the run")
    ap.add_argument("--trace-cmd", default="", help="the rocprofv3 command recorded by --trace-report")
    ap.add_argument("--hbm-ceiling", metavar="OUT_MD",
                    help="plain read, copy and write kernels: what the card's HBM streams sustain (markdown)")
    ap.add_argument("--gemm-pairs", metavar="OUT_MD",
                    help="a layer's backward GEMM pair as one launch against two, by depth (markdown)")
    ap.add_argument("--mfma-ceiling", metavar="OUT_MD",
                    help="register-only MFMA loops: the matrix cores' sustained bf16 and fp32 rates (markdown)")
    ap.add_argument("--vendor-gemm", metavar="OUT_MD",
                    help="time the C4/C5 GEMM shapes against torch.matmul (hipBLASLt) and write a markdown summary")
    args = ap.parse_args()
    if args.trace_report:
        trace_report(Path(args.trace_report[0]), Path(args.trace_report[1]), args.trace_report[2], args.trace_cmd)
        return
    if args.gemm_k_sweep:
        gemm_k_sweep(Path(args.gemm_k_sweep), f"python3 bench.py --gemm-k-sweep {args.gemm_k_sweep}")
        return
    if args.vendor_gemm:
        vendor_gemm(Path(args.vendor_gemm), "python3 bench.py --vendor-gemm profiles/gemm_vs_hipblaslt.md")
        return
    if args.mfma_ceiling:
        mfma_ceiling(Path(args.mfma_ceiling), f"python3 bench.py --mfma-ceiling {args.mfma_ceiling}")
        return
    if args.hbm_ceiling:
        hbm_ceiling(Path(args.hbm_ceiling), f"python3 bench.py --hbm-ceiling {args.hbm_ceiling}")
        return
    if args.gemm_pairs:
        gemm_pair_sweep(Path(args.gemm_pairs), f"python3 bench.py --gemm-pairs {args.gemm_pairs}")
        return
    if args.mfma_report:
        only = args.only or "c4"
        out_md = Path(args.mfma_report[1])
        mfma_report(Path(args.mfma_report[0]), out_md,
                    "rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_MFMA SQ_LDS_BANK_CONFLICT GRBM_GUI_ACTIVE "
                    f"--kernel-trace -d {args.mfma_report[0]} -o run --output-format csv -- python3 bench.py "
                    f"--only {only} --steps {30 if only == 'c5' else 5} --warmup 1; python3 bench.py --only {only} "
                    f"--mfma-report {args.mfma_report[0]} {out_md.as_posix()}")
        return
    if args.wave_report:
        wave_report(args.wave_report[:2], Path(args.wave_report[2]),
                    " ; ".join(f"rocprofv3 --pmc {c} --kernel-trace -d {d} -o run --output-format csv "
                               "-- python3 bench.py --only c4 --steps 5 --warmup 1"
                               for d, c in zip(args.wave_report[:2], WAVE_COUNTERS))
                    + f" ; python3 bench.py --wave-report {' '.join(args.wave_report)}")
        return
    if args.pmc_report:
        pmc_report(Path(args.pmc_report[0]), Path(args.pmc_report[1]),
                   "for each (label, args) in (copy, --only copy), (c2, --no-extra --no-cpu), (c3, --only c3), "
                   "(c4, --only c4) and COUNTER in FETCH_SIZE, WRITE_SIZE: rocprofv3 --pmc COUNTER "
                   "-d <PMC_DIR>/<label>_COUNTER -o run --output-format csv -- python3 bench.py <args> --steps 5 "
                   "--warmup 1; and rocprofv3 --pmc TCC_EA0_RDREQ_sum TCC_EA0_RDREQ_32B_sum TCC_BUBBLE_sum "
                   "-d <PMC_DIR>/copy_raw ... -- python3 bench.py --only copy --steps 5 --warmup 1; then "
                   "python3 bench.py --pmc-report <PMC_DIR> profiles/hbm_traffic.md")
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "the multi-GPU sharding plan is a design note, not an implemented path.", file=sys.stderr)
        sys.exit(2)

    import ormi_amd

    if not ormi_amd.ormi_backend.hip_available():
        raise SystemExit("bench.py: HIP device unavailable (no GPU visible); refusing to report a number.")
    ev = Events()
    if args.only:
        n = max(10, min(args.steps, 30))
        res = {"copy": lambda: bench_copy(args, ev), "c1": lambda: bench_c1(ev, n), "c3": lambda: bench_c3(ev, n),
               "c4": lambda: bench_c4(ev, n), "c5": lambda: bench_c5(ev, max(10, min(args.steps, 30)))}[args.only]()
        print(json.dumps({"only": args.only, **res}), flush=True)
        return
    main_res = bench_c2(args, ev)
    props = _Props()
    assert ev.lib.ormi_hip_get_props(ctypes.byref(props)) == 0
    device = {"name": props.name.decode(errors="replace"), "compute_units": props.compute_units,
              "peak_clock_mhz": props.clock_khz // 1000, "hbm_bytes": props.total_mem_bytes}
    extra = {}
    if not args.no_extra:
        n = max(10, min(args.steps, 30))
        extra["copy_calibration_neg_8192x4096"] = bench_copy(args, ev)
        extra["C1_fused_pointwise_rowsum_1024"] = bench_c1(ev, n)
        extra["C3_reductions_16384x8192"] = bench_c3(ev, n)
        extra["C4_gemm"] = bench_c4(ev, n)
        extra["C5_mlp_step_ms"] = bench_c5(ev, max(10, min(args.steps, 30)))
    cpu = None if args.no_cpu else cpu_baseline_c2()
    if not args.no_cpu and not args.no_extra:
        log("CPU baselines of the other configs")
        extra["cpu_baselines"] = cpu_baselines_extra()
    line = {
        "metric": METRIC,
        "value": round(main_res["value"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(main_res["step_s"] * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (numpy default_rng seeds from BASELINE.json configs)",
        "config": {"workload": "C2 fused broadcast chain tanh((x+bias)*scale)*sigmoid(x)-0.1*x*x, "
                               "x (8192,4096) fp32, bias (4096,), scale (8192,1), seed 1",
                   "bytes_per_step": c2_bytes(), "parallelism": "single GPU"},
        "roofline": main_res["roofline"],
        "cpu_baseline": cpu,
        # Untimed: the process's first C2 realize, which compiles the fused
        # kernel through hipRTC before launching it.
        "first_realize_ms": round(main_res["first_realize_ms"], 1),
        "device": device,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
