#!/usr/bin/env python3
"""Benchmark of the silarray GPU hot path on one MI355X.

Headline (BASELINE.json metric): fp32 SGEMM TFLOP/s at M=N=K=8192 (the
compute-bound config) with the 1x4096x4096 GEMV GB/s beside it, each as a
fraction of the MI355X roofline.  A "step" is one 8192^3 SGEMM (C = A.B) on
uniform[-1,1] inputs already resident in HBM.  Every kernel runs through the
C ABI (libsilgpu.so); times come from HIP events recorded on the library's
stream around back-to-back launches, and the wall clock brackets the timed
steps with a device synchronisation on both sides.

The other rows of the workload (GEMV, small-batch SGEMM, linear_sigmoid, row
softmax / layer_norm / sum(axis=1), full sum/min/max/argmax, the 20-op affine
chain, the 2048^3 and 4096^3 SGEMMs, the reference's three conv2d layers)
are reported under "secondary" with their own roofline fractions, together
with whole sil::eval graphs run through the C++ front end (the encoder
block, the reference's transformer and MLP benchmarks, the affine chain at
the API level).  Bandwidth rows rotate >= 1 GiB of buffers so the 256 MiB
Infinity Cache cannot serve repeated reads.

cpu_baseline: cblas_sgemm from OpenBLAS (the x86 stand-in for the
reference's Accelerate call, include/cpu.h:239-264) on the headline 8192^3
workload, on the host cores of the same machine, for a sample of ~10 s.
Every secondary row of the cpu.h path (the SGEMM sweep including config 1's
1024^3, GEMV, the small-batch product, linear_sigmoid, the row ops, the
reductions and the affine chain) carries its own cpu_baseline: OpenBLAS for
the products, the oracle's single-threaded loops for the vDSP calls, each on
a stated sample of ~1 s.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "fp32 SGEMM TFLOPS (8192^3) + GEMV GB/s (1x4096x4096); % of roofline"
PEAK_FP32_MFMA_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0
SEED = 20261201
# Rows held to 75% of HBM bandwidth, in the order they close the JSON line.
GATED_ROWS = ("sgemm_32x768x4096", "linear_sigmoid_256x4096x4096", "affine_chain20_64M",
              "sum_axis1_4096x8192", "sum_64M", "min_64M", "max_64M", "argmax_64M",
              "layer_norm_4096x8192", "softmax_4096x8192", "gemv_1x4096x4096")
# Secondary workloads warm up for at least this long (the GPU leaves its idle
# clocks within ~0.1 s of sustained work; short kernels would otherwise be
# timed partly at idle clocks).
WARM_S = 0.2


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--only", default="", help="comma list of workloads (default: all)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--cpu-row-seconds", type=float, default=1.0,
                    help="sample length of each secondary row's CPU baseline")
    return ap.parse_args()


def log(msg: str) -> None:
    sys.stderr.write(f"[bench] {msg}\n")
    sys.stderr.flush()


class Timer:
    """HIP events on the library stream around `reps` launches of fn."""

    def __init__(self, nat):
        self.nat = nat
        self.e0 = nat.Event()
        self.e1 = nat.Event()

    def warm(self, fn, warmup: int, min_s: float = WARM_S) -> None:
        """At least `warmup` calls and at least `min_s` seconds of them, so the
        clocks have left their idle state before anything is timed."""
        i, t0 = 0, time.perf_counter()
        while i < warmup or time.perf_counter() - t0 < min_s:
            fn(i)
            i += 1
            if i % 16 == 0:
                self.nat.sync()
        self.nat.sync()

    def ms_per_launch(self, fn, reps: int, warmup: int = 2) -> float:
        """Mean time per launch over `reps` back-to-back launches.  One more
        untimed launch (fn(-1): the buffer before call 0 in the rotation) is
        queued ahead of the start event, so the event is taken when that
        launch ends and the host's time to issue the first timed launch
        does not count as device time."""
        self.warm(fn, warmup)
        fn(-1)
        self.e0.record()
        for i in range(reps):
            fn(i)
        self.e1.record()
        return self.e0.elapsed_ms(self.e1) / reps


def roofline(bound: str, achieved: float, traffic=None) -> dict:
    peak = PEAK_FP32_MFMA_TFLOPS if bound == "mfma" else PEAK_HBM_GBS
    return {"bound": bound, "achieved": round(achieved, 3), "peak": peak,
            "unit": "TFLOP/s" if bound == "mfma" else "GB/s",
            "frac": round(achieved / peak, 4), "traffic": traffic}


def load_traffic(name: str):
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE +
    WRITE_SIZE, copy-kernel calibrated), committed under profiles/."""
    p = ROOT / "profiles" / "traffic.json"
    if not p.exists():
        return None
    try:
        return json.loads(p.read_text()).get(name)
    except Exception:
        return None


def uniform(g, shape):
    return g.uniform(-1.0, 1.0, shape).astype(np.float32)


def normal(g, shape, std):
    return g.normal(0.0, std, shape).astype(np.float32)


# ---- workloads -------------------------------------------------------------------

def bench_sgemm(nat, S, steps, warmup, g, min_warm_s=0.0):
    """The headline passes min_warm_s=0: exactly `warmup` untimed steps."""
    A = nat.DeviceBuffer.from_array(uniform(g, (S, S)))
    B = nat.DeviceBuffer.from_array(uniform(g, (S, S)))
    C = nat.DeviceBuffer(S * S * 4)

    def step(_i):
        nat.sgemm(0, 0, S, S, S, A, S, 0, B, S, 0, C, S, 0)

    t = Timer(nat)
    t.warm(step, warmup, min_warm_s)
    t0 = time.perf_counter()
    t.e0.record()
    for i in range(steps):
        step(i)
    t.e1.record()
    nat.sync()
    wall = time.perf_counter() - t0
    kern_ms = t.e0.elapsed_ms(t.e1) / steps
    flops = 2.0 * S * S * S
    return {"wall_ms_per_step": wall * 1e3 / steps, "kernel_ms": kern_ms,
            "tflops_wall": flops / (wall / steps) / 1e12, "tflops_kernel": flops / (kern_ms / 1e3) / 1e12}


def bench_gemv(nat, g, reps=200, hot=True):
    """GEMV 1x4096 . 4096x4096 over 16 rotated copies of B (1 GiB, so the
    256 MiB Infinity Cache cannot serve it); beside it the same-bytes read
    floor: the library's one-launch sum over the same rotated matrices (one
    read of 64 MiB and a 4-byte result); then, with hot=True, one B kept hot."""
    K = N = 4096
    copies = 16  # 16 x 64 MiB = 1 GiB in rotation
    x = nat.DeviceBuffer.from_array(normal(g, K, 0.02))
    B0 = normal(g, (K, N), 0.02)
    Bs = [nat.DeviceBuffer.from_array(B0) for _ in range(copies)]
    y = nat.DeviceBuffer(N * 4)
    s = nat.DeviceBuffer(4)
    t = Timer(nat)
    ms = t.ms_per_launch(lambda i: nat.sgemv(x, Bs[i % copies], N, y, N, K), reps, warmup=copies)
    ms_read = t.ms_per_launch(lambda i: nat.sum_f32(Bs[i % copies], K * N, s), reps,
                              warmup=copies)
    nbytes = 4 * (K + K * N + N)
    r = {"gbs": nbytes / (ms / 1e3) / 1e9, "us": ms * 1e3, "bytes": nbytes,
         "read_gbs": 4.0 * K * N / (ms_read / 1e3) / 1e9, "read_us": ms_read * 1e3}
    if hot:
        ms_hot = t.ms_per_launch(lambda i: nat.sgemv(x, Bs[0], N, y, N, K), reps)
        r["gbs_hot"] = nbytes / (ms_hot / 1e3) / 1e9
    return r


def bench_small_batch(nat, g, reps=200):
    M, N, K = 32, 768, 4096
    copies = 64
    A = nat.DeviceBuffer.from_array(normal(g, (M, K), 0.02))
    B0 = normal(g, (K, N), 0.02)
    Bs = [nat.DeviceBuffer.from_array(B0) for _ in range(copies)]
    C = nat.DeviceBuffer(M * N * 4)
    t = Timer(nat)
    ms = t.ms_per_launch(lambda i: nat.sgemm(0, 0, M, N, K, A, K, 0, Bs[i % copies], N, 0, C, N, 0),
                         reps, warmup=copies)
    ms_hot = t.ms_per_launch(lambda i: nat.sgemm(0, 0, M, N, K, A, K, 0, Bs[0], N, 0, C, N, 0), reps)
    nbytes = 4 * (M * K + K * N + M * N)
    return {"gbs": nbytes / (ms / 1e3) / 1e9, "gbs_hot": nbytes / (ms_hot / 1e3) / 1e9,
            "us": ms * 1e3,
            "tflops": 2 * M * N * K / (ms / 1e3) / 1e12, "bytes": nbytes}


def bench_linear_sigmoid(nat, g, reps=50):
    M, N, K = 256, 4096, 4096
    X = nat.DeviceBuffer.from_array(normal(g, (M, K), 0.02))
    W = nat.DeviceBuffer.from_array(normal(g, (K, N), 0.02))
    b = nat.DeviceBuffer.from_array(normal(g, N, 0.02))
    Y = nat.DeviceBuffer(M * N * 4)
    t = Timer(nat)
    ms = t.ms_per_launch(lambda i: nat.sgemm(0, 0, M, N, K, X, K, 0, W, N, 0, Y, N, 0, 1, b, N,
                                             nat.EPI_BIAS_SIGMOID), reps)
    return {"tflops": 2.0 * M * N * K / (ms / 1e3) / 1e12, "us": ms * 1e3}


# The reference's conv2d benchmark layers (bench/micro/bench_nn_ops.cpp:193-195)
# with its published sil-gpu times on the M1 Pro (bench/README.md:131-133).
CONV_LAYERS = [("imagenet_first", 1, 224, 224, 3, 3, 32, 0.564),
               ("resnet_mid", 16, 56, 56, 64, 3, 128, 2.89),
               ("resnet_deep", 16, 28, 28, 128, 3, 256, 2.93)]


def bench_conv2d(nat, g, reps=50, layers=None):
    """Implicit-GEMM conv2d (stride 1, same padding) on the reference's
    layers (all, or the names in `layers`); flops = 2 N H W C_out K K C_in."""
    out = {}
    for name, N, H, W, Ci, K, Co, ref_ms in CONV_LAYERS:
        if layers and name not in layers:
            continue
        x = nat.DeviceBuffer.from_array(uniform(g, (N, H, W, Ci)))
        w = nat.DeviceBuffer.from_array(uniform(g, (Co, K, K, Ci)))
        y = nat.DeviceBuffer(N * H * W * Co * 4)
        t = Timer(nat)
        ms = t.ms_per_launch(lambda i: nat.conv2d(x, w, y, N, H, W, Ci, K, Co), reps)
        flops = 2.0 * N * H * W * Co * K * K * Ci
        nbytes = 4.0 * (N * H * W * Ci + Co * K * K * Ci + N * H * W * Co)
        out[f"conv2d_{name}_{N}x{Ci}x{H}x{W}_k{K}_co{Co}"] = {
            "tflops": flops / (ms / 1e3) / 1e12, "gbs": nbytes / (ms / 1e3) / 1e9,
            "hbm_bound": flops / nbytes < PEAK_FP32_MFMA_TFLOPS / PEAK_HBM_GBS * 1e3,
            "us": ms * 1e3, "ref_ms": ref_ms, "traffic_key": f"conv2d_{name}"}
    return out


def bench_rowops(nat, g, reps=100):
    R, Cc = 4096, 8192
    pairs = 4  # 4 x (128 MiB in + 128 MiB out) = 1 GiB in rotation
    x0 = normal(g, (R, Cc), 3.0)
    xs = [nat.DeviceBuffer.from_array(x0) for _ in range(pairs)]
    ys = [nat.DeviceBuffer(R * Cc * 4) for _ in range(pairs)]
    gamma = nat.DeviceBuffer.from_array(np.ones(Cc, np.float32))
    beta = nat.DeviceBuffer.from_array(np.zeros(Cc, np.float32))
    t = Timer(nat)
    out = {}
    # Rotated (gated) and hot (one pair, partly served by the 256 MiB
    # Infinity Cache) rates.
    ops = {
        "softmax": (lambda i, j: nat.softmax_rows_f32(xs[j], ys[j], R, Cc), 8 * R * Cc),
        "layer_norm": (lambda i, j: nat.layer_norm_rows_f32(xs[j], ys[j], gamma, beta, R, Cc, 1e-5),
                       8 * R * Cc + 8 * Cc),
        "sum_axis1": (lambda i, j: nat.sum_axis_f32(xs[j], R, Cc, 1, ys[j]), 4 * R * Cc + 4 * R),
    }
    for name, (fn, nb) in ops.items():
        ms = t.ms_per_launch(lambda i: fn(i, i % pairs), reps, pairs)
        ms_hot = t.ms_per_launch(lambda i: fn(i, 0), reps)
        out[name] = {"gbs": nb / (ms / 1e3) / 1e9, "gbs_hot": nb / (ms_hot / 1e3) / 1e9,
                     "us": ms * 1e3, "bytes": nb}
    # The ceiling beside them: a device copy of the same 128 MiB input into the
    # same output buffers through silgpu_memcpy_d2d, which runs this library's
    # streaming copy kernel (copy16_k) on 16-byte-aligned ranges; same rotation.
    nb = 8 * R * Cc
    ms = t.ms_per_launch(lambda i: nat.call("silgpu_memcpy_d2d", nat.vp(ys[i % pairs]),
                                            nat.vp(xs[i % pairs]), 4 * R * Cc), reps, pairs)
    copy_gbs = nb / (ms / 1e3) / 1e9
    for name in ("softmax", "layer_norm"):
        out[name]["copy_gbs"] = copy_gbs
        out[name]["of_copy"] = out[name]["gbs"] / copy_gbs
    return out


def bench_reductions(nat, g, reps=100):
    n = 64 * 1024 * 1024
    copies = 4  # 4 x 256 MiB
    x0 = uniform(g, n)
    x0[(n * 7) // 9 + 1] = 2.0  # unique planted maximum, not 4- or chunk-aligned
    xs = [nat.DeviceBuffer.from_array(x0) for _ in range(copies)]
    o = nat.DeviceBuffer(4096)
    t = Timer(nat)
    out = {}
    ops = [("sum", lambda x: nat.sum_f32(x, n, o)), ("min", lambda x: nat.min_f32(x, n, o)),
           ("max", lambda x: nat.max_f32(x, n, o)),
           ("argmax", lambda x: nat.argmax_rows_f32(x, 1, n, o))]
    for name, fn in ops:
        ms = t.ms_per_launch(lambda i: fn(xs[i % copies]), reps, copies)
        ms_hot = t.ms_per_launch(lambda i: fn(xs[0]), reps)
        out[name] = {"gbs": 4 * n / (ms / 1e3) / 1e9, "gbs_hot": 4 * n / (ms_hot / 1e3) / 1e9,
                     "us": ms * 1e3, "bytes": 4 * n}
    nat.sync()
    idx = int(o.download(1, np.int32)[0])
    out["argmax"]["index_ok"] = idx == (n * 7) // 9 + 1
    return out


def bench_affine_chain(nat, g, reps=100):
    n = 64 * 1024 * 1024
    copies = 2  # 2 x (256 MiB in + 256 MiB out)
    x0 = uniform(g, n)
    xs = [nat.DeviceBuffer.from_array(x0) for _ in range(copies)]
    ys = [nat.DeviceBuffer(4 * n) for _ in range(copies)]
    sc = g.uniform(0.9, 1.1, 20).astype(np.float32)
    of = g.uniform(-0.1, 0.1, 20).astype(np.float32)
    progs = []
    for k in range(copies):
        instrs = [(nat.PI_LOAD, 0, 0, 0, 0.0, 0.0)] + [(nat.PI_FMAI, 0, 0, 0, float(a), float(b))
                                                       for a, b in zip(sc, of)]
        progs.append(nat.make_program((n,), [(xs[k], (1,))], instrs))
    t = Timer(nat)
    ms = t.ms_per_launch(lambda i: nat.program_f32(progs[i % copies], ys[i % copies]), reps, copies)
    return {"gbs": 8 * n / (ms / 1e3) / 1e9, "us": ms * 1e3, "bytes": 8 * n, "ops": 20}


def bench_copy(nat, g, reps=100):
    """Plain device copy of 256 MiB (hipMemcpyAsync D2D), the calibration
    kernel for the FETCH_SIZE / WRITE_SIZE counters: it reads and writes
    exactly 268,435,456 bytes per launch."""
    n = 64 * 1024 * 1024
    src = nat.DeviceBuffer.from_array(uniform(g, n))
    dst = nat.DeviceBuffer(4 * n)
    t = Timer(nat)
    ms = t.ms_per_launch(lambda i: nat.call("silgpu_memcpy_d2d", nat.vp(dst), nat.vp(src), 4 * n),
                         reps)
    return {"gbs": 8 * n / (ms / 1e3) / 1e9, "us": ms * 1e3, "bytes": 8 * n}


GRAPH_BENCH = ROOT / "silarray_amd" / "bench" / "bench_graph"
# The reference's published sil-gpu times for its single-head transformer
# block on an Apple M1 Pro (bench/README.md:196-199), keyed by (seq, d_model).
REF_TRANSFORMER_MS = {(256, 512): 1.53, (256, 768): 2.30, (256, 1024): 2.93, (512, 1024): 5.32}
# The reference's training step on an M1 Pro (bench/README.md:187-188), by batch.
REF_TRAIN_MS = {64: 1.11, 128: 1.51}
# The reference's MNIST benchmarks on the M1 Pro, sil-gpu column
# (bench/README.md:205-220): ms.
REF_MNIST_MS = {"classifier_train_epoch_ms": 283.83, "classifier_inference_ms": 0.920,
                "autoencoder_train_epoch_ms": 1080.0, "autoencoder_inference_ms": 8.65}
# The reference's GPU micro-benchmarks on the M1 Pro, sil-gpu column
# (bench/README.md:96-153): us per iteration (the op, its eval and the wait).
REF_MICRO_US = {
    "broadcast (1024x1024)+(1024)": 327, "broadcast (4096x512)+(512)": 412,
    "broadcast (4096x4096)+(4096)": 1050,
    "add (1000000)": 317, "add (10000000)": 967, "mul (1000000)": 316, "mul (10000000)": 993,
    "div (1000000)": 319, "div (10000000)": 1050, "pow (1000000)": 324, "pow (10000000)": 981,
    "softmax (256x512)": 246, "softmax (1024x1024)": 307, "softmax (4096x2048)": 763,
    "softmax (256x8192)": 458, "layer_norm (256x512)": 235, "layer_norm (1024x1024)": 277,
    "layer_norm (4096x2048)": 611, "bmm attention (8h, seq=128, d=64)": 228,
    "bmm attention (8h, seq=512, d=64)": 301, "bmm attention (16h, seq=256, d=128)": 292,
    "sum (1000000)": 230, "sum (10000000)": 445, "sum axis=0 (1024x256)": 213,
    "sum axis=0 (4096x256)": 231, "min (1000000)": 229, "min (10000000)": 455,
    "max (1000000)": 229, "max (10000000)": 443, "argmax (1024x256)": 240,
    "argmax (4096x256)": 333}


def bench_graphs(timeout: float = 300.0) -> list[dict]:
    """Whole sil::eval graphs through the C++ front end (bench_graph): the
    B4 S512 d768 H12 encoder block, the reference's single-head transformer
    and linear_sigmoid MLP benchmarks, and the 20-op affine chain at the API
    level, host <-> HBM copies of a 256 MiB array through its pinned host
    mirror, the reference's MNIST classifier and autoencoder benchmarks and
    its GPU micro-benchmarks at their shapes.  Each iteration is eval +
    synchronize, as the reference times it."""
    import subprocess

    if not GRAPH_BENCH.exists():
        raise RuntimeError(f"{GRAPH_BENCH} is not built (run __graft_entry__.build())")
    out = []
    for argv in (["encoder", "10"], ["transformer"], ["mlp"], ["train"],
                 ["chain", str(64 << 20), "20"], ["transfer", str(64 << 20), "10"], ["mnist"],
                 ["micro"]):
        log(f"bench_graph {' '.join(argv)}")
        proc = subprocess.run([str(GRAPH_BENCH), *argv], capture_output=True, text=True,
                              timeout=timeout)
        if proc.returncode != 0:
            raise RuntimeError(f"bench_graph {argv} failed ({proc.returncode}): {proc.stderr}")
        out += [json.loads(l) for l in proc.stdout.splitlines() if l.startswith("{")]
    return out


def cpu_baseline(seconds: float) -> dict:
    """cblas_sgemm (OpenBLAS) on the headline workload, 8192^3 fp32 NN, on this
    host's cores (at most 16 threads): one untimed call, then whole calls
    until at least `seconds` have elapsed (a bounded sample of the GPU's
    workload, the reference's CPU path include/cpu.h:239-264)."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import openblas  # test-infrastructure baseline, oracle/openblas.py

    try:
        cores = len(os.sched_getaffinity(0))
    except Exception:
        cores = os.cpu_count() or 1
    cores = max(1, min(cores, 16))
    openblas.set_threads(cores)
    S = 8192
    g = np.random.default_rng(SEED)
    A = uniform(g, (S, S))
    B = uniform(g, (S, S))
    Cm = np.empty((S, S), np.float32)
    openblas.sgemm(A, B, Cm)  # warmup
    runs = 0
    t0 = time.perf_counter()
    while True:
        openblas.sgemm(A, B, Cm)
        runs += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    tflops = 2.0 * S ** 3 * runs / el / 1e12
    del A, B, Cm
    # One thread, as a per-core figure: 2048^3 (8192^3 takes ~20 s per call
    # on one core), whole calls for about 3 s.
    openblas.set_threads(1)
    S1 = 2048
    A1, B1 = uniform(g, (S1, S1)), uniform(g, (S1, S1))
    C1 = np.empty((S1, S1), np.float32)
    openblas.sgemm(A1, B1, C1)
    runs1, t1 = 0, time.perf_counter()
    while True:
        openblas.sgemm(A1, B1, C1)
        runs1 += 1
        el1 = time.perf_counter() - t1
        if el1 >= 3.0:
            break
    openblas.set_threads(cores)
    return {"value": round(tflops, 4), "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": f"cblas_sgemm (OpenBLAS, {Path(openblas.LIB_PATH).name}) {S}^3 fp32 "
                      f"row-major NN, uniform[-1,1], {runs} whole calls in {el:.1f} s after one "
                      f"untimed call, {cores} threads",
            "host": host_cpu_info(),
            "one_thread": {"value": round(2.0 * S1 ** 3 * runs1 / el1 / 1e12, 4),
                           "unit": "TFLOP/s", "cores": 1,
                           "sample": f"{S1}^3, {runs1} whole calls in {el1:.1f} s"}}


def _cpu_rate(fn, units_per_call: float, seconds: float):
    """One untimed call, then whole calls until `seconds` have elapsed;
    returns (units per second, calls, elapsed s)."""
    fn()
    runs, t0 = 0, time.perf_counter()
    while True:
        fn()
        runs += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            return units_per_call * runs / el, runs, el


def cpu_rows(seconds: float) -> dict:
    """The reference's cpu.h path restated on this host for each secondary
    workload, keyed like the `secondary` rows: cblas_sgemm (OpenBLAS, the
    x86 stand-in for Accelerate, include/cpu.h:239-264) on up to 16 threads
    for the products, and the oracle's single-threaded loops (oracle.c built
    -O3 for the widest x86-64 level this host runs, no contraction) for the
    vDSP calls and the host loops: softmax
    with the row-minimum shift (include/array.h:2140-2149), two-pass
    layer_norm (include/cpu.h:352-373), sum over axis 1 in float
    (include/array.h:2309-2314), sequential sum, min, max, the argmax loop
    (include/array.h:1728-1745) and the affine chain node by node (one pass
    over the array per lazy node, include/array.h:1996-2015).  Each is
    timed on a bounded sample of the GPU row's workload (stated per row) for
    about `seconds`, in the GPU row's unit."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import openblas  # test-infrastructure baseline, oracle/openblas.py
    import cpubase  # oracle/cpubase.py: oracle.c built -O3 for this host's x86-64 level

    oracle, level = cpubase.load()
    loops = f"-O3 x86-64-{level}"
    try:
        cores = len(os.sched_getaffinity(0))
    except Exception:
        cores = os.cpu_count() or 1
    cores = max(1, min(cores, 16))
    g = np.random.default_rng(SEED + 1)
    out = {}

    def row(key, rate, unit, ncores, sample, runs, el):
        out[key] = {"value": round(rate, 4 if unit == "TFLOP/s" else 2), "unit": unit,
                    "cores": ncores, "kind": "port",
                    "sample": f"{sample}; {runs} whole calls in {el:.2f} s after one untimed call"}

    openblas.set_threads(cores)
    blas = f"cblas_sgemm (OpenBLAS, {Path(openblas.LIB_PATH).name}), {cores} threads"
    for S in (1024, 2048, 4096):
        A, B = uniform(g, (S, S)), uniform(g, (S, S))
        Cm = np.empty((S, S), np.float32)
        r, n, el = _cpu_rate(lambda: openblas.sgemm(A, B, Cm), 2.0 * S ** 3 / 1e12, seconds)
        row(f"sgemm_{S}", r, "TFLOP/s", cores, f"{blas}, {S}^3 NN uniform[-1,1] (the full workload)",
            n, el)
    K = N = 4096
    x = normal(g, (1, K), 0.02)
    Bm = normal(g, (K, N), 0.02)
    y = np.empty((1, N), np.float32)
    nbytes = 4.0 * (K + K * N + N)
    r, n, el = _cpu_rate(lambda: openblas.sgemm(x, Bm, y), nbytes / 1e9, seconds)
    row("gemv_1x4096x4096", r, "GB/s", cores, f"{blas}, M=1 (the full workload)", n, el)
    r1, n1, el1 = _cpu_rate(lambda: oracle.gemv_f32(x[0], Bm), nbytes / 1e9, seconds)
    out["gemv_1x4096x4096"]["scalar_loop_one_thread"] = {
        "value": round(r1, 2), "unit": "GB/s", "cores": 1,
        "sample": f"oracle_gemv_f32 scalar loop ({loops}), full workload, {n1} calls in "
                  f"{el1:.2f} s"}
    M, N, K = 32, 768, 4096
    A, Bm = normal(g, (M, K), 0.02), normal(g, (K, N), 0.02)
    Cm = np.empty((M, N), np.float32)
    r, n, el = _cpu_rate(lambda: openblas.sgemm(A, Bm, Cm), 4.0 * (M * K + K * N + M * N) / 1e9,
                         seconds)
    row("sgemm_32x768x4096", r, "GB/s", cores, f"{blas}, the full workload", n, el)
    M, N, K = 256, 4096, 4096
    X, W, bias = normal(g, (M, K), 0.02), normal(g, (K, N), 0.02), normal(g, N, 0.02)
    Y = np.empty((M, N), np.float32)

    def lin_sig():
        openblas.sgemm(X, W, Y)
        oracle.bias_sigmoid(Y, bias)

    r, n, el = _cpu_rate(lin_sig, 2.0 * M * N * K / 1e12, seconds)
    row("linear_sigmoid_256x4096x4096", r, "TFLOP/s", cores,
        f"{blas} + oracle_bias_sigmoid loop ({loops}, one thread), the full workload", n, el)
    R, Cc = 256, 8192  # 256 of the 4096 rows of the [4096, 8192] workload
    xr = normal(g, (R, Cc), 3.0)
    ones, zeros = np.ones(Cc, np.float32), np.zeros(Cc, np.float32)
    sub = f"{R} of the 4096 rows of [4096, 8192] N(0, 3), one thread, {loops}"
    r, n, el = _cpu_rate(lambda: oracle.softmax_rows_ref(xr), 8.0 * R * Cc / 1e9, seconds)
    row("softmax_4096x8192", r, "GB/s", 1, f"oracle_softmax_rows_ref, {sub}", n, el)
    r, n, el = _cpu_rate(lambda: oracle.layer_norm_ref(xr, ones, zeros),
                         (8.0 * R * Cc + 8 * Cc) / 1e9, seconds)
    row("layer_norm_4096x8192", r, "GB/s", 1, f"oracle_layer_norm_ref, {sub}", n, el)
    r, n, el = _cpu_rate(lambda: oracle.sum_axis_ref(xr, 1), (4.0 * R * Cc + 4 * R) / 1e9,
                         seconds)
    row("sum_axis1_4096x8192", r, "GB/s", 1, f"oracle_sum_axis_ref, {sub}", n, el)
    n64 = 16 * 1024 * 1024  # a quarter of the 64M-element workload
    v = uniform(g, n64)
    v[(n64 * 7) // 9 + 1] = 2.0
    sub = f"16M of the 64M uniform[-1,1] elements, one thread, {loops}"
    for key, fn, nm in (("sum_64M", lambda: oracle.sum_ref(v), "oracle_sum_ref"),
                        ("min_64M", lambda: oracle.fmin(v), "oracle_min"),
                        ("max_64M", lambda: oracle.fmax(v), "oracle_max"),
                        ("argmax_64M", lambda: oracle.argmax_rows_cpu_ref(v.reshape(1, -1)),
                         "oracle_argmax_rows_cpu_ref")):
        r, n, el = _cpu_rate(fn, 4.0 * n64 / 1e9, seconds)
        row(key, r, "GB/s", 1, f"{nm}, {sub}", n, el)
    sc = g.uniform(0.9, 1.1, 20).astype(np.float32)
    of = g.uniform(-0.1, 0.1, 20).astype(np.float32)
    # The reference's CPU evaluation of the lazy chain x*a_1+b_1 ... x*a_20+b_20:
    # every node is evaluated in topological order, and each mul / add node
    # whose input is already evaluated folds to one affine pass over the array
    # (include/array.h:1888-1940, 1996-2015: cpu::affine for >= 5M elements), so
    # the chain costs 40 passes.  The rate is in the GPU row's unit: one read and
    # one write of the array per chain.
    bufs = (np.empty_like(v), np.empty_like(v))

    def chain_per_node():
        src = v
        for i in range(20):
            oracle.affine_into(src, bufs[0], float(sc[i]), 0.0)
            oracle.affine_into(bufs[0], bufs[1], 1.0, float(of[i]))
            src = bufs[1]

    r, n, el = _cpu_rate(chain_per_node, 8.0 * n64 / 1e9, seconds)
    row("affine_chain20_64M", r, "GB/s", 1,
        f"oracle_affine, one pass per lazy node (40 nodes: x*a_i then +b_i), {sub}", n, el)
    return out


def host_cpu_info() -> dict:
    """nproc, the CPUs this process may use, and sockets x cores from
    /proc/cpuinfo (Linux)."""
    info = {"nproc": os.cpu_count()}
    try:
        info["affinity"] = len(os.sched_getaffinity(0))
    except Exception:
        pass
    try:
        phys, cores, model = set(), set(), None
        cur = {}
        for line in open("/proc/cpuinfo"):
            if ":" in line:
                k, v = (x.strip() for x in line.split(":", 1))
                cur[k] = v
            elif cur:
                phys.add(cur.get("physical id"))
                cores.add((cur.get("physical id"), cur.get("core id")))
                model = model or cur.get("model name")
                cur = {}
        info.update({"sockets": len(phys), "physical_cores": len(cores), "model": model})
    except Exception:
        pass
    return info


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "the multi-GPU sharding is a design only and is not run.", file=sys.stderr)
        return 2
    from silarray_amd import _native as nat

    nat.init()
    info = nat.device_info()
    log(f"device {info}")
    only = set(filter(None, args.only.split(",")))
    want = (lambda k: not only or k in only)
    g = np.random.default_rng(SEED)

    res = {}
    S = 8192
    if want("sgemm"):
        log(f"sgemm {S}^3: warmup {args.warmup}, steps {args.steps}")
        res["sgemm"] = bench_sgemm(nat, S, args.steps, args.warmup, g)
        log(f"sgemm {res['sgemm']}")
    secondary = {}
    gemv_rotated_only = "gemv_rotated" in only
    if want("gemv") or gemv_rotated_only:
        r = bench_gemv(nat, g, hot=not gemv_rotated_only)
        log(f"gemv {r}")
        secondary["gemv_1x4096x4096"] = {
            "value": round(r["gbs"], 1), "unit": "GB/s", "us": round(r["us"], 2),
            # the same 64 MiB read by the library's one-launch sum, same rotation
            "read_same_bytes_gbs": round(r["read_gbs"], 1), "read_same_bytes_us":
            round(r["read_us"], 2), "of_read": round(r["gbs"] / r["read_gbs"], 3),
            "roofline": roofline("hbm", r["gbs"], load_traffic("gemv_1x4096x4096"))}
        if "gbs_hot" in r:
            secondary["gemv_1x4096x4096"]["hot_cache_gbs"] = round(r["gbs_hot"], 1)
    if want("small_batch"):
        r = bench_small_batch(nat, g)
        log(f"small_batch {r}")
        secondary["sgemm_32x768x4096"] = {
            "value": round(r["gbs"], 1), "unit": "GB/s", "hot_cache_gbs": round(r["gbs_hot"], 1),
            "tflops": round(r["tflops"], 2),
            "us": round(r["us"], 2),
            "roofline": roofline("hbm", r["gbs"], load_traffic("sgemm_32x768x4096"))}
    if want("linear_sigmoid"):
        r = bench_linear_sigmoid(nat, g)
        log(f"linear_sigmoid {r}")
        secondary["linear_sigmoid_256x4096x4096"] = {
            "value": round(r["tflops"], 2), "unit": "TFLOP/s", "us": round(r["us"], 1),
            "roofline": roofline("mfma", r["tflops"], load_traffic("linear_sigmoid_256x4096x4096"))}
    conv_layers = {n for n, *_ in CONV_LAYERS if f"conv2d_{n}" in only}
    if want("conv2d") or conv_layers:
        for k, v in bench_conv2d(nat, g, layers=conv_layers or None).items():
            log(f"{k} {v}")
            traffic = load_traffic(v["traffic_key"])
            if v["hbm_bound"]:  # below the ridge (19.7 flop/B): priced against HBM
                secondary[k] = {"value": round(v["gbs"], 1), "unit": "GB/s",
                                "tflops": round(v["tflops"], 2), "us": round(v["us"], 2),
                                "reference_m1pro_ms": v["ref_ms"],
                                "roofline": roofline("hbm", v["gbs"], traffic)}
            else:
                secondary[k] = {"value": round(v["tflops"], 2), "unit": "TFLOP/s",
                                "us": round(v["us"], 1), "reference_m1pro_ms": v["ref_ms"],
                                "roofline": roofline("mfma", v["tflops"], traffic)}
            # no cpu_baseline: the reference's conv2d has no CPU path
            secondary[k]["cpu_baseline"] = None
            secondary[k]["cpu_baseline_note"] = (
                "the reference evaluates conv2d on the GPU only (include/array.h:2259-2272 "
                "calls gpu::conv2d on every device)")
    if want("rowops"):
        r = bench_rowops(nat, g)
        log(f"rowops {r}")
        for k, v in r.items():
            secondary[f"{k}_4096x8192"] = {"value": round(v["gbs"], 1), "unit": "GB/s",
                                           "hot_cache_gbs": round(v["gbs_hot"], 1),
                                           "us": round(v["us"], 2),
                                           "roofline": roofline("hbm", v["gbs"],
                                                                load_traffic(f"{k}_4096x8192"))}
            if "copy_gbs" in v:
                # same-bytes device copy timed in this run: the shape-free ceiling
                secondary[f"{k}_4096x8192"]["copy_same_bytes_gbs"] = round(v["copy_gbs"], 1)
                secondary[f"{k}_4096x8192"]["of_copy"] = round(v["of_copy"], 3)
    if want("reductions"):
        r = bench_reductions(nat, g)
        log(f"reductions {r}")
        for k, v in r.items():
            e = {"value": round(v["gbs"], 1), "unit": "GB/s",
                 "hot_cache_gbs": round(v["gbs_hot"], 1), "us": round(v["us"], 2),
                 "roofline": roofline("hbm", v["gbs"], load_traffic(f"{k}_64M"))}
            if "index_ok" in v:
                e["index_ok"] = v["index_ok"]
            secondary[f"{k}_64M"] = e
    if want("affine_chain"):
        r = bench_affine_chain(nat, g)
        log(f"affine_chain {r}")
        secondary["affine_chain20_64M"] = {"value": round(r["gbs"], 1), "unit": "GB/s",
                                           "us": round(r["us"], 2),
                                           "roofline": roofline("hbm", r["gbs"],
                                                                load_traffic("affine_chain20_64M"))}
    if only and "copy" in only:
        r = bench_copy(nat, g)
        log(f"copy {r}")
        secondary["copy_256MiB"] = {"value": round(r["gbs"], 1), "unit": "GB/s",
                                    "us": round(r["us"], 2)}
    if want("sgemm_sweep"):
        # 1024^3 is BASELINE config 1 (the reference times it through
        # sil::array::dot, bench/micro/bench_sgemm.cpp:34)
        for s in (1024, 2048, 4096):
            r = bench_sgemm(nat, s, 20, 3, g, min_warm_s=WARM_S)
            log(f"sgemm {s}^3 {r}")
            secondary[f"sgemm_{s}"] = {"value": round(r["tflops_kernel"], 2), "unit": "TFLOP/s",
                                       "roofline": roofline("mfma", r["tflops_kernel"])}

    if want("graphs"):
        for r in bench_graphs():
            log(f"graph {r}")
            w = r["workload"]
            if w == "encoder_block":
                key = f"encoder_block_B{r['B']}_S{r['S']}_D{r['D']}_H{r['H']}_F{r['F']}"
            elif w == "transformer_block":
                key = f"transformer_block_seq{r['seq']}_d{r['d_model']}"
            elif w == "mlp_linear_sigmoid":
                key = f"mlp_linear_sigmoid_batch{r['batch']}"
            elif w == "train_step":
                key = f"train_step_768x2048_batch{r['batch']}"
            elif w == "mnist":
                for k, ref in REF_MNIST_MS.items():
                    secondary[f"mnist_{k[:-3]}"] = {
                        "value": r[k], "unit": "ms", "higher_is_better": False,
                        "reference_m1pro_ms": ref,
                        "data": "synthetic images in [0,1) and labels, MNIST shapes "
                                "(60000 train, 10000 test)"}
                continue
            elif w == "micro":
                name = r["name"]
                key = "micro_" + "".join(ch if ch.isalnum() else "_" for ch in name).strip("_")
                while "__" in key:
                    key = key.replace("__", "_")
                secondary[key] = {"value": r["us"], "unit": "us", "higher_is_better": False,
                                  "reference_m1pro_us": REF_MICRO_US.get(name),
                                  "timing": "median of op + eval + synchronize iterations",
                                  "reference_case": name}
                continue
            elif w == "transfer":
                secondary["host_transfer_256MiB"] = {
                    "value": r["h2d_gbs"], "unit": "GB/s (host to HBM)", "d2h_gbs": r["d2h_gbs"],
                    "timing": "median of upload/download + one kernel, kernel time subtracted",
                    "note": "pinned host mirrors; pageable memory gives 31.7 / 18.3 GB/s here"}
                continue
            else:
                key = f"{w}_64M_api"
            if "gemm_tflops" in r:
                e = {"value": r["gemm_tflops"], "unit": "TFLOP/s (GEMM flops / wall)",
                     "ms": r["ms"], "timing": "median of eval+synchronize iterations"}
            else:
                e = {"value": r["gbs"], "unit": "GB/s", "ms": r["ms"],
                     "timing": "median of eval+synchronize iterations"}
            ref = REF_TRANSFORMER_MS.get((r.get("seq"), r.get("d_model")))
            if w == "transformer_block" and ref is not None:
                e["reference_m1pro_ms"] = ref
            if w == "train_step" and r["batch"] in REF_TRAIN_MS:
                e["reference_m1pro_ms"] = REF_TRAIN_MS[r["batch"]]
            secondary[key] = e

    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline")
        cpu = cpu_baseline(args.cpu_seconds)
        log(f"cpu {cpu}")
        for key, base in cpu_rows(args.cpu_row_seconds).items():
            log(f"cpu {key} {base}")
            if key in secondary:
                secondary[key]["cpu_baseline"] = base

    line = {"metric": METRIC, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
            "data": f"synthetic: uniform[-1,1] fp32 A, B from numpy PCG64 seed {SEED}",
            "config": {"workload": "sgemm_8192x8192x8192", "M": S, "N": S, "K": S,
                       "layout": "row-major NN", "parallelism": "single GPU"}}
    if "sgemm" in res:
        r = res["sgemm"]
        line.update({"value": round(r["tflops_wall"], 2), "unit": "TFLOP/s",
                     "ms_per_step": round(r["wall_ms_per_step"], 4),
                     "roofline": roofline("mfma", r["tflops_kernel"],
                                          load_traffic("sgemm_8192x8192x8192"))})
    else:
        line.update({"value": None, "unit": "TFLOP/s", "ms_per_step": None, "roofline": None})
    line["cpu_baseline"] = cpu
    # The rows BASELINE.json gates (HBM-bound kernels against 75% of 8 TB/s)
    # go last in `secondary`, with the GEMV half of the headline metric at the
    # very end, followed by a copy of the GEMV row: the end of the line is what
    # a truncated log keeps.
    gated = [k for k in GATED_ROWS if k in secondary]
    line["secondary"] = {**{k: v for k, v in secondary.items() if k not in gated},
                         **{k: secondary[k] for k in gated}}
    line["device"] = info
    if "gemv_1x4096x4096" in secondary:
        gv = secondary["gemv_1x4096x4096"]
        line["gemv_1x4096x4096"] = {"value": gv["value"], "unit": "GB/s", "us": gv["us"],
                                    "frac": gv["roofline"]["frac"],
                                    "read_same_bytes_gbs": gv["read_same_bytes_gbs"]}
    summary = ", ".join(f"{k} {secondary[k]['value']} {secondary[k]['unit']}"
                        f" ({secondary[k]['roofline']['frac']:.3f})" for k in gated)
    if summary:
        log(f"gated rows: {summary}")
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
