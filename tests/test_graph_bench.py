"""The sil::eval graph benchmark (silarray_amd/bench/bench_graph.cpp): one
transformer encoder block written against the C++ sil::array API, lowered by
sil::eval onto the HIP kernels, checked against a float64 numpy restatement of
the same block.  The block combines every operator of the hot path the reference
exposes to a model (examples/transformer_*.cpp use the same operators):
layer_norm, linear (bias epilogue), strided batched products over head views,
row softmax, the relu epilogue fusion and fused residual adds."""

from __future__ import annotations

import json
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
BENCH = ROOT / "silarray_amd" / "bench" / "bench_graph"


def _bench() -> Path:
    if not BENCH.exists():
        pytest.fail(f"{BENCH} is not built (run __graft_entry__.build())")
    return BENCH


def test_usage_without_gpu():
    proc = subprocess.run([str(_bench()), "no-such-mode"], capture_output=True, text=True,
                          timeout=60)
    assert proc.returncode == 2 and "usage" in proc.stderr


def test_rejects_bad_head_split():
    proc = subprocess.run([str(_bench()), "encoder", "1", "8", "30", "4", "16", "1"],
                          capture_output=True, text=True, timeout=60)
    assert proc.returncode == 2 and "multiple of H" in proc.stderr


def _layer_norm(x, eps=1e-5):
    mu = x.mean(axis=1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps)


def _softmax(x):
    e = np.exp(x - x.max(axis=-1, keepdims=True))
    return e / e.sum(axis=-1, keepdims=True)


def encoder_f64(p, B, S, D, H, F):
    """Float64 restatement of the block bench_graph builds (gamma=1, beta=0)."""
    dh = D // H
    x = p["x"].reshape(B * S, D)
    h = _layer_norm(x)
    qkv = h @ p["Wqkv"].reshape(D, 3 * D) + p["bqkv"]
    heads = qkv.reshape(B, S, 3, H, dh).transpose(2, 0, 3, 1, 4)
    q, k, v = heads[0], heads[1], heads[2]
    scores = (q @ k.transpose(0, 1, 3, 2)) * (1.0 / np.sqrt(np.float32(dh)).astype(np.float64))
    ctx = _softmax(scores) @ v
    merged = ctx.transpose(0, 2, 1, 3).reshape(B * S, D)
    r1 = x + merged @ p["Wo"].reshape(D, D) + p["bo"]
    ff = np.maximum(_layer_norm(r1) @ p["W1"].reshape(D, F) + p["c1"], 0.0)
    return r1 + ff @ p["W2"].reshape(F, D) + p["c2"]


@pytest.mark.gpu
# The last case is BASELINE config 5 at its stated size (head dim 64: the
# fused attention kernel's D = 64 path, the head-merge relayout, the
# out-projection and FFN products with residual epilogues).
@pytest.mark.parametrize("dims", [(2, 64, 128, 4, 256), (1, 37, 96, 3, 200),
                                  (4, 512, 768, 12, 3072)])
def test_encoder_block_matches_f64(tmp_path, dims):
    B, S, D, H, F = dims
    print(f"encoder-dump {dims}", flush=True)
    proc = subprocess.run([str(_bench()), "encoder-dump", *map(str, dims), str(tmp_path)],
                          capture_output=True, text=True, timeout=120)
    assert proc.returncode == 0, proc.stderr
    p = {n: np.fromfile(tmp_path / f"{n}.bin", dtype=np.float32).astype(np.float64)
         for n in ("x", "Wqkv", "bqkv", "Wo", "bo", "W1", "c1", "W2", "c2")}
    out = np.fromfile(tmp_path / "out.bin", dtype=np.float32).reshape(B * S, D)
    ref = encoder_f64(p, B, S, D, H, F)
    # fp32 products over K <= F with O(1) activations: 1e-5 * sqrt(K) per
    # product, four products deep, plus the two layer norms.
    tol = 4e-5 * np.sqrt(max(D, F))
    err = np.abs(out - ref).max()
    assert err <= tol, f"max abs error {err:.3e} > {tol:.3e}"


@pytest.mark.gpu
def test_chain_and_encoder_report_json():
    print("bench_graph chain / encoder (small)", flush=True)
    out = subprocess.run([str(_bench()), "chain", str(1 << 20), "3"], capture_output=True,
                         text=True, timeout=120, check=True).stdout
    rec = json.loads(out.strip().splitlines()[-1])
    assert rec["workload"] == "affine_chain20" and rec["ms"] > 0
    out = subprocess.run([str(_bench()), "encoder", "1", "32", "64", "2", "128", "3"],
                         capture_output=True, text=True, timeout=120, check=True).stdout
    rec = json.loads(out.strip().splitlines()[-1])
    assert rec["workload"] == "encoder_block" and rec["ms"] > 0


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def train_step_f64(p, B, D, lr=0.01):
    """Float64 restatement of one step of the reference's training benchmark
    (bench/composite/bench_train.cpp:39-58): D -> H -> D sigmoid MLP, MSE
    gradient (o2 - Y) * 2 / (B D), sigmoid_backward = dout * s * (1 - s)
    (include/gpu_kernels.metal:1469-1477), SGD with learning rate lr."""
    x, Y = p["x"].reshape(B, D), p["Y"].reshape(B, D)
    W1, W2 = p["W1"].reshape(D, -1), p["W2"].reshape(-1, D)
    b1, b2 = p["b1"], p["b2"]
    n1 = x @ W1 + b1
    o1 = _sigmoid(n1)
    n2 = o1 @ W2 + b2
    o2 = _sigmoid(n2)
    dout = (o2 - Y) * 2.0 * (1.0 / (B * D))
    s2 = _sigmoid(n2)
    dout = dout * s2 * (1.0 - s2)
    dW2, db2 = o1.T @ dout, dout.sum(axis=0)
    dout1 = dout @ W2.T
    s1 = _sigmoid(n1)
    dout1 = dout1 * s1 * (1.0 - s1)
    dW1, db1 = x.T @ dout1, dout1.sum(axis=0)
    return {"W1": W1 - lr * dW1, "b1": b1 - lr * db1, "W2": W2 - lr * dW2, "b2": b2 - lr * db2,
            "dW1": dW1, "db1": db1, "dW2": dW2, "db2": db2}


@pytest.mark.gpu
@pytest.mark.parametrize("dims", [(64, 768, 2048), (5, 33, 70), (32, 4, 3)])
def test_train_step_matches_f64(tmp_path, dims):
    """One training step through sil::eval (linear, sigmoid, sigmoid_backward,
    transposed products, sum(0), SGD update) against float64.  The update is
    compared as the implied gradient (W - W_new) / lr, relative to the f64
    gradient's scale, since lr * grad is far below W's own rounding."""
    B, D, H = dims
    print(f"train-dump {dims}", flush=True)
    proc = subprocess.run([str(_bench()), "train-dump", str(B), str(D), str(H), str(tmp_path)],
                          capture_output=True, text=True, timeout=120)
    assert proc.returncode == 0, proc.stderr
    p = {n: np.fromfile(tmp_path / f"{n}.bin", dtype=np.float32).astype(np.float64)
         for n in ("x", "Y", "W1", "b1", "W2", "b2")}
    ref = train_step_f64(p, B, D)
    lr = 0.01
    for name in ("W1", "b1", "W2", "b2"):
        new = np.fromfile(tmp_path / f"{name}_new.bin", dtype=np.float32).astype(np.float64)
        ref_new = ref[name].reshape(-1)
        # the parameter itself: fp32 rounding of W - lr * grad
        assert np.all(np.abs(new - ref_new) <= 2 * np.finfo(np.float32).eps * np.abs(ref_new)
                      + 1e-4 * np.abs(ref["d" + name]).max() * lr + 1e-30), name
        # the step: (W - W_new) / lr against the f64 gradient; the fp32
        # subtraction W + (-lr * g) loses log2(|W| / |lr g|) bits of the step
        g = (p[name] - new) / lr
        gref = ref["d" + name].reshape(-1)
        ulp_w = np.finfo(np.float32).eps * np.abs(p[name]).max()
        tol = 1e-4 * np.abs(gref).max() + 2 * ulp_w / lr
        assert np.abs(g - gref).max() <= tol, (name, np.abs(g - gref).max(), tol)


@pytest.mark.gpu
def test_train_reports_json():
    print("bench_graph train (small)", flush=True)
    out = subprocess.run([str(_bench()), "train", "16", "3"], capture_output=True, text=True,
                         timeout=120, check=True).stdout
    rec = json.loads(out.strip().splitlines()[-1])
    assert rec["workload"] == "train_step" and rec["batch"] == 16 and rec["ms"] > 0


@pytest.mark.gpu
def test_transfer_reports_json():
    print("bench_graph transfer (4M floats)", flush=True)
    out = subprocess.run([str(_bench()), "transfer", str(1 << 22), "3"], capture_output=True,
                         text=True, timeout=120, check=True).stdout
    rec = json.loads(out.strip().splitlines()[-1])
    assert rec["workload"] == "transfer" and rec["check"] == 1
    assert rec["h2d_ms"] > 0 and rec["d2h_ms"] > 0


@pytest.mark.gpu
def test_mnist_reports_json():
    """The reference's MNIST classifier and autoencoder loops on a small
    synthetic set: every phase runs and the classifier's squared error on
    its first batch goes down over the epoch (the labels are random, so
    the network can only fit them as noise, which SGD at lr 0.5 does)."""
    print("bench_graph mnist (2000 train, 500 test)", flush=True)
    out = subprocess.run([str(_bench()), "mnist", "2000", "500"], capture_output=True,
                         text=True, timeout=120, check=True).stdout
    rec = json.loads(out.strip().splitlines()[-1])
    assert rec["workload"] == "mnist"
    for k in ("classifier_train_epoch_ms", "classifier_inference_ms",
              "autoencoder_train_epoch_ms", "autoencoder_inference_ms"):
        assert rec[k] > 0, k
    first, last = rec["classifier_mse_first_batch"]
    assert np.isfinite(first) and np.isfinite(last) and last < first


@pytest.mark.gpu
def test_micro_reports_every_reference_case():
    """`bench_graph micro` times the reference's GPU micro-benchmarks: one
    JSON line per case, named as bench.py's table of published figures."""
    print("bench_graph micro", flush=True)
    import bench

    out = subprocess.run([str(_bench()), "micro"], capture_output=True, text=True, timeout=240,
                         check=True).stdout
    recs = [json.loads(l) for l in out.splitlines() if l.startswith("{")]
    assert all(r["workload"] == "micro" and r["us"] > 0 for r in recs)
    assert sorted(r["name"] for r in recs) == sorted(bench.REF_MICRO_US)
