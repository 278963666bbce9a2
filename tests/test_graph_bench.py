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


U32 = 2.0 ** -24  # fp32 unit roundoff


def _gemm_ref(A, W, bias, K, resid=None):
    """One product stage c = A W + bias (+ resid) against float64 from the
    same fp32 inputs.  Per element: |c - c64| <= 1e-5 sqrt(K) (sum_k |a w| +
    |bias|) -- the SGEMM bar -- plus 2 ulp of |resid| + |c64| for a residual
    add.  Normwise: the RMS error is at most sqrt(K) u RMS(sum_k |a w| +
    |bias|), u = 2^-24.  Rounding errors of a K-term fp32 sum grow like a
    random walk, RMS about u sum|a w|, so this bar holds with a margin of
    sqrt(K) while a defect of 1e-4 in the epilogue (a lost or doubled bias
    rounding, a wrong residual row) already fails it at K = 768."""
    ref = A @ W + (bias if bias is not None else 0.0)
    mag = np.abs(A) @ np.abs(W) + (np.abs(bias) if bias is not None else 0.0)
    bar = 1e-5 * np.sqrt(K) * mag
    if resid is not None:
        ref = ref + resid
        bar = bar + 2 * 2 * U32 * (np.abs(resid) + np.abs(ref))
    return ref, mag, bar


def _check(name, got, ref, bar, mag=None, K=None):
    err = np.abs(got - ref)
    worst = float(np.max(err / bar))
    assert worst <= 1.0, f"{name}: per-element error {worst:.3f} of its bar"
    if mag is not None:
        rms, rms_bar = np.sqrt(np.mean(err ** 2)), np.sqrt(K) * U32 * np.sqrt(np.mean(mag ** 2))
        assert rms <= rms_bar, f"{name}: RMS error {rms:.3e} > {rms_bar:.3e}"


def _attention_check(qkv, merged, B, S, D, H):
    """Attention from this run's fp32 qkv against float64, per element:
    ctx = P v with P = softmax(scale q k^T).  First-order propagation of the
    per-op bars: a score error d_j <= 1e-5 sqrt(dh) scale sum_e |q_e k_je|
    (+ its scaling's rounding) moves ctx by sum_j P_j |v_j - ctx| d_j; the
    softmax's relative 1e-5 by 1e-5 sum_j P_j |v_j|; the P v product's SGEMM
    bar is 1e-5 sqrt(S) sum_j P_j |v_j|.  |v_j - ctx| <= |v_j| + |ctx| keeps
    every term a matrix product."""
    dh = D // H
    scale = float(np.float32(1.0) / np.sqrt(np.float32(dh)))
    heads = qkv.reshape(B, S, 3, H, dh).transpose(2, 0, 3, 1, 4)
    got = merged.reshape(B, S, H, dh).transpose(0, 2, 1, 3)
    worst = 0.0
    for b in range(B):
        for h in range(H):
            q, k, v = heads[0, b, h], heads[1, b, h], heads[2, b, h]
            sc = (q @ k.T) * scale
            P = np.exp(sc - sc.max(axis=1, keepdims=True))
            P /= P.sum(axis=1, keepdims=True)
            ctx = P @ v
            tau = 1e-5 * np.sqrt(dh) * scale * (np.abs(q) @ np.abs(k).T) + 2 * U32 * np.abs(sc)
            Pt = P * tau
            bar = (Pt @ np.abs(v) + Pt.sum(axis=1, keepdims=True) * np.abs(ctx) +
                   (1e-5 + 1e-5 * np.sqrt(S)) * (P @ np.abs(v)))
            worst = max(worst, float(np.max(np.abs(got[b, h] - ctx) / bar)))
    assert worst <= 1.0, f"attention: per-element error {worst:.3f} of its bar"


@pytest.mark.gpu
# The last case is BASELINE config 5 at its stated size (head dim 64: the
# fused attention kernel's D = 64 path, the head-merge relayout, the
# out-projection and FFN products with residual epilogues).
@pytest.mark.parametrize("dims", [(2, 64, 128, 4, 256), (1, 37, 96, 3, 200),
                                  (4, 512, 768, 12, 3072)])
def test_encoder_block_stages_match_f64(tmp_path, dims):
    """Each stage of the block, as sil::eval lowered it, against float64
    computed from this run's own fp32 inputs to that stage, with that op's
    bar: layer_norm relative 1e-5 (of max(1, |y|)), each product the SGEMM
    bar plus the normwise rounding bar, attention the propagated bar.  The
    block evaluated alone and with its intermediates held give the same bits."""
    B, S, D, H, F = dims
    print(f"encoder-dump {dims}", flush=True)
    proc = subprocess.run([str(_bench()), "encoder-dump", *map(str, dims), str(tmp_path)],
                          capture_output=True, text=True, timeout=120)
    assert proc.returncode == 0, proc.stderr
    M = B * S
    shapes = {"x": (M, D), "Wqkv": (D, 3 * D), "bqkv": (3 * D,), "Wo": (D, D), "bo": (D,),
              "W1": (D, F), "c1": (F,), "W2": (F, D), "c2": (D,), "h": (M, D),
              "qkv": (M, 3 * D), "merged": (M, D), "r1": (M, D), "h2": (M, D), "ff": (M, F),
              "out": (M, D), "out_staged": (M, D)}
    a32 = {n: np.fromfile(tmp_path / f"{n}.bin", dtype=np.float32).reshape(sh)
           for n, sh in shapes.items()}
    assert np.array_equal(a32["out"], a32["out_staged"])
    p = {n: v.astype(np.float64) for n, v in a32.items()}

    ref = _layer_norm(p["x"])
    _check("layer_norm 1", p["h"], ref, 1e-5 * np.maximum(1.0, np.abs(ref)))
    ref, mag, bar = _gemm_ref(p["h"], p["Wqkv"], p["bqkv"], D)
    _check("qkv", p["qkv"], ref, bar, mag, D)
    _attention_check(p["qkv"], p["merged"], B, S, D, H)
    ref, mag, bar = _gemm_ref(p["merged"], p["Wo"], p["bo"], D, resid=p["x"])
    _check("out-proj + residual", p["r1"], ref, bar, mag, D)
    ref = _layer_norm(p["r1"])
    _check("layer_norm 2", p["h2"], ref, 1e-5 * np.maximum(1.0, np.abs(ref)))
    ref, mag, bar = _gemm_ref(p["h2"], p["W1"], p["c1"], D)
    _check("FFN1 + relu", p["ff"], np.maximum(ref, 0.0), bar, mag, D)
    ref, mag, bar = _gemm_ref(p["ff"], p["W2"], p["c2"], F, resid=p["r1"])
    _check("FFN2 + residual", p["out"], ref, bar, mag, F)


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
