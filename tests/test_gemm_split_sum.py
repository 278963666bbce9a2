"""K-split products on the 128 x 64 LDS-direct tiles: each split writes the
raw product over its K range to a partial plane, and splitk_sum_k adds the
planes and applies the epilogue.

Bar: bit-identical to the planes added in float32 in the kernel's order,
each plane being the same product over that split's K range alone (forced
to one split), then the bias and residual added in float32.  The order is
s = 0, 1, ... from zero, except with 8 or more splits over fewer than 65536
output groups of four, where wave w of a workgroup adds planes w, w + 4, ...
and the four sums are added in wave order.  C is filled with NaN first, so a
tile that was not written shows.  A product repeated after other split
products gives the same bits (the workspace keeps nothing between calls).
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import rng
from gpu_util import announce, down, up

pytestmark = pytest.mark.gpu

TILE_128x64 = 4


def _cdiv(a, b):
    return -(-a // b)


def _ranges(K, splits):
    # the K range of each split: klen rounded up to the 32-deep K tile
    klen = _cdiv(_cdiv(K, splits), 32) * 32
    n = _cdiv(K, klen)
    return [(s * klen, min(K, (s + 1) * klen)) for s in range(n)]


def _nan_buffer(native, n):
    return up(native, np.full(n, np.nan, np.float32))


def _planes_sum(native, A, B, ranges):
    """float32 sum over the splits' planes in splitk_sum_k's order."""
    M, N = A.shape[0], B.shape[1]
    planes = []
    for ks, ke in ranges:
        As, Bs = np.ascontiguousarray(A[:, ks:ke]), np.ascontiguousarray(B[ks:ke])
        dA, dB, dC = up(native, As), up(native, Bs), _nan_buffer(native, M * N)
        native.sgemm_tuned(0, 0, M, N, ke - ks, dA, ke - ks, 0, dB, N, 0, dC, N, 0,
                           tile=TILE_128x64, splits=1)
        assert native.last_plan() == [(TILE_128x64, 1, M)], native.last_plan()
        planes.append(down(native, dC, (M, N)))
    deep = len(planes) >= 8 and M * N // 4 < 65536
    if not deep:
        v = np.zeros((M, N), np.float32)
        for x in planes:
            v = v + x
        return v
    waves = []
    for w in range(4):
        v = np.zeros((M, N), np.float32)
        for x in planes[w::4]:
            v = v + x
        waves.append(v)
    return ((waves[0] + waves[1]) + waves[2]) + waves[3]


@pytest.mark.parametrize("M,N,K,splits", [
    (1024, 1024, 1024, 2),   # 256 workgroups: the 8-wave launch
    (2048, 768, 768, 4),     # 768 workgroups: 4 waves, 3 per CU
    (256, 1024, 4096, 8),
    (512, 512, 800, 3),      # the last split shorter (288, 288, 224)
    (256, 2048, 2048, 16),
    (128, 768, 2048, 16),    # 24576 output groups: the planes spread over four waves
])
def test_split_sum_is_the_plane_sum_in_order(native, M, N, K, splits):
    announce(f"split sum {M}x{N}x{K} splits={splits}")
    g = rng(M + N + K + splits)
    A = g.normal(0, 1, (M, K)).astype(np.float32)
    B = g.normal(0, 1, (K, N)).astype(np.float32)
    b = g.normal(0, 1, N).astype(np.float32)
    ranges = _ranges(K, splits)
    dA, dB, db = up(native, A), up(native, B), up(native, b)
    dC = _nan_buffer(native, M * N)
    native.sgemm_tuned(0, 0, M, N, K, dA, K, 0, dB, N, 0, dC, N, 0, bias=db, bias_len=N,
                       epi=native.EPI_BIAS, tile=TILE_128x64, splits=splits)
    assert native.last_plan() == [(TILE_128x64, len(ranges), M)], native.last_plan()
    C = down(native, dC, (M, N))
    want = _planes_sum(native, A, B, ranges) + b[None, :]
    assert not np.isnan(C).any()
    assert np.array_equal(C, want), float(np.max(np.abs(C - want)))


@pytest.mark.parametrize("M,N,K", [(1024, 768, 2048), (2048, 768, 3072)])
def test_split_sum_with_residual_matches_the_plane_sum(native, M, N, K):
    # silgpu_gemm with bias and residual on the planner's own pick (128 x 64
    # tiles with a K split for these shapes)
    announce(f"split sum residual {M}x{N}x{K}")
    g = rng(17 + M)
    A = g.normal(0, 1, (M, K)).astype(np.float32)
    B = g.normal(0, 1, (K, N)).astype(np.float32)
    b = g.normal(0, 1, N).astype(np.float32)
    R = g.normal(0, 1, (M, N)).astype(np.float32)
    dA, dB, db, dR = up(native, A), up(native, B), up(native, b), up(native, R)
    dC = _nan_buffer(native, M * N)
    native.gemm(0, 0, M, N, K, dA, K, dB, N, dC, N, epi=native.EPI_BIAS, bias=db, bias_len=N,
                residual=dR, ldr=N)
    plan = native.last_plan()
    assert len(plan) == 1 and plan[0][0] == TILE_128x64 and plan[0][1] > 1, plan
    C = down(native, dC, (M, N))
    want = (_planes_sum(native, A, B, _ranges(K, plan[0][1])) + b[None, :]) + R
    assert np.array_equal(C, want), float(np.max(np.abs(C - want)))


def test_split_products_repeat_bit_identically(native):
    # X, then two other split products, then X again: the same bits
    def run(M, N, K, splits, seed):
        g = rng(seed)
        A = g.normal(0, 1, (M, K)).astype(np.float32)
        B = g.normal(0, 1, (K, N)).astype(np.float32)
        dA, dB, dC = up(native, A), up(native, B), _nan_buffer(native, M * N)
        native.sgemm_tuned(0, 0, M, N, K, dA, K, 0, dB, N, 0, dC, N, 0, tile=TILE_128x64,
                           splits=splits)
        return down(native, dC, (M, N))

    announce("split products repeated")
    first = run(1024, 1024, 1024, 4, 3)
    run(512, 1024, 2048, 8, 4)
    run(1024, 1024, 1024, 2, 5)
    again = run(1024, 1024, 1024, 4, 3)
    assert not np.isnan(first).any()
    assert np.array_equal(first, again)


def test_split_dropped_where_tile_rows_exceed_32_bit_offsets(native):
    # 128 x 2^21 x 32 forced to two K splits: a 128-row tile of a split plane
    # spans 128 * N * 4 = 2^30 bytes, beyond the kernel's 32-bit plane
    # offsets, so the product runs unsplit (and correct)
    M, N, K = 128, 1 << 21, 32
    announce(f"split guard {M}x{N}x{K}")
    g = rng(23)
    A = g.uniform(-1, 1, (M, K)).astype(np.float32)
    B = g.uniform(-1, 1, (K, N)).astype(np.float32)
    dA, dB, dC = up(native, A), up(native, B), _nan_buffer(native, M * N)
    native.sgemm_tuned(0, 0, M, N, K, dA, K, 0, dB, N, 0, dC, N, 0, tile=TILE_128x64, splits=2)
    assert native.last_plan() == [(TILE_128x64, 1, M)], native.last_plan()
    C = down(native, dC, (M, N))
    cols = np.concatenate([np.arange(0, 64), g.integers(0, N, 256), np.arange(N - 64, N)])
    want = A.astype(np.float64) @ B[:, cols].astype(np.float64)
    err = np.abs(C[:, cols] - want)
    bar = 1e-5 * np.sqrt(K) * (np.abs(A).astype(np.float64) @ np.abs(B[:, cols]).astype(np.float64))
    assert not np.isnan(C).any()
    assert np.all(err <= bar), float(np.max(err / bar))


@pytest.mark.parametrize("ta,tb", [(0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K,splits", [(1024, 1024, 1024, 2), (2048, 768, 768, 4)])
def test_split_sum_with_transposed_operands(native, ta, tb, M, N, K, splits):
    # the same bar for the NT, TN and TT instantiations of the kernel: A
    # stored [K, M] when transposed, B stored [N, K]
    announce(f"split sum ta={ta} tb={tb} {M}x{N}x{K} splits={splits}")
    g = rng(M + N + K + 10 * ta + tb)
    A = g.normal(0, 1, (M, K)).astype(np.float32)
    B = g.normal(0, 1, (K, N)).astype(np.float32)
    As = np.ascontiguousarray(A.T) if ta else A
    Bs = np.ascontiguousarray(B.T) if tb else B
    lda, ldb = (M if ta else K), (K if tb else N)
    dA, dB, dC = up(native, As), up(native, Bs), _nan_buffer(native, M * N)
    native.sgemm_tuned(ta, tb, M, N, K, dA, lda, 0, dB, ldb, 0, dC, N, 0, tile=TILE_128x64,
                       splits=splits)
    ranges = _ranges(K, splits)
    assert native.last_plan() == [(TILE_128x64, len(ranges), M)], native.last_plan()
    C = down(native, dC, (M, N))
    # each plane: the same transposed product over its K range alone
    planes = []
    for ks, ke in ranges:
        Ap = np.ascontiguousarray(A[:, ks:ke].T) if ta else np.ascontiguousarray(A[:, ks:ke])
        Bp = np.ascontiguousarray(B[ks:ke].T) if tb else np.ascontiguousarray(B[ks:ke])
        Kp = ke - ks
        pA, pB, pC = up(native, Ap), up(native, Bp), _nan_buffer(native, M * N)
        native.sgemm_tuned(ta, tb, M, N, Kp, pA, (M if ta else Kp), 0, pB, (Kp if tb else N), 0,
                           pC, N, 0, tile=TILE_128x64, splits=1)
        assert native.last_plan() == [(TILE_128x64, 1, M)], native.last_plan()
        planes.append(down(native, pC, (M, N)))
    want = np.zeros((M, N), np.float32)
    for x in planes:
        want = want + x
    assert not np.isnan(C).any()
    assert np.array_equal(C, want), float(np.max(np.abs(C - want)))
