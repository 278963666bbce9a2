"""Times every fixed GEMM plan (tile x K split, silgpu_sgemm_tuned) and the
library's own choice (silgpu_sgemm) for the given row-major NN products on
device 0, one JSON line per shape: {"shape": [M, N, K], "us": {"auto": t,
"<tile>/<splits>": t, ...}} with microseconds per launch over back-to-back
launches (HIP events).  Tiles: 1 = 128x128, 2 = 64x64, 4 = 128x64,
5 = 256x256 (M, N multiples of 256 only).  These sweeps are what the cost
model in choose_plan (csrc/gemm.hip) is fitted to.

    python silarray_amd/bench/gemm_plan_sweep.py 256x768x3072 2048x2048x2048 ...
"""
import json
import sys
from pathlib import Path

import numpy as np

sys.path.insert(0, str(Path(__file__).resolve().parents[2]))
import bench  # noqa: E402  (the repository's bench.py: Timer)
from silarray_amd import _native as nat  # noqa: E402


def sweep(M, N, K, g, t):
    A = nat.DeviceBuffer.from_array(g.uniform(-1, 1, (M, K)).astype(np.float32))
    B = nat.DeviceBuffer.from_array(g.uniform(-1, 1, (K, N)).astype(np.float32))
    C = nat.DeviceBuffer(4 * M * N)
    reps = 100 if M * N * K < 2**32 else 20
    us = {"auto": t.ms_per_launch(
        lambda i: nat.sgemm(0, 0, M, N, K, A, K, 0, B, N, 0, C, N, 0), reps, 5) * 1e3}
    for tile in (1, 2, 4, 5):
        if tile == 5 and (M % 256 or N % 256):
            continue
        for sp in (1, 2, 4, 8, 16):
            if K // sp < 32:
                continue
            us[f"{tile}/{sp}"] = t.ms_per_launch(
                lambda i: nat.sgemm_tuned(0, 0, M, N, K, A, K, 0, B, N, 0, C, N, 0, 1, None, 0,
                                          0, tile, sp), reps, 5) * 1e3
    return {"shape": [M, N, K], "us": {k: round(v, 2) for k, v in us.items()}}


def main(argv):
    if not argv:
        print(__doc__)
        return 2
    nat.init()
    g = np.random.default_rng(1)
    t = bench.Timer(nat)
    for s in argv:
        M, N, K = (int(x) for x in s.lower().split("x"))
        print(json.dumps(sweep(M, N, K, g, t)), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
