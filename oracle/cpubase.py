"""The CPU baseline's build of the oracle's loops.

TEST INFRASTRUCTURE ONLY (the cpu_baseline leg of bench.py): the same C
source as liboracle.so (oracle.c), compiled -O3 for each x86-64 level by
oracle/Makefile; load() picks the widest level this host's CPU supports,
which is what -march=native would give when built on that host (the GPU
box's CPU is not the build container's).
"""

from __future__ import annotations

import importlib.util
from pathlib import Path

HERE = Path(__file__).resolve().parent

_V3 = {"avx", "avx2", "bmi1", "bmi2", "f16c", "fma", "movbe", "xsave"}
_V4 = _V3 | {"avx512f", "avx512bw", "avx512cd", "avx512dq", "avx512vl"}


def host_level() -> str:
    """x86-64 microarchitecture level of this host: v4, v3 or v2."""
    flags = set()
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("flags"):
                flags = set(line.split(":", 1)[1].split())
                break
    except OSError:
        pass
    if _V4 <= flags:
        return "v4"
    if _V3 <= flags:
        return "v3"
    return "v2"


def load():
    """(module, level): oracle.py's wrappers bound to libcpubase_<level>.so."""
    level = host_level()
    path = HERE / f"libcpubase_{level}.so"
    if not path.exists():
        raise FileNotFoundError(f"{path} is missing: run make -C oracle cpubase")
    spec = importlib.util.spec_from_file_location(f"oracle_cpubase_{level}", HERE / "oracle.py")
    mod = importlib.util.module_from_spec(spec)
    mod.LIB_OVERRIDE = str(path)
    spec.loader.exec_module(mod)
    return mod, level
