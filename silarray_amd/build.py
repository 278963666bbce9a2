"""Build recipe for libsilgpu.so (HIP, gfx950) and the C++ front-end test binary.

Every HIP translation unit under csrc/ is compiled with hipcc for gfx950 only
and linked into silarray_amd/libsilgpu.so, in-tree, so the library travels
with the repository snapshot.  Flags:
  --offload-arch=gfx950            CDNA4 code objects only
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                   no packed-fp32 VALU instructions
  -ffp-contract=off                every elementwise op rounds on its own, so
                                   fused eval programs equal node-by-node fp32
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libsilgpu.so"
INCLUDE = ROOT / "include"

HIP_SOURCES = ["runtime.hip", "elementwise.hip", "reduce.hip", "rowops.hip", "gemm.hip",
               "attention.hip", "conv.hip"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    f"-I{INCLUDE}",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = proc.stdout
    # hipcc's host pass does not know the packed-fp32 feature; that warning is noise.
    lines = [l for l in out.splitlines() if "packed-fp32-ops" not in l and l.strip()]
    if proc.returncode != 0:
        raise RuntimeError("command failed:\n  " + " ".join(cmd) + "\n" + "\n".join(lines))
    if lines:
        sys.stderr.write("\n".join(lines) + "\n")


def _compile(src: str) -> Path:
    obj = BUILD / (Path(src).stem + ".o")
    _run([HIPCC, *HIP_FLAGS, "-c", str(CSRC / src), "-o", str(obj)])
    return obj


def build_library(jobs: int = 5) -> Path:
    """Compiles csrc/*.hip for gfx950 and links libsilgpu.so (always rebuilds)."""
    if not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    BUILD.mkdir(exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, HIP_SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, LIB)
    return LIB


CXX = os.environ.get("SIL_CXX", "/opt/rocm/llvm/bin/clang++")
CPP_TESTS = ROOT / "tests" / "cpp"


def _cxx(src: Path, out: Path, rpath: str) -> Path:
    tmp = out.with_suffix(".tmp")
    _run([CXX, "-std=c++23", "-O2", "-ffp-contract=off", "-Wall", "-Wno-unused-function",
          f"-I{PKG / 'include'}", str(src), "-o", str(tmp), f"-L{PKG}", "-lsilgpu",
          f"-Wl,-rpath,{rpath}"])
    os.replace(tmp, out)
    return out


def build_cpp_tests() -> Path:
    """Compiles the C++ front-end tests (tests/cpp/test_array.cpp) against the
    headers in silarray_amd/include, linked to the in-tree libsilgpu.so."""
    return _cxx(CPP_TESTS / "test_array.cpp", CPP_TESTS / "test_array",
                "$ORIGIN/../../silarray_amd")


def build_cpp_random_graphs() -> Path:
    """Compiles the random sil::eval graph test (tests/cpp/random_graphs.cpp)."""
    return _cxx(CPP_TESTS / "random_graphs.cpp", CPP_TESTS / "random_graphs",
                "$ORIGIN/../../silarray_amd")


def build_cpp_bench() -> Path:
    """Compiles the sil::eval graph benchmark (silarray_amd/bench/bench_graph.cpp)."""
    return _cxx(PKG / "bench" / "bench_graph.cpp", PKG / "bench" / "bench_graph", "$ORIGIN/..")


def build_cpp() -> list[Path]:
    return [build_cpp_tests(), build_cpp_random_graphs(), build_cpp_bench()]


if __name__ == "__main__":
    print(build_library())
    print(build_cpp())
