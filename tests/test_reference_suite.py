"""The drop-in check: the reference's own doctest suite, unchanged, against
this build.

The reference's test files (test/test_array.cpp, test_examples.cpp,
test_perceptron.cpp, test_2lnn.cpp and the runner test.cpp, with the doctest.h
the reference vendors next to them) are compiled where they lie, with
silarray_amd/include on the include path in place of the reference's
include/, by oracle/Makefile into oracle/_ref/reference_tests (linked to
libsilgpu.so).  Nothing of the reference is copied into this repository.

- CPU: each file passes a syntax-only compile against silarray_amd/include
  (needs the reference checkout; skipped without it).
- GPU: the built suite runs on the MI355X in its default mode and with
  --gpu (the reference's use_mps()), and every test case passes.  The GPU box
  has no reference checkout, so this runs the binary build() made here.
"""

from __future__ import annotations

import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
REF_TEST_DIR = Path("/root/reference/test")
FILES = ["test_array.cpp", "test_examples.cpp", "test_perceptron.cpp", "test_2lnn.cpp",
         "test.cpp"]
CXX = "/opt/rocm/llvm/bin/clang++"
SUITE = ROOT / "oracle" / "_ref" / "reference_tests"


@pytest.mark.parametrize("name", FILES)
def test_reference_test_file_compiles_against_this_build(name):
    src = REF_TEST_DIR / name
    if not src.exists():
        pytest.skip("no reference checkout on this machine")
    proc = subprocess.run([CXX, "-std=c++23", "-fsyntax-only",
                           f"-I{ROOT / 'silarray_amd' / 'include'}", f"-I{REF_TEST_DIR}",
                           str(src)], capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0, proc.stderr[-4000:]


def _run_suite(args):
    if not SUITE.exists():
        pytest.skip(f"{SUITE} is not built (build() builds it where the reference "
                    "checkout exists)")
    print(f"reference doctest suite {' '.join(args) or '(default mode)'}", flush=True)
    proc = subprocess.run([str(SUITE), *args], capture_output=True, text=True, timeout=600)
    print(proc.stdout[-6000:])
    print(proc.stderr[-2000:])
    return proc


@pytest.mark.gpu
@pytest.mark.parametrize("mode", [[], ["--gpu"]])
def test_reference_suite_passes_on_mi355x(mode):
    proc = _run_suite(mode)
    m = re.search(r"test cases:\s*(\d+)\s*\|\s*(\d+) passed\s*\|\s*(\d+) failed", proc.stdout)
    assert m, proc.stdout[-2000:]
    total, passed, failed = map(int, m.groups())
    assert total >= 50 and failed == 0 and passed == total, proc.stdout[-4000:]
    assert proc.returncode == 0
