"""Runs the C++ front-end test binary (tests/cpp/test_array.cpp, built by
__graft_entry__.build()).  Host-only cases need no GPU; the full run does."""

import subprocess
from pathlib import Path

import pytest

BIN = Path(__file__).resolve().parent / "cpp" / "test_array"
RANDOM_GRAPHS = Path(__file__).resolve().parent / "cpp" / "random_graphs"


def _run(args, timeout):
    assert BIN.exists(), f"{BIN} not built: run __graft_entry__.build()"
    proc = subprocess.run([str(BIN), *args], capture_output=True, text=True, timeout=timeout)
    print(proc.stdout[-4000:])
    print(proc.stderr[-4000:])
    return proc


def test_cpp_host_cases():
    proc = _run(["--host-only"], 120)
    assert proc.returncode == 0, proc.stderr
    assert "failed checks" in proc.stdout and " 0 failed checks" in proc.stdout


@pytest.mark.gpu
def test_cpp_all_cases_on_gpu():
    proc = _run([], 300)
    assert proc.returncode == 0, proc.stderr
    assert " 0 failed checks" in proc.stdout


@pytest.mark.gpu
def test_random_eval_graphs_on_gpu():
    """800 seeded random sil::eval graphs (tests/cpp/random_graphs.cpp), every
    root against a float64 host shadow of the same nodes."""
    assert RANDOM_GRAPHS.exists(), f"{RANDOM_GRAPHS} not built: run __graft_entry__.build()"
    proc = subprocess.run([str(RANDOM_GRAPHS), "2026", "800"], capture_output=True, text=True,
                          timeout=300)
    print(proc.stdout[-4000:])
    print(proc.stderr[-4000:])
    assert proc.returncode == 0 and "800 graphs, 0 failures" in proc.stdout
