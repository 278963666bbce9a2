"""bench.py's command-line contract, checked without a GPU."""

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_more_than_one_gpu_is_refused():
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                          capture_output=True, text=True, timeout=120)
    assert proc.returncode == 2
    assert "one GPU" in proc.stderr and proc.stdout == ""


def test_help_lists_the_contract_flags():
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--help"],
                          capture_output=True, text=True, timeout=120)
    assert proc.returncode == 0
    for flag in ("--gpus", "--steps", "--warmup"):
        assert flag in proc.stdout
