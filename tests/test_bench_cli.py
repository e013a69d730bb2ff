"""bench.py's command-line contract on the CPU: more than one GPU is refused
with a message and exit status 2 before anything touches torch or the
device (this build measures one GPU)."""

import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


@pytest.mark.parametrize("n", [2, 8])
def test_more_than_one_gpu_is_refused(n):
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", str(n), "--steps", "1", "--warmup", "0"],
                       capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    assert f"--gpus {n}" in r.stderr and "one GPU" in r.stderr
    assert r.stdout == ""  # no JSON line
