"""bench.py's command-line contract without a GPU: more than one GPU is
refused with a one-line JSON message and exit status 2 (the path runs no
collectives, so only the one-GPU figure exists), and a host without a visible
GPU gets a JSON error line and a non-zero status instead of a traceback."""
import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def _run(*args):
    res = subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True,
                         text=True, cwd=ROOT, timeout=300)
    lines = [ln for ln in res.stdout.splitlines() if ln.startswith("{")]
    return res.returncode, lines


@pytest.mark.parametrize("n", ["2", "8"])
def test_more_than_one_gpu_is_refused(n):
    rc, lines = _run("--gpus", n)
    assert rc == 2
    assert len(lines) == 1
    msg = json.loads(lines[0])
    assert "error" in msg and "--gpus must be 1" in msg["error"]


def test_no_visible_gpu_gives_a_json_error():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible here")
    rc, lines = _run("--steps", "1", "--warmup", "0", "--no-cpu-baseline")
    assert rc != 0
    assert len(lines) == 1 and "error" in json.loads(lines[0])
