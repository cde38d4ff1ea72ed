"""bench.py's command-line contract that holds without a GPU: more than one GPU is refused with a
message (the hot path is measured on one GPU), and a machine without a GPU gets a message and a
non-zero status instead of a traceback."""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent


def _bench(*args: str) -> subprocess.CompletedProcess:
    return subprocess.run([sys.executable, str(REPO / "bench.py"), *args], capture_output=True, text=True, timeout=300)


@pytest.mark.parametrize("gpus", ["2", "8"])
def test_more_than_one_gpu_is_refused_with_a_message(gpus: str) -> None:
    proc = _bench("--gpus", gpus)
    assert proc.returncode == 2
    assert "one GPU only" in proc.stderr and f"--gpus {gpus}" in proc.stderr
    assert proc.stdout.strip() == ""


def test_no_gpu_gives_a_message_not_a_traceback() -> None:
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    proc = _bench("--steps", "1", "--warmup", "0")
    assert proc.returncode == 2
    assert "needs a GPU" in proc.stderr and "Traceback" not in proc.stderr
