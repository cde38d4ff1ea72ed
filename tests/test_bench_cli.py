"""bench.py's command-line contract that holds without a GPU: more than one GPU is refused with a
message (the hot path is measured on one GPU), and a machine without a GPU gets a message and a
non-zero status instead of a traceback.  Also the paged prefill workload's byte and flop
bookkeeping on a case small enough to count by hand."""

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


def test_prefill_workload_counts_bytes_and_flops_by_hand() -> None:
    # Two rows with prefixes drawn from the generator (checked below), 64 new tokens in two 32-token
    # launches, 2 query heads over 1 KV head of dim 8, 16-token blocks.  Per launch and row: K/V of
    # the keys the chunk sees (2 x 1 x 8 bf16 = 32 B each), a 4-byte table entry per 16-key block,
    # and q, gate and out of the 32 new tokens (3 x 32 x 2 x 8 x 2 B = 3072 B).
    sys.path.insert(0, str(REPO))
    import bench

    w = bench.prefill_workload("cpu", batch=2, new=64, heads=2, kv_heads=1, dim=8, bs=16, max_prefix=40, chunk=32)
    prefixes = [int(p) for p in w["prefixes"]]
    expected_bytes = 0
    expected_flops = 0
    for p in prefixes:
        for c0 in (0, 32):
            keys = p + c0 + 32
            expected_bytes += keys * 32 + ((keys + 15) // 16) * 4 + 3072
        # causal: new token n sees p + n + 1 keys; 4 * heads * dim flop per (query, key)
        expected_flops += sum(4 * 2 * 8 * (p + n + 1) for n in range(64))
    assert w["launches"] == 2
    assert w["algo_bytes"] == expected_bytes
    assert w["flops"] == expected_flops
