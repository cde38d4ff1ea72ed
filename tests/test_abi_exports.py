"""The C-ABI library loads without a GPU and exports every symbol the header declares."""

from __future__ import annotations

import re
import subprocess
from pathlib import Path

import pytest

import hip_loader

HEADER_DIR = Path(__file__).resolve().parents[1] / "include"


def _declared_symbols() -> set[str]:
    names: set[str] = set()
    for header in HEADER_DIR.glob("*.h"):
        text = header.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for match in re.finditer(r"\b(qa_[a-z0-9_]+)\s*\(", text):
            names.add(match.group(1))
    return names


def _library() -> Path:
    if not hip_loader.LIBRARY_PATH.exists():
        pytest.fail(f"{hip_loader.LIBRARY_PATH} is not built; run __graft_entry__.build()")
    return hip_loader.LIBRARY_PATH


def test_header_declares_the_expected_entry_points() -> None:
    declared = _declared_symbols()
    for name in ("qa_paged_attention_decode", "qa_paged_attention_decode_batched", "qa_paged_kv_append", "qa_paged_kv_gather", "qa_last_error"):
        assert name in declared


def test_library_exports_every_declared_symbol() -> None:
    out = subprocess.run(["nm", "-D", "--defined-only", str(_library())], capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = sorted(_declared_symbols() - exported)
    assert not missing, f"declared but not exported: {missing}"


def test_loader_binds_every_declared_symbol_and_reports_arch() -> None:
    _library()
    lib = hip_loader.load_library()
    assert set(hip_loader.SIGNATURES) == _declared_symbols()
    assert lib.qa_arch() == b"gfx950"
    assert lib.qa_version() >= 1


def test_host_validation_errors_need_no_gpu() -> None:
    _library()
    lib = hip_loader.load_library()
    desc = hip_loader.PagedKV()
    desc.kv_heads = 2
    desc.dtype = hip_loader.QA_BF16
    import ctypes

    status = lib.qa_paged_attention_decode(
        ctypes.c_void_p(8), hip_loader.QA_F16, 0, 0, 1, 16, 256, ctypes.byref(desc), ctypes.c_void_p(8), hip_loader.QA_I32, 1, 1, 16, 0.0,
        ctypes.c_void_p(8), ctypes.c_void_p(8), 1 << 20, ctypes.c_void_p(0),
    )
    assert status != 0
    assert "query must be float32" in hip_loader.last_error(lib)
    assert lib.qa_paged_attention_decode_workspace(64, 16, 256, 32768, 16) > 0


def test_kernel_timing_reads_zero_without_launches() -> None:
    _library()
    lib = hip_loader.load_library()
    import ctypes

    lib.qa_set_kernel_timing(1)
    total, launches = ctypes.c_double(-1.0), ctypes.c_int64(-1)
    assert lib.qa_read_kernel_timing(b"decode_partial_mfma", ctypes.byref(total), ctypes.byref(launches)) == 0
    lib.qa_set_kernel_timing(0)
    assert total.value == 0.0 and launches.value == 0
