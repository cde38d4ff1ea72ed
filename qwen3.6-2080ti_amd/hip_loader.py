"""Loader of the gfx950 hot-path library (``build/libqwen36_hip.so``).

Replaces ``src/cuda_loader.py`` of the reference (``load_fp8_extension``,
``src/cuda_loader.py:40-54``): the library is a plain C-ABI shared object
loaded with ``ctypes`` instead of a pybind11 module.  As in the reference, a
missing build raises ``RuntimeError`` (``src/cuda_loader.py:46``) so callers
that catch it keep their fallback logic; there is no silent substitute.

``torch`` is imported before the library is opened so that the library's
``libamdhip64.so.7`` dependency resolves to the HIP runtime PyTorch already
loaded (same soname): device pointers and ``hipStream_t`` handles from torch
are then valid inside the library.
"""

from __future__ import annotations

import ctypes
from pathlib import Path
from typing import Any

PACKAGE_DIR = Path(__file__).resolve().parent
LIBRARY_PATH = PACKAGE_DIR / "build" / "libqwen36_hip.so"

_LIB: Any | None = None

QA_F32, QA_BF16, QA_F16, QA_I32, QA_I64 = 0, 1, 2, 3, 4

c_void_p = ctypes.c_void_p
c_int32 = ctypes.c_int32
c_int64 = ctypes.c_int64
c_float = ctypes.c_float


class PagedKV(ctypes.Structure):
    """Mirror of ``qa_paged_kv`` in ``include/qwen36_hip.h``."""

    _fields_ = [
        ("key", c_void_p),
        ("value", c_void_p),
        ("row_key_ptrs", c_void_p),
        ("row_value_ptrs", c_void_p),
        ("row_blocks", c_void_p),
        ("num_blocks", c_int64),
        ("stride_batch", c_int64),
        ("stride_block", c_int64),
        ("stride_head", c_int64),
        ("stride_token", c_int64),
        ("kv_heads", c_int32),
        ("dtype", c_int32),
    ]


# name -> (restype, argtypes); every symbol include/qwen36_hip.h declares.
SIGNATURES: dict[str, tuple[Any, list[Any]]] = {
    "qa_last_error": (ctypes.c_char_p, []),
    "qa_version": (c_int32, []),
    "qa_arch": (ctypes.c_char_p, []),
    "qa_set_kernel_timing": (None, [c_int32]),
    "qa_read_kernel_timing": (c_int32, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(c_int64)]),
    "qa_paged_attention_decode_workspace": (c_int64, [c_int64, c_int32, c_int32, c_int64, c_int32]),
    "qa_paged_attention_decode": (
        c_int32,
        [c_void_p, c_int32, c_int64, c_int64, c_int64, c_int32, c_int32, ctypes.POINTER(PagedKV), c_void_p, c_int32, c_int64,
         c_int64, c_int32, c_float, c_void_p, c_void_p, c_int64, c_void_p],
    ),
    "qa_paged_attention_decode_batched": (
        c_int32,
        [c_void_p, c_int32, c_int64, c_int64, c_int64, c_int32, c_int32, ctypes.POINTER(PagedKV), c_void_p, c_int32, c_int64,
         c_int64, c_void_p, c_int32, c_int32, c_float, c_void_p, c_void_p, c_int64, c_void_p],
    ),
    "qa_paged_attention_decode_batched_noalloc": (
        c_int32,
        [c_void_p, c_int32, c_int64, c_int64, c_int64, c_int32, c_int32, ctypes.POINTER(PagedKV), c_void_p, c_int32, c_int64,
         c_int64, c_void_p, c_int32, c_int32, c_float, c_void_p, c_void_p],
    ),
    "qa_paged_kv_append": (
        c_int32,
        [c_void_p, c_void_p, c_int32, c_int64, c_int64, c_int64, c_int64, c_int32, c_int64, c_int32, ctypes.POINTER(PagedKV),
         c_void_p, c_int32, c_int64, c_int64, c_void_p, c_int32, c_int64, c_void_p, c_int32, c_int32, c_void_p],
    ),
    "qa_qk_norm_rope_append": (
        c_int32,
        [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_int32, c_void_p, c_void_p, c_int32,
         c_float, c_void_p, c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_int32, c_int64, c_int64, c_int32, c_int32, ctypes.POINTER(PagedKV),
         c_void_p, c_int32, c_int64, c_int64, c_int32, c_void_p, c_void_p],
    ),
    "qa_fp8_linear_workspace": (c_int64, [c_int64, c_int64, c_int64]),
    "qa_fp8_pack_weight": (c_int32, [c_void_p, c_void_p, c_int64, c_int64, c_void_p]),
    "qa_fp8_linear": (
        c_int32,
        [c_void_p, c_int32, c_int64, c_int64, c_void_p, c_int32, c_void_p, c_int64, c_int64, c_void_p, c_int32, c_int64, c_void_p,
         c_int64, c_void_p],
    ),
    "qa_paged_kv_reserve": (
        c_int32,
        [c_void_p, c_int32, c_int64, c_int64, c_void_p, c_int32, c_void_p, c_int32, c_void_p, c_int32, c_int64, c_int64, c_int32,
         c_void_p, c_int64, c_void_p, c_void_p, c_void_p],
    ),
    "qa_paged_kv_gather": (
        c_int32,
        [ctypes.POINTER(PagedKV), c_int32, c_int64, c_void_p, c_int32, c_int64, c_int64, c_int64, c_int32, c_void_p, c_void_p,
         c_void_p],
    ),
    "qa_causal_conv1d_prefill": (
        c_int32,
        [c_void_p, c_int32, c_int64, c_int64, c_void_p, c_void_p, c_int64, c_void_p, c_int32, c_int64, c_void_p, c_int64, c_int64,
         c_int32, c_int32, c_void_p, c_int32, c_int64, c_int64, c_int32, c_void_p],
    ),
    "qa_causal_conv1d_update": (
        c_int32,
        [c_void_p, c_int32, c_int64, c_void_p, c_int64, c_void_p, c_int32, c_int64, c_void_p, c_int64, c_int32, c_int32, c_void_p,
         c_int32, c_int64, c_int32, c_void_p],
    ),
    "qa_linear_attention_recurrent_core": (
        c_int32,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int32, c_int64, c_int32, c_int32,
         c_void_p],
    ),
    "qa_gated_delta_step": (
        c_int32,
        [c_void_p, c_int64, c_void_p, c_void_p, c_int32, c_int64, c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_int32, c_int64,
         c_void_p, c_int32, c_int64, c_int64, c_int32, c_int32, c_int32, c_int32, c_void_p],
    ),
    "qa_gated_delta_step_norm": (
        c_int32,
        [c_void_p, c_int64, c_void_p, c_void_p, c_int32, c_int64, c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_int32, c_int64,
         c_void_p, c_int32, c_int64, c_void_p, c_int32, c_float, c_void_p, c_int32, c_int64, c_int64, c_int32, c_int32, c_int32, c_int32,
         c_void_p],
    ),
    "qa_gated_delta_step_conv": (
        c_int32,
        [c_void_p, c_int32, c_int64, c_void_p, c_int64, c_void_p, c_int32, c_void_p, c_void_p, c_int32, c_int64, c_void_p, c_void_p,
         c_void_p, c_int64, c_void_p, c_int32, c_int64, c_void_p, c_int32, c_int64, c_void_p, c_int32, c_float, c_void_p, c_int32, c_int64,
         c_int64, c_int32, c_int32, c_int32, c_int32, c_void_p],
    ),
    "qa_gated_rms_norm": (
        c_int32,
        [c_void_p, c_int32, c_int64, c_int64, c_void_p, c_int32, c_int64, c_int64, c_void_p, c_int32, c_float, c_int64, c_int32, c_int32,
         c_void_p, c_int32, c_int64, c_int64, c_void_p],
    ),
    "qa_chunk_gated_delta_rule": (
        c_int32,
        [c_void_p, c_int32, c_int64, c_int64, c_void_p, c_void_p, c_int32, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p,
         c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int64, c_int64, c_int64, c_int64, c_int32, c_int32, c_int32, c_int32,
         c_int32, c_void_p, c_int64, c_void_p],
    ),
    "qa_chunk_gated_delta_workspace": (c_int64, [c_int64, c_int64, c_int32, c_int32]),
    "qa_chunk_gated_delta_lds_bytes": (c_int64, []),
    "qa_paged_attention_prefill": (
        c_int32,
        [c_void_p, c_int32, c_int64, c_int64, c_void_p, c_void_p, c_int32, c_int64, c_int64, c_int32, c_int32, ctypes.POINTER(PagedKV),
         c_void_p, c_int32, c_int64, c_int64, c_int32, c_float, c_void_p, c_int64, c_int64, c_void_p, c_void_p],
    ),
}


class NativeLibraryMissing(RuntimeError):
    """The HIP library is not built or cannot be opened.  Never caught by a fallback."""


def load_library() -> Any:
    """Open (once) and return the ctypes handle; :class:`NativeLibraryMissing` if not built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIBRARY_PATH.exists():
        raise NativeLibraryMissing(f"qwen36 HIP library is not built ({LIBRARY_PATH}); run `python build_native.py`")
    import torch  # noqa: F401  -- binds libamdhip64.so.7 to torch's HIP runtime first

    try:
        lib = ctypes.CDLL(str(LIBRARY_PATH), mode=ctypes.RTLD_GLOBAL)
    except OSError as exc:
        raise NativeLibraryMissing(f"cannot open {LIBRARY_PATH}: {exc}") from exc
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _LIB = lib
    return lib


def last_error(lib: Any) -> str:
    message = lib.qa_last_error()
    return message.decode() if message else "unknown error"


def check(lib: Any, status: int, what: str) -> None:
    if status != 0:
        raise RuntimeError(f"{what}: {last_error(lib)}")


class KernelTiming:
    """Context manager around the library's opt-in kernel timer.

    ``with KernelTiming() as t: ...`` then ``t.read("decode_partial_mfma")``
    returns ``(total_ms, launches)`` of that kernel inside the block.
    """

    def __enter__(self) -> "KernelTiming":
        self._lib = load_library()
        self._lib.qa_set_kernel_timing(1)
        return self

    def read(self, label: str) -> tuple[float, int]:
        total = ctypes.c_double(0.0)
        count = c_int64(0)
        self._lib.qa_read_kernel_timing(label.encode(), ctypes.byref(total), ctypes.byref(count))
        return float(total.value), int(count.value)

    def __exit__(self, *exc: object) -> None:
        self._lib.qa_set_kernel_timing(0)
