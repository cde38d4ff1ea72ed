"""Python operator surface of the gfx950 hot path.

The names, arguments, return shapes and ``RuntimeError`` behaviour of the three
hot wrappers of the reference's ``src/fp8_cuda.py`` are kept:

* :func:`paged_attention_decode` -- ``src/fp8_cuda.py:217-232``
* :func:`paged_attention_decode_batched` -- ``src/fp8_cuda.py:235-250``
* :func:`linear_attention_recurrent_core` -- ``src/fp8_cuda.py:206-214``

so a caller such as ``src/tp_runtime.py:613-643`` / ``:2778-2787`` only changes
its import.  Beyond the reference they also accept bfloat16 tensors, a shared
GQA-native block pool ``(P, H_kv, bs, D)`` and int32 tables.  New operators of
the path sit beside them (KV append/gather, prefill, conv1d, chunked delta
rule, fused decode step).

Every operator validates on the host and raises ``RuntimeError`` with the
library's message on failure.  Outputs and workspaces are allocated here with
torch (its caching allocator owns them); kernels run on torch's current stream.
"""

from __future__ import annotations

import ctypes
from typing import Any, Sequence

import torch

import hip_loader as L

_DTYPE_CODES = {
    torch.float32: L.QA_F32,
    torch.bfloat16: L.QA_BF16,
    torch.float16: L.QA_F16,
    torch.int32: L.QA_I32,
    torch.int64: L.QA_I64,
}


def _code(tensor: torch.Tensor) -> int:
    try:
        return _DTYPE_CODES[tensor.dtype]
    except KeyError as exc:
        raise RuntimeError(f"unsupported dtype {tensor.dtype}") from exc


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _ptr(tensor: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if tensor is None else tensor.data_ptr())


def _require(cond: bool, message: str) -> None:
    if not cond:
        raise RuntimeError(message)


def _require_cuda(tensor: Any, name: str, device: torch.device | None = None) -> None:
    _require(isinstance(tensor, torch.Tensor) and tensor.is_cuda, f"{name} must be CUDA")
    if device is not None:
        _require(tensor.device == device, f"{name} must be on same CUDA device as query")


def _float_dtype(tensor: torch.Tensor, name: str) -> None:
    _require(tensor.dtype in (torch.float32, torch.bfloat16), f"{name} must be float32 or bfloat16")


def _index_dtype(tensor: torch.Tensor, name: str) -> None:
    _require(tensor.dtype in (torch.int32, torch.int64), f"{name} must be int64/torch.long or int32")


def _pool_descriptor(key_pool: torch.Tensor, value_pool: torch.Tensor, layout: str) -> L.PagedKV:
    """Descriptor for a reference-layout ``(B, heads, P, bs, D)`` pool or a shared ``(P, H_kv, bs, D)`` pool."""
    _require(key_pool.shape == value_pool.shape, "key/value physical block count must match")
    _require(key_pool.dtype == value_pool.dtype, "key/value blocks must have the same dtype")
    _require(key_pool.stride(-1) == 1 and value_pool.stride(-1) == 1, "key/value blocks must be contiguous in head_dim")
    _require(key_pool.stride() == value_pool.stride(), "key/value blocks must share strides")
    desc = L.PagedKV()
    desc.key = key_pool.data_ptr()
    desc.value = value_pool.data_ptr()
    desc.row_key_ptrs = None
    desc.row_value_ptrs = None
    desc.row_blocks = None
    desc.dtype = _code(key_pool)
    if layout == "reference":  # (B, heads, P, bs, D)
        desc.num_blocks = key_pool.shape[2]
        desc.stride_batch = key_pool.stride(0)
        desc.stride_head = key_pool.stride(1)
        desc.stride_block = key_pool.stride(2)
        desc.stride_token = key_pool.stride(3)
        desc.kv_heads = key_pool.shape[1]
    else:  # shared (P, H_kv, bs, D)
        desc.num_blocks = key_pool.shape[0]
        desc.stride_batch = 0
        desc.stride_block = key_pool.stride(0)
        desc.stride_head = key_pool.stride(1)
        desc.stride_token = key_pool.stride(2)
        desc.kv_heads = key_pool.shape[1]
    return desc


def _decode_workspace(lib: Any, batch: int, heads: int, head_dim: int, max_tokens: int, block_size: int, device: torch.device) -> torch.Tensor:
    nbytes = int(lib.qa_paged_attention_decode_workspace(batch, heads, head_dim, max_tokens, block_size))
    return torch.empty(max(nbytes, 4), dtype=torch.uint8, device=device)


def paged_attention_decode(
    query: torch.Tensor,
    block_table: torch.Tensor,
    key_blocks: torch.Tensor,
    value_blocks: torch.Tensor,
    sequence_length: int,
    block_size: int,
    *,
    scale: float | None = None,
) -> torch.Tensor:
    """Single-token paged attention over one block table.

    ``query`` ``(B, H, 1, D)``; ``block_table`` ``(L,)``; ``key_blocks`` either
    the reference's per-request pool ``(B, heads, P, bs, D)`` with ``heads`` = H
    or H_kv (GQA), or a shared pool ``(P, H_kv, bs, D)``.  Returns
    ``(B, H, 1, D)`` in the query dtype.  Reference:
    ``src/fp8_cuda.py:217-232`` -> ``src/csrc/fp8_linear_cuda.cu:1192-1266``.
    """
    lib = L.load_library()
    _require_cuda(query, "query")
    device = query.device
    _require_cuda(block_table, "block_table", device)
    _require_cuda(key_blocks, "key_blocks", device)
    _require_cuda(value_blocks, "value_blocks", device)
    _float_dtype(query, "query")
    _float_dtype(key_blocks, "key_blocks")
    _index_dtype(block_table, "block_table")
    _require(query.dim() == 4, "query must have shape [batch, heads, 1, head_dim]")
    _require(query.shape[2] == 1, "query seq_len must be 1 for paged decode")
    _require(block_table.dim() == 1, "block_table must be rank-1")
    _require(key_blocks.dim() in (4, 5), "key_blocks must have shape [batch, heads, blocks, block_size, head_dim] or [blocks, kv_heads, block_size, head_dim]")
    _require(value_blocks.dim() == key_blocks.dim(), "value_blocks must match key_blocks rank")
    _require(int(sequence_length) > 0, "sequence_length must be positive")
    _require(int(block_size) > 0, "block_size must be positive")
    batch, heads, _, head_dim = query.shape
    layout = "reference" if key_blocks.dim() == 5 else "shared"
    if layout == "reference":
        _require(key_blocks.shape[0] == batch and value_blocks.shape[0] == batch, "KV batch must match query")
    _require(key_blocks.shape[-2] == block_size, "KV block_size mismatch")
    _require(key_blocks.shape[-1] == head_dim, "KV head_dim must match query")
    table = block_table.contiguous()
    _require(table.numel() * int(block_size) >= int(sequence_length), "block_table does not cover sequence_length")
    q = query.contiguous()
    desc = _pool_descriptor(key_blocks, value_blocks, layout)
    _require(heads % desc.kv_heads == 0, "KV heads must divide query heads")
    out = torch.empty_like(q)
    ws = _decode_workspace(lib, batch, heads, head_dim, int(sequence_length), int(block_size), device)
    status = lib.qa_paged_attention_decode(
        _ptr(q), _code(q), q.stride(0), q.stride(1), batch, heads, head_dim, ctypes.byref(desc), _ptr(table), _code(table),
        table.numel(), int(sequence_length), int(block_size), float(scale or 0.0), _ptr(out), _ptr(ws), ws.numel(), _stream(device),
    )
    L.check(lib, status, "paged_attention_decode")
    return out


def paged_attention_decode_batched(
    query: torch.Tensor,
    block_tables: torch.Tensor,
    key_blocks: Sequence[torch.Tensor] | torch.Tensor,
    value_blocks: Sequence[torch.Tensor] | torch.Tensor,
    sequence_lengths: torch.Tensor,
    block_size: int,
    *,
    scale: float | None = None,
) -> torch.Tensor:
    """Batched single-token paged attention with per-row tables and lengths.

    ``block_tables`` ``(B, max_blocks)`` padded with -1, ``sequence_lengths``
    ``(B,)``.  ``key_blocks``/``value_blocks`` are either one shared
    ``(P, H_kv, bs, D)`` pool, or (as the reference) a list of per-request
    pools ``(1, heads, P_b, bs, D)``; a list whose entries are all the same
    tensor is treated as one shared pool.  Rows of length <= 0 give zeros.
    Reference: ``src/fp8_cuda.py:235-250`` -> ``src/csrc/fp8_linear_cuda.cu:1269-1365``.
    """
    lib = L.load_library()
    _require_cuda(query, "query")
    device = query.device
    _require_cuda(block_tables, "block_tables", device)
    _require_cuda(sequence_lengths, "sequence_lengths", device)
    _float_dtype(query, "query")
    _index_dtype(block_tables, "block_tables")
    _index_dtype(sequence_lengths, "sequence_lengths")
    _require(query.dim() == 4, "query must have shape [batch, heads, 1, head_dim]")
    _require(block_tables.dim() == 2, "block_tables must have shape [batch, max_blocks]")
    _require(sequence_lengths.dim() == 1, "sequence_lengths must be rank-1")
    _require(query.shape[2] == 1, "query seq_len must be 1 for paged decode")
    _require(int(block_size) > 0, "block_size must be positive")
    batch, heads, _, head_dim = query.shape
    _require(block_tables.shape[0] == batch, "block_tables batch must match query")
    _require(sequence_lengths.shape[0] == batch, "sequence_lengths batch must match query")
    _require(block_tables.shape[1] > 0, "max_blocks must be positive and fit int32")
    keepalive: list[torch.Tensor] = []
    if isinstance(key_blocks, torch.Tensor):
        _require(isinstance(value_blocks, torch.Tensor), "value_blocks must match key_blocks")
        _require(key_blocks.dim() == 4, "shared pools must have shape [blocks, kv_heads, block_size, head_dim]")
        _require_cuda(key_blocks, "key_blocks", device)
        _require_cuda(value_blocks, "value_blocks", device)
        _float_dtype(key_blocks, "key_blocks")
        desc = _pool_descriptor(key_blocks, value_blocks, "shared")
        pool_block_size = key_blocks.shape[2]
    else:
        key_list = list(key_blocks)
        value_list = list(value_blocks)
        _require(len(key_list) == batch, "key_blocks list length must match batch")
        _require(len(value_list) == batch, "value_blocks list length must match batch")
        first_k, first_v = key_list[0], value_list[0]
        for k, v in zip(key_list, value_list):
            _require(isinstance(k, torch.Tensor) and isinstance(v, torch.Tensor), "key/value blocks must be CUDA")
            _require(k.is_cuda and v.is_cuda, "key/value blocks must be CUDA")
            _require(k.device == device and v.device == device, "key/value blocks must be on same CUDA device as query")
            _require(k.dtype == first_k.dtype and v.dtype == first_k.dtype, "key/value blocks must share one dtype")
            _float_dtype(k, "key/value blocks")
            _require(k.dim() == first_k.dim() and v.dim() == first_k.dim(), "key/value blocks must share one rank")
            _require(k.shape == v.shape, "key/value physical block count must match")
        shared = all(k is first_k for k in key_list) and all(v is first_v for v in value_list)
        if shared and first_k.dim() == 4:
            desc = _pool_descriptor(first_k, first_v, "shared")
            pool_block_size = first_k.shape[2]
        else:
            for k in key_list:
                _require(k.dim() == 5, "key/value blocks must have shape [1, heads, blocks, block_size, head_dim]")
                _require(k.shape[0] == 1, "per-request KV pools must have batch dim 1")
                _require(k.shape[1] == first_k.shape[1], "KV heads must match across pools")
                _require(k.shape[3:] == first_k.shape[3:], "KV block_size/head_dim must match across pools")
                _require(k.stride(-1) == 1 and k.is_contiguous(), "key/value blocks must be contiguous")
            for v in value_list:
                _require(v.is_contiguous(), "key/value blocks must be contiguous")
            desc = _per_request_descriptor(key_list, value_list, device, keepalive)
            pool_block_size = first_k.shape[3]
    _require(pool_block_size == block_size, "KV block_size mismatch")
    _require(heads % desc.kv_heads == 0, "KV heads must divide query heads")
    q = query.contiguous()
    tables = block_tables.contiguous()
    lens = sequence_lengths.contiguous()
    max_blocks = tables.shape[1]
    out = torch.empty_like(q)
    ws = _decode_workspace(lib, batch, heads, head_dim, max_blocks * int(block_size), int(block_size), device)
    status = lib.qa_paged_attention_decode_batched(
        _ptr(q), _code(q), q.stride(0), q.stride(1), batch, heads, head_dim, ctypes.byref(desc), _ptr(tables), _code(tables),
        tables.stride(0), max_blocks, _ptr(lens), _code(lens), int(block_size), float(scale or 0.0), _ptr(out), _ptr(ws), ws.numel(),
        _stream(device),
    )
    L.check(lib, status, "paged_attention_decode_batched")
    return out


def paged_attention_decode_batched_noalloc(
    query: torch.Tensor,
    block_tables: torch.Tensor,
    key_blocks: torch.Tensor,
    value_blocks: torch.Tensor,
    sequence_lengths: torch.Tensor,
    block_size: int,
    *,
    scale: float | None = None,
) -> torch.Tensor:
    """``paged_attention_decode_batched`` on one shared ``(P, H_kv, bs, D)`` pool with the split-K
    partials in the library's static per-device scratch (``qa_paged_attention_decode_batched_noalloc``):
    the library allocates nothing; only the output is a new tensor.  Sizes whose partials exceed the
    scratch raise ``RuntimeError``; calls that overlap on one device race."""
    lib = L.load_library()
    _require_cuda(query, "query")
    device = query.device
    for tensor, name in ((block_tables, "block_tables"), (sequence_lengths, "sequence_lengths"), (key_blocks, "key_blocks"),
                         (value_blocks, "value_blocks")):
        _require_cuda(tensor, name, device)
    _float_dtype(query, "query")
    _float_dtype(key_blocks, "key_blocks")
    _index_dtype(block_tables, "block_tables")
    _index_dtype(sequence_lengths, "sequence_lengths")
    _require(query.dim() == 4 and query.shape[2] == 1, "query must have shape [batch, heads, 1, head_dim]")
    _require(key_blocks.dim() == 4 and value_blocks.shape == key_blocks.shape, "shared pools must have shape [blocks, kv_heads, block_size, head_dim]")
    batch, heads, _, head_dim = query.shape
    _require(block_tables.dim() == 2 and block_tables.shape[0] == batch and block_tables.shape[1] > 0, "block_tables must have shape [batch, max_blocks]")
    _require(sequence_lengths.dim() == 1 and sequence_lengths.shape[0] == batch, "sequence_lengths batch must match query")
    _require(key_blocks.shape[2] == block_size, "KV block_size mismatch")
    desc = _pool_descriptor(key_blocks, value_blocks, "shared")
    _require(heads % desc.kv_heads == 0, "KV heads must divide query heads")
    q = query.contiguous()
    tables = block_tables.contiguous()
    lens = sequence_lengths.contiguous()
    out = torch.empty_like(q)
    status = lib.qa_paged_attention_decode_batched_noalloc(
        _ptr(q), _code(q), q.stride(0), q.stride(1), batch, heads, head_dim, ctypes.byref(desc), _ptr(tables), _code(tables),
        tables.stride(0), tables.shape[1], _ptr(lens), _code(lens), int(block_size), float(scale or 0.0), _ptr(out), _stream(device),
    )
    L.check(lib, status, "paged_attention_decode_batched_noalloc")
    return out


def _per_request_descriptor(key_list: list[torch.Tensor], value_list: list[torch.Tensor], device: torch.device, keepalive: list[torch.Tensor]) -> L.PagedKV:
    """Pointer-array descriptor for contiguous per-request pools ``(1, heads, P_b, bs, D)``.

    As the reference host wrapper (``src/csrc/fp8_linear_cuda.cu:1308-1340``),
    row pointers and block counts are copied to the device for each call.
    ``stride_head = 0`` tells the kernels that row ``b``'s head stride is
    ``P_b * stride_block`` (pools of different ``P_b``).
    """
    first = key_list[0]
    key_ptrs = torch.tensor([k.data_ptr() for k in key_list], dtype=torch.int64, device=device)
    value_ptrs = torch.tensor([v.data_ptr() for v in value_list], dtype=torch.int64, device=device)
    counts = torch.tensor([k.shape[2] for k in key_list], dtype=torch.int64, device=device)
    keepalive.extend([key_ptrs, value_ptrs, counts])
    desc = L.PagedKV()
    desc.key = None
    desc.value = None
    desc.row_key_ptrs = key_ptrs.data_ptr()
    desc.row_value_ptrs = value_ptrs.data_ptr()
    desc.row_blocks = counts.data_ptr()
    desc.num_blocks = max(k.shape[2] for k in key_list)
    desc.stride_batch = 0
    desc.stride_head = 0
    desc.stride_block = first.stride(2)
    desc.stride_token = first.stride(3)
    desc.kv_heads = first.shape[1]
    desc.dtype = _code(first)
    return desc


def paged_kv_append(
    key: torch.Tensor,
    value: torch.Tensor,
    key_pool: torch.Tensor,
    value_pool: torch.Tensor,
    block_tables: torch.Tensor,
    starts: torch.Tensor | int,
    block_size: int,
    *,
    counts: torch.Tensor | None = None,
) -> None:
    """Write new K/V ``(B, H_kv, S, D)`` into pool slots in place (bit-exact).

    Row ``b`` token ``s`` goes to slot ``(table[b][(start_b+s)//bs], (start_b+s)%bs)``
    of the shared pool ``(P, H_kv, bs, D)`` or of the reference-layout pool
    ``(B, heads, P, bs, D)``.  ``block_tables`` is ``(B, max_blocks)`` or a single
    ``(max_blocks,)`` table shared by all rows.  Replaces the fragment loop of
    ``FullAttentionCache.append_blocks`` (``src/decode_state.py:271-293``).
    """
    lib = L.load_library()
    _require_cuda(key, "key")
    device = key.device
    for tensor, name in ((value, "value"), (key_pool, "key_pool"), (value_pool, "value_pool"), (block_tables, "block_tables")):
        _require_cuda(tensor, name, device)
    _require(key.shape == value.shape and key.dim() == 4, "key/value must have shape [batch, kv_heads, seq, head_dim]")
    _require(key.dtype == key_pool.dtype and value.dtype == key_pool.dtype, "new KV dtype must match the pool dtype")
    _require(key.stride() == value.stride() and key.stride(-1) == 1, "key/value must share strides with a contiguous head_dim")
    _index_dtype(block_tables, "block_tables")
    layout = "reference" if key_pool.dim() == 5 else "shared"
    desc = _pool_descriptor(key_pool, value_pool, layout)
    batch, kv_heads, seq, head_dim = key.shape
    _require(kv_heads == desc.kv_heads, "new KV heads must match the pool")
    _require(key_pool.shape[-1] == head_dim and key_pool.shape[-2] == block_size, "pool block_size/head_dim mismatch")
    tables = block_tables.contiguous()
    table_stride = tables.stride(0) if tables.dim() == 2 else 0
    max_blocks = tables.shape[-1]
    start_ptr, start_code, start_scalar = ctypes.c_void_p(0), L.QA_I64, 0
    if isinstance(starts, torch.Tensor):
        _require_cuda(starts, "starts", device)
        _index_dtype(starts, "starts")
        starts = starts.contiguous()
        start_ptr, start_code = _ptr(starts), _code(starts)
    else:
        start_scalar = int(starts)
    count_ptr, count_code = ctypes.c_void_p(0), L.QA_I64
    if counts is not None:
        _require_cuda(counts, "counts", device)
        _index_dtype(counts, "counts")
        counts = counts.contiguous()
        count_ptr, count_code = _ptr(counts), _code(counts)
    status = lib.qa_paged_kv_append(
        _ptr(key), _ptr(value), _code(key), key.stride(0), key.stride(1), key.stride(2), batch, kv_heads, seq, head_dim,
        ctypes.byref(desc), _ptr(tables), _code(tables), table_stride, max_blocks, start_ptr, start_code, start_scalar,
        count_ptr, count_code, int(block_size), _stream(device),
    )
    L.check(lib, status, "paged_kv_append")


def paged_kv_reserve(
    block_tables: torch.Tensor,
    lengths: torch.Tensor,
    free_list: torch.Tensor,
    free_state: torch.Tensor,
    status: torch.Tensor,
    block_size: int,
    *,
    counts: torch.Tensor | int = 1,
    positions: torch.Tensor | None = None,
) -> None:
    """Reserve the blocks a batched step needs, on the device (no host round trip).

    Row ``b`` grows from ``lengths[b]`` to ``lengths[b] + counts_b`` tokens: its new
    logical blocks get ids from the head of the ascending ``free_list`` (int32),
    rows in order -- the reference's lowest-free-id policy
    (``src/decode_state.py:72-78``).  ``free_state`` (int32 ``[head, count]``) is
    advanced, ``lengths`` are advanced in place, ``positions`` (if given) receives
    the old lengths.  ``status`` (int32 ``[1]``) becomes 0, or 1 (pool exhausted),
    2 (a table row too short), 3 (corrupt free state), 4 (negative or overflowing
    length or count), in which case nothing else is written.  Every argument is a
    device tensor and nothing is read back, so the call can be captured in a HIP graph.
    """
    lib = L.load_library()
    _require_cuda(block_tables, "block_tables")
    device = block_tables.device
    for tensor, name in ((lengths, "lengths"), (free_list, "free_list"), (free_state, "free_state"), (status, "status")):
        _require_cuda(tensor, name, device)
    _index_dtype(block_tables, "block_tables")
    _index_dtype(lengths, "lengths")
    _require(block_tables.dim() == 2 and block_tables.stride(1) == 1, "block_tables must have shape [batch, max_blocks] with contiguous rows")
    _require(lengths.dim() == 1 and lengths.is_contiguous() and lengths.shape[0] == block_tables.shape[0], "lengths must be a contiguous [batch] tensor")
    _require(free_list.dtype == torch.int32 and free_list.dim() == 1 and free_list.is_contiguous(), "free_list must be a contiguous int32 vector")
    _require(free_state.dtype == torch.int32 and free_state.numel() == 2 and free_state.is_contiguous(), "free_state must be int32 [head, count]")
    _require(status.dtype == torch.int32 and status.numel() >= 1, "status must be an int32 tensor")
    count_ptr, count_code, count_scalar = ctypes.c_void_p(0), L.QA_I64, 0
    if isinstance(counts, torch.Tensor):
        _require_cuda(counts, "counts", device)
        _index_dtype(counts, "counts")
        _require(counts.dim() == 1 and counts.is_contiguous() and counts.shape[0] == lengths.shape[0], "counts must be a contiguous [batch] tensor")
        count_ptr, count_code = _ptr(counts), _code(counts)
    else:
        count_scalar = int(counts)
        _require(count_scalar >= 0, "counts must be non-negative")
    pos_ptr, pos_code = ctypes.c_void_p(0), L.QA_I64
    if positions is not None:
        _require_cuda(positions, "positions", device)
        _index_dtype(positions, "positions")
        _require(positions.dim() == 1 and positions.is_contiguous() and positions.shape[0] == lengths.shape[0], "positions must be a contiguous [batch] tensor")
        pos_ptr, pos_code = _ptr(positions), _code(positions)
    status_code = lib.qa_paged_kv_reserve(
        _ptr(block_tables), _code(block_tables), block_tables.stride(0), block_tables.shape[1], _ptr(lengths), _code(lengths),
        pos_ptr, pos_code, count_ptr, count_code, count_scalar, lengths.shape[0], int(block_size), _ptr(free_list),
        free_list.numel(), _ptr(free_state), _ptr(status), _stream(device),
    )
    L.check(lib, status_code, "paged_kv_reserve")


class PackedFp8Weight:
    """An fp8 E4M3 weight re-laid by ``fp8_pack_weight`` (same bytes, streaming order)."""

    def __init__(self, data: torch.Tensor, out_features: int, in_features: int) -> None:
        self.data = data
        self.shape = (out_features, in_features)
        self.device = data.device


def fp8_pack_weight(weight: torch.Tensor) -> PackedFp8Weight:
    """Re-lay an ``(N, K)`` fp8 weight once (at load time) into 16 x 128 tiles of 2 KB, consecutive
    along K, in the order the linear kernel reads them: each wave then streams contiguous memory.
    No counterpart in the reference, whose weights stay row-major."""
    lib = L.load_library()
    _require_cuda(weight, "weight")
    _require(weight.dtype in (torch.float8_e4m3fn, torch.uint8) and weight.dim() == 2, "weight must be a rank-2 torch.float8_e4m3fn tensor")
    rows, cols = weight.shape
    _require(rows % 128 == 0 and cols % 128 == 0, "weight rows and cols must be divisible by 128 for the FP8 op")
    src = weight.contiguous()
    dst = torch.empty((rows * cols,), dtype=torch.uint8, device=weight.device)
    L.check(lib, lib.qa_fp8_pack_weight(_ptr(src), _ptr(dst), rows, cols, _stream(weight.device)), "fp8_pack_weight")
    return PackedFp8Weight(dst, rows, cols)


def fp8_e4m3_bf16_linear(input: torch.Tensor, weight: torch.Tensor | PackedFp8Weight, scale: torch.Tensor, *, out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """``y = input @ (E4M3(weight) * block scale)^T`` with 128 x 128 bf16 scale blocks.

    Same name, arguments and result as the reference's ``fp8_cuda.fp8_e4m3_bf16_linear``
    (``src/fp8_cuda.py:16-17`` -> ``src/csrc/fp8_linear_cuda.cu:1368-1466``): ``weight``
    ``(N, K)`` ``torch.float8_e4m3fn`` (or its uint8 codes), ``scale`` ``(N/128, K/128)``
    bf16, ``input`` ``(..., K)`` float32 (bf16 also accepted); returns ``(..., N)`` float32
    (or ``out_dtype`` bf16).  N and K must be multiples of 128, as in the reference's op.
    ``weight`` may also be the ``fp8_pack_weight`` form of the same weight (faster streaming).
    """
    lib = L.load_library()
    _require_cuda(input, "input")
    device = input.device
    _require_cuda(weight.data if isinstance(weight, PackedFp8Weight) else weight, "weight", device)
    _require_cuda(scale, "scale", device)
    _require(input.dtype in (torch.float32, torch.bfloat16), "input must be float32 or bfloat16")
    packed = isinstance(weight, PackedFp8Weight)
    _require(packed or weight.dtype in (torch.float8_e4m3fn, torch.uint8), "weight must be torch.float8_e4m3fn")
    _require(scale.dtype == torch.bfloat16, "scale must be bfloat16")
    _require(packed or weight.dim() == 2, "weight must be rank-2")
    _require(scale.dim() == 2, "scale must be rank-2")
    _require(input.dim() >= 2, "input must be at least rank-2")
    _require(out_dtype in (torch.float32, torch.bfloat16), "out_dtype must be float32 or bfloat16")
    rows, cols = weight.shape
    _require(input.shape[-1] == cols, "input last dim must match weight cols")
    _require(rows % 128 == 0, "weight rows must be divisible by 128 for the FP8 op")
    _require(cols % 128 == 0, "weight cols must be divisible by 128 for the FP8 op")
    _require(tuple(scale.shape) == (rows // 128, cols // 128), "scale blocks mismatch")
    x = input.contiguous().view(-1, cols)
    w = weight.data if packed else weight.contiguous()
    s = scale.contiguous()
    out = torch.empty((x.shape[0], rows), dtype=out_dtype, device=device)
    nbytes = int(lib.qa_fp8_linear_workspace(x.shape[0], rows, cols))
    ws = torch.empty(max(nbytes, 4), dtype=torch.uint8, device=device)
    status = lib.qa_fp8_linear(
        _ptr(x), _code(x), x.stride(0), x.shape[0], _ptr(w), int(packed), _ptr(s), rows, cols, _ptr(out), _code(out), out.stride(0), _ptr(ws),
        ws.numel(), _stream(device),
    )
    L.check(lib, status, "fp8_e4m3_bf16_linear")
    return out.view(*input.shape[:-1], rows)


def paged_kv_gather(key_pool: torch.Tensor, value_pool: torch.Tensor, block_tables: torch.Tensor, valid: int, block_size: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Dense ``(B, H_kv, valid, D)`` logical-order K/V (``src/decode_state.py:295-303,395-404``)."""
    lib = L.load_library()
    _require_cuda(key_pool, "key_pool")
    device = key_pool.device
    _require_cuda(value_pool, "value_pool", device)
    _require_cuda(block_tables, "block_tables", device)
    _index_dtype(block_tables, "block_tables")
    layout = "reference" if key_pool.dim() == 5 else "shared"
    desc = _pool_descriptor(key_pool, value_pool, layout)
    tables = block_tables.contiguous()
    if tables.dim() == 1:
        tables = tables.unsqueeze(0)
    batch = tables.shape[0] if layout == "shared" else key_pool.shape[0]
    table_stride = tables.stride(0) if tables.shape[0] > 1 else 0
    head_dim = key_pool.shape[-1]
    key_out = torch.empty((batch, desc.kv_heads, int(valid), head_dim), dtype=key_pool.dtype, device=device)
    value_out = torch.empty_like(key_out)
    status = lib.qa_paged_kv_gather(
        ctypes.byref(desc), head_dim, batch, _ptr(tables), _code(tables), table_stride, tables.shape[1], int(valid), int(block_size),
        _ptr(key_out), _ptr(value_out), _stream(device),
    )
    L.check(lib, status, "paged_kv_gather")
    return key_out, value_out


# --------------------------------------------------------------------------- gated delta rule


def _f32_contig(tensor: torch.Tensor, name: str, device: torch.device) -> torch.Tensor:
    _require_cuda(tensor, name, device)
    _require(tensor.dtype == torch.float32, f"{name} must be float32")
    return tensor.contiguous()


def linear_attention_recurrent_core(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, g: torch.Tensor, beta: torch.Tensor, initial_state: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Token-serial gated delta rule on prepared inputs.

    ``query``/``key`` ``(B, H, S, dk)``, ``value`` ``(B, H, S, dv)``,
    ``g``/``beta`` ``(B, H, S)``, ``initial_state`` ``(B, H, dk, dv)``, all
    float32 (already L2-normalised and scaled, ``src/tp_runtime.py:2790-2805``).
    Returns ``(output (B, H, S, dv), final_state)`` fp32.  Reference:
    ``src/fp8_cuda.py:206-214`` -> ``src/csrc/fp8_linear_cuda.cu:2491-2573``.
    """
    lib = L.load_library()
    _require_cuda(query, "query")
    device = query.device
    q = _f32_contig(query, "query", device)
    k = _f32_contig(key, "key", device)
    v = _f32_contig(value, "value", device)
    gg = _f32_contig(g, "g", device)
    bb = _f32_contig(beta, "beta", device)
    s0 = _f32_contig(initial_state, "initial_state", device)
    _require(q.dim() == 4, "query must have shape [batch, heads, seq_len, key_dim]")
    _require(k.dim() == 4, "key must have shape [batch, heads, seq_len, key_dim]")
    _require(v.dim() == 4, "value must have shape [batch, heads, seq_len, value_dim]")
    _require(gg.dim() == 3, "g must have shape [batch, heads, seq_len]")
    _require(bb.dim() == 3, "beta must have shape [batch, heads, seq_len]")
    _require(s0.dim() == 4, "initial_state must have shape [batch, heads, key_dim, value_dim]")
    batch, heads, seq, key_dim = q.shape
    value_dim = v.shape[3]
    _require(batch > 0 and heads > 0 and seq > 0 and key_dim > 0 and value_dim > 0, "seq_len must be positive and fit int32")
    _require(k.shape == q.shape, "key shape must match query shape")
    _require(tuple(v.shape[:3]) == (batch, heads, seq), "value batch/head/seq must match query")
    _require(tuple(gg.shape) == (batch, heads, seq), "g shape must match [batch, heads, seq_len]")
    _require(tuple(bb.shape) == (batch, heads, seq), "beta shape must match [batch, heads, seq_len]")
    _require(tuple(s0.shape[:2]) == (batch, heads), "initial_state batch/head must match query")
    _require(tuple(s0.shape[2:]) == (key_dim, value_dim), "initial_state key/value dims must match query/value")
    out = torch.empty((batch, heads, seq, value_dim), dtype=torch.float32, device=device)
    final = torch.empty_like(s0)
    status = lib.qa_linear_attention_recurrent_core(
        _ptr(q), _ptr(k), _ptr(v), _ptr(gg), _ptr(bb), _ptr(s0), _ptr(out), _ptr(final), batch, heads, seq, key_dim, value_dim, _stream(device)
    )
    L.check(lib, status, "linear_attention_recurrent_core")
    return out, final


def _conv_weight(weight: torch.Tensor, channels: int, device: torch.device) -> torch.Tensor:
    _require_cuda(weight, "conv weight", device)
    w = weight.reshape(weight.shape[0], weight.shape[-1]).float().contiguous()
    _require(w.shape[0] == channels, "conv weight must have one row per channel")
    return w


def causal_conv1d_prefill(
    x: torch.Tensor, weight: torch.Tensor, conv_state: torch.Tensor | None = None, *, apply_silu: bool = True, out_dtype: torch.dtype = torch.float32
) -> tuple[torch.Tensor, torch.Tensor]:
    """Depthwise causal conv1d (+SiLU) over a token-major ``(B, T, C)`` input.

    ``conv_state`` ``(B, C, K-1)`` holds the previous K-1 inputs (zeros when
    None).  Returns ``(out (B, T, C), new_state (B, C, K-1))``; the math is the
    fp32 ``F.conv1d`` of ``src/reference_ops.py:245-258``.
    """
    lib = L.load_library()
    _require_cuda(x, "x")
    device = x.device
    _require(x.dim() == 3 and x.stride(-1) == 1, "x must be (batch, seq, channels) with contiguous channels")
    _float_dtype(x, "x")
    batch, seq, channels = x.shape
    w = _conv_weight(weight, channels, device)
    kernel = w.shape[1]
    state_in = None
    if conv_state is not None:
        state_in = _f32_contig(conv_state, "conv_state", device)
        _require(tuple(state_in.shape) == (batch, channels, kernel - 1), "conv_state must be (batch, channels, kernel-1)")
    new_state = torch.empty((batch, channels, kernel - 1), dtype=torch.float32, device=device)
    out = torch.empty((batch, seq, channels), dtype=out_dtype, device=device)
    status = lib.qa_causal_conv1d_prefill(
        _ptr(x), _code(x), x.stride(0), x.stride(1), _ptr(state_in), _ptr(new_state), channels * (kernel - 1), ctypes.c_void_p(0), L.QA_I32,
        batch, _ptr(w), batch, seq, channels, kernel, _ptr(out), _code(out), out.stride(0), out.stride(1), int(apply_silu), _stream(device),
    )
    L.check(lib, status, "causal_conv1d_prefill")
    return out, new_state


def causal_conv1d_update(x: torch.Tensor, conv_state: torch.Tensor, weight: torch.Tensor, slots: torch.Tensor | None = None, *, apply_silu: bool = True) -> torch.Tensor:
    """One token ``x`` ``(B, C)`` through the conv; ``conv_state`` ``(rows, C, K-1)`` updated in place.

    Row ``b`` uses state row ``slots[b]`` (or ``b``).  Returns fp32 ``(B, C)``.
    """
    lib = L.load_library()
    _require_cuda(x, "x")
    device = x.device
    _require(x.dim() == 2 and x.stride(-1) == 1, "x must be (batch, channels)")
    _float_dtype(x, "x")
    batch, channels = x.shape
    w = _conv_weight(weight, channels, device)
    kernel = w.shape[1]
    _require_cuda(conv_state, "conv_state", device)
    _require(conv_state.dtype == torch.float32 and conv_state.is_contiguous(), "conv_state must be contiguous float32")
    _require(tuple(conv_state.shape[1:]) == (channels, kernel - 1), "conv_state must be (rows, channels, kernel-1)")
    slot_ptr, slot_code = ctypes.c_void_p(0), L.QA_I32
    if slots is not None:
        _require_cuda(slots, "slots", device)
        _index_dtype(slots, "slots")
        slots = slots.contiguous()
        slot_ptr, slot_code = _ptr(slots), _code(slots)
    out = torch.empty((batch, channels), dtype=torch.float32, device=device)
    status = lib.qa_causal_conv1d_update(
        _ptr(x), _code(x), x.stride(0), _ptr(conv_state), channels * (kernel - 1), slot_ptr, slot_code, conv_state.shape[0], _ptr(w), batch,
        channels, kernel,
        _ptr(out), L.QA_F32, out.stride(0), int(apply_silu), _stream(device),
    )
    L.check(lib, status, "causal_conv1d_update")
    return out


def gated_delta_step(
    qkv: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
    a_log: torch.Tensor,
    dt_bias: torch.Tensor,
    state: torch.Tensor,
    *,
    key_heads: int,
    slots: torch.Tensor | None = None,
    out_dtype: torch.dtype = torch.bfloat16,
    z: torch.Tensor | None = None,
    norm_weight: torch.Tensor | None = None,
    eps: float = 1e-6,
) -> torch.Tensor:
    """Fused single-token recurrence of a linear-attention layer.

    ``qkv`` ``(B, 2*Hqk*dk + Hv*dv)`` fp32 is the conv+SiLU output; ``a``/``b``
    ``(B, Hv)`` the raw ``in_proj_a``/``in_proj_b`` outputs; ``state``
    ``(slots, Hv, dk, dv)`` fp32 is updated in place at ``slots[b]`` (or ``b``).
    Returns ``(B, Hv, dv)`` in ``out_dtype``.  Follows
    ``src/reference_ops.py:271-283,291-322`` for one token.  With ``z`` (the
    ``in_proj_z`` output ``(B, Hv*dv)``) and ``norm_weight`` ``(dv,)`` the same
    kernel also applies the layer's output stage, ``gated_rms_norm`` on the fp32
    core (``src/reference_ops.py:172-178,284-287``).
    """
    lib = L.load_library()
    _require_cuda(qkv, "qkv")
    device = qkv.device
    _require(qkv.dtype == torch.float32 and qkv.dim() == 2 and qkv.stride(-1) == 1, "qkv must be (batch, channels) float32")
    _require_cuda(state, "state", device)
    _require(state.dtype == torch.float32 and state.dim() == 4 and state.is_contiguous(), "state must be contiguous (slots, Hv, dk, dv) float32")
    _, value_heads, key_dim, value_dim = state.shape
    batch = qkv.shape[0]
    _require_cuda(a, "a", device)
    _require_cuda(b, "b", device)
    _require(a.shape == (batch, value_heads) and b.shape == (batch, value_heads), "a/b must be (batch, value_heads)")
    _require(a.dtype == b.dtype and a.dtype in (torch.float32, torch.bfloat16), "a/b must share a float32/bfloat16 dtype")
    a_c, b_c = a.contiguous(), b.contiguous()
    alog = _f32_contig(a_log.reshape(-1), "a_log", device)
    dtb = _f32_contig(dt_bias.reshape(-1), "dt_bias", device)
    slot_ptr, slot_code = ctypes.c_void_p(0), L.QA_I32
    if slots is not None:
        _require_cuda(slots, "slots", device)
        _index_dtype(slots, "slots")
        slots = slots.contiguous()
        slot_ptr, slot_code = _ptr(slots), _code(slots)
    out = torch.empty((batch, value_heads, value_dim), dtype=out_dtype, device=device)
    if z is None:
        _require(norm_weight is None, "norm_weight needs z")
        status = lib.qa_gated_delta_step(
            _ptr(qkv), qkv.stride(0), _ptr(a_c), _ptr(b_c), _code(a_c), a_c.stride(0), _ptr(alog), _ptr(dtb), _ptr(state), state.stride(0),
            slot_ptr, slot_code, state.shape[0], _ptr(out), _code(out), out.stride(0), batch, int(key_heads), value_heads, key_dim, value_dim, _stream(device),
        )
    else:
        _require_cuda(z, "z", device)
        _float_dtype(z, "z")
        _require(norm_weight is not None, "the output stage needs norm_weight")
        zz = z.reshape(batch, value_heads * value_dim)
        _require(zz.stride(-1) == 1, "z rows must be contiguous")
        w = norm_weight.reshape(-1).to(device=device).contiguous()
        _float_dtype(w, "norm_weight")
        _require(w.numel() == value_dim, "norm_weight must have value_dim elements")
        status = lib.qa_gated_delta_step_norm(
            _ptr(qkv), qkv.stride(0), _ptr(a_c), _ptr(b_c), _code(a_c), a_c.stride(0), _ptr(alog), _ptr(dtb), _ptr(state), state.stride(0),
            slot_ptr, slot_code, state.shape[0], _ptr(zz), _code(zz), zz.stride(0), _ptr(w), _code(w), float(eps), _ptr(out), _code(out), out.stride(0), batch,
            int(key_heads), value_heads, key_dim, value_dim, _stream(device),
        )
    L.check(lib, status, "gated_delta_step")
    return out


def gated_delta_step_conv(
    x: torch.Tensor,
    conv_state: torch.Tensor,
    conv_weight: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
    a_log: torch.Tensor,
    dt_bias: torch.Tensor,
    state: torch.Tensor,
    *,
    key_heads: int,
    slots: torch.Tensor | None = None,
    out_dtype: torch.dtype = torch.bfloat16,
    z: torch.Tensor | None = None,
    norm_weight: torch.Tensor | None = None,
    eps: float = 1e-6,
) -> torch.Tensor:
    """``causal_conv1d_update`` followed by ``gated_delta_step`` in one kernel.

    ``x`` ``(B, C)`` is the token's raw ``in_proj_qkv`` row (float32 or bfloat16),
    ``conv_state`` ``(rows, C, K-1)`` fp32 and ``state`` ``(rows, Hv, dk, dv)`` fp32 are
    both updated in place at row ``slots[b]`` (or ``b``); the other arguments and the
    result are ``gated_delta_step``'s.  The activations and outputs equal those of the
    two calls.
    """
    lib = L.load_library()
    _require_cuda(x, "x")
    device = x.device
    _require(x.dim() == 2 and x.stride(-1) == 1, "x must be (batch, channels)")
    _float_dtype(x, "x")
    batch, channels = x.shape
    w = _conv_weight(conv_weight, channels, device)
    kernel = w.shape[1]
    _require_cuda(conv_state, "conv_state", device)
    _require(conv_state.dtype == torch.float32 and conv_state.is_contiguous(), "conv_state must be contiguous float32")
    _require(tuple(conv_state.shape[1:]) == (channels, kernel - 1), "conv_state must be (rows, channels, kernel-1)")
    _require_cuda(state, "state", device)
    _require(state.dtype == torch.float32 and state.dim() == 4 and state.is_contiguous(), "state must be contiguous (slots, Hv, dk, dv) float32")
    _require(conv_state.shape[0] == state.shape[0], "conv_state and state must have the same rows")
    _, value_heads, key_dim, value_dim = state.shape
    _require(channels == 2 * int(key_heads) * key_dim + value_heads * value_dim, "x must hold the q, k and v channels")
    _require_cuda(a, "a", device)
    _require_cuda(b, "b", device)
    _require(a.shape == (batch, value_heads) and b.shape == (batch, value_heads), "a/b must be (batch, value_heads)")
    _require(a.dtype == b.dtype and a.dtype in (torch.float32, torch.bfloat16), "a/b must share a float32/bfloat16 dtype")
    a_c, b_c = a.contiguous(), b.contiguous()
    alog = _f32_contig(a_log.reshape(-1), "a_log", device)
    dtb = _f32_contig(dt_bias.reshape(-1), "dt_bias", device)
    slot_ptr, slot_code = ctypes.c_void_p(0), L.QA_I32
    if slots is not None:
        _require_cuda(slots, "slots", device)
        _index_dtype(slots, "slots")
        slots = slots.contiguous()
        slot_ptr, slot_code = _ptr(slots), _code(slots)
    z_ptr, z_code, z_sb, w_ptr, w_code = ctypes.c_void_p(0), L.QA_F32, 0, ctypes.c_void_p(0), L.QA_F32
    if z is not None:
        _require_cuda(z, "z", device)
        _float_dtype(z, "z")
        _require(norm_weight is not None, "the output stage needs norm_weight")
        zz = z.reshape(batch, value_heads * value_dim)
        _require(zz.stride(-1) == 1, "z rows must be contiguous")
        nw = norm_weight.reshape(-1).to(device=device).contiguous()
        _float_dtype(nw, "norm_weight")
        _require(nw.numel() == value_dim, "norm_weight must have value_dim elements")
        z_ptr, z_code, z_sb, w_ptr, w_code = _ptr(zz), _code(zz), zz.stride(0), _ptr(nw), _code(nw)
    else:
        _require(norm_weight is None, "norm_weight needs z")
    out = torch.empty((batch, value_heads, value_dim), dtype=out_dtype, device=device)
    status = lib.qa_gated_delta_step_conv(
        _ptr(x), _code(x), x.stride(0), _ptr(conv_state), channels * (kernel - 1), _ptr(w), kernel, _ptr(a_c), _ptr(b_c), _code(a_c),
        a_c.stride(0), _ptr(alog), _ptr(dtb), _ptr(state), state.stride(0), slot_ptr, slot_code, state.shape[0], z_ptr, z_code, z_sb, w_ptr,
        w_code, float(eps), _ptr(out), _code(out), out.stride(0), batch, int(key_heads), value_heads, key_dim, value_dim, _stream(device),
    )
    L.check(lib, status, "gated_delta_step_conv")
    return out


def chunk_gated_delta_rule(
    mixed_qkv: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
    a_log: torch.Tensor,
    dt_bias: torch.Tensor,
    conv_weight: torch.Tensor,
    *,
    key_heads: int,
    value_heads: int,
    conv_state: torch.Tensor | None = None,
    initial_state: torch.Tensor | None = None,
    out_dtype: torch.dtype = torch.bfloat16,
    keep_conv_state: bool = True,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor | None]:
    """Chunked prefill of a linear-attention layer from its raw projections.

    ``mixed_qkv`` ``(B, T, 2*Hqk*128 + Hv*128)`` (the ``in_proj_qkv`` output),
    ``a``/``b`` ``(B, T, Hv)``, ``a_log``/``dt_bias`` ``(Hv,)``, ``conv_weight``
    ``(C, 1, 4)`` or ``(C, 4)``.  Returns ``(core (B, T, Hv, 128), final_state
    (B, Hv, 128, 128) fp32, conv_state (B, C, 3) fp32 or None)``; ``core`` is
    the recurrence output before the gated RMSNorm
    (``src/reference_ops.py:240-283`` with the recurrence ``:291-322``).
    """
    lib = L.load_library()
    _require_cuda(mixed_qkv, "mixed_qkv")
    device = mixed_qkv.device
    _require(mixed_qkv.dtype == torch.bfloat16, "mixed_qkv must be bfloat16")
    _require(mixed_qkv.dim() == 3 and mixed_qkv.stride(-1) == 1, "mixed_qkv must be (batch, seq, channels) with contiguous channels")
    batch, seq, channels = mixed_qkv.shape
    dk = dv = 128
    _require(channels == 2 * key_heads * dk + value_heads * dv, "mixed_qkv channels must be 2*key_heads*128 + value_heads*128")
    _require_cuda(a, "a", device)
    _require_cuda(b, "b", device)
    _require(a.shape == (batch, seq, value_heads) and b.shape == a.shape, "a/b must be (batch, seq, value_heads)")
    _require(a.dtype == b.dtype and a.dtype in (torch.float32, torch.bfloat16), "a/b must share a float32/bfloat16 dtype")
    _require(a.stride() == b.stride() and a.stride(-1) == 1, "a/b must share strides with contiguous heads")
    alog = _f32_contig(a_log.reshape(-1), "a_log", device)
    dtb = _f32_contig(dt_bias.reshape(-1), "dt_bias", device)
    w = _conv_weight(conv_weight, channels, device)
    _require(w.shape[1] == 4, "conv kernel must be 4")
    conv_in = None
    if conv_state is not None:
        conv_in = _f32_contig(conv_state, "conv_state", device)
        _require(tuple(conv_in.shape) == (batch, channels, 3), "conv_state must be (batch, channels, 3)")
    state_in = None
    if initial_state is not None:
        state_in = _f32_contig(initial_state, "initial_state", device)
        _require(tuple(state_in.shape) == (batch, value_heads, dk, dv), "initial_state must be (batch, value_heads, 128, 128)")
    out = torch.empty((batch, seq, value_heads, dv), dtype=out_dtype, device=device)
    final = torch.empty((batch, value_heads, dk, dv), dtype=torch.float32, device=device)
    conv_out = torch.empty((batch, channels, 3), dtype=torch.float32, device=device) if keep_conv_state else None
    ws_bytes = lib.qa_chunk_gated_delta_workspace(batch, seq, int(key_heads), int(value_heads))
    workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
    status = lib.qa_chunk_gated_delta_rule(
        _ptr(mixed_qkv), _code(mixed_qkv), mixed_qkv.stride(0), mixed_qkv.stride(1), _ptr(a), _ptr(b), _code(a), a.stride(0), a.stride(1),
        _ptr(alog), _ptr(dtb), _ptr(w), _ptr(conv_in), _ptr(conv_out), _ptr(state_in), _ptr(final), _ptr(out), _code(out), out.stride(0),
        out.stride(1), batch, seq, int(key_heads), int(value_heads), dk, dv, 4, _ptr(workspace), ws_bytes, _stream(device),
    )
    L.check(lib, status, "chunk_gated_delta_rule")
    return out, final, conv_out


def gated_rms_norm(core: torch.Tensor, z: torch.Tensor, weight: torch.Tensor, eps: float, *, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """The output stage of a linear-attention layer: gated RMSNorm + SiLU(z) per value head.

    ``core`` ``(..., heads, head_dim)`` (the recurrence output, float32 or bfloat16; its
    ``head_dim`` axis contiguous), ``z`` the ``in_proj_z`` output ``(..., heads * head_dim)`` or
    ``(..., heads, head_dim)``, ``weight`` ``(head_dim,)``.  Returns ``(..., heads * head_dim)``
    in ``out_dtype`` (default: ``core``'s dtype, as ``gated_rms_norm`` returns,
    ``src/reference_ops.py:172-178,284-287``).
    """
    lib = L.load_library()
    _require_cuda(core, "core")
    device = core.device
    _require_cuda(z, "z", device)
    _float_dtype(core, "core")
    _float_dtype(z, "z")
    _require(core.dim() >= 2 and core.stride(-1) == 1, "core must be (..., heads, head_dim) with a contiguous head_dim axis")
    heads, head_dim = core.shape[-2], core.shape[-1]
    lead = core.shape[:-2]
    x = core.reshape(-1, heads, head_dim)
    gate = z.reshape(*lead, heads, head_dim).reshape(-1, heads, head_dim)
    _require(gate.stride(-1) == 1, "z must have a contiguous head_dim axis")
    w = weight.reshape(-1).to(device=device).contiguous()
    _float_dtype(w, "weight")
    _require(w.numel() == head_dim, "weight must have head_dim elements")
    out = torch.empty((x.shape[0], heads, head_dim), dtype=out_dtype or core.dtype, device=device)
    _float_dtype(out, "out")
    status = lib.qa_gated_rms_norm(
        _ptr(x), _code(x), x.stride(0), x.stride(1), _ptr(gate), _code(gate), gate.stride(0), gate.stride(1), _ptr(w), _code(w), float(eps),
        x.shape[0], int(heads), int(head_dim), _ptr(out), _code(out), out.stride(0), out.stride(1), _stream(device),
    )
    L.check(lib, status, "gated_rms_norm")
    return out.reshape(*lead, heads * head_dim)


def paged_attention_prefill(
    query: torch.Tensor,
    cu_seqlens: torch.Tensor,
    prefix_lens: torch.Tensor,
    key_pool: torch.Tensor,
    value_pool: torch.Tensor,
    block_tables: torch.Tensor,
    block_size: int,
    *,
    max_new: int,
    gate: torch.Tensor | None = None,
    scale: float | None = None,
) -> torch.Tensor:
    """Causal attention of packed new tokens over the shared paged pool, with optional gate.

    ``query`` ``(total_new, H, D)`` bf16; ``cu_seqlens`` ``(B+1,)`` and
    ``prefix_lens`` ``(B,)`` device index arrays; the new tokens' K/V must
    already be appended to ``key_pool``/``value_pool`` ``(P, H_kv, bs, D)`` at
    positions ``prefix_b + n``.  ``gate`` ``(total_new, H*D)`` bf16 logits, or a
    ``(total_new, H, D)`` view with a contiguous last dimension (such as the second half of
    each ``q_proj`` head, read in place), give ``out * sigmoid(gate)``
    (``src/reference_ops.py:338-340,360``).  Returns
    ``(total_new, H, D)`` bf16.
    """
    lib = L.load_library()
    _require_cuda(query, "query")
    device = query.device
    _require(query.dtype == torch.bfloat16 and query.dim() == 3 and query.stride(-1) == 1, "query must be (tokens, heads, head_dim) bfloat16")
    for tensor, name in ((cu_seqlens, "cu_seqlens"), (prefix_lens, "prefix_lens"), (block_tables, "block_tables")):
        _require_cuda(tensor, name, device)
        _index_dtype(tensor, name)
    _require(cu_seqlens.dtype == prefix_lens.dtype, "cu_seqlens and prefix_lens must share a dtype")
    _require(key_pool.dim() == 4, "prefill needs a shared pool (blocks, kv_heads, block_size, head_dim)")
    desc = _pool_descriptor(key_pool, value_pool, "shared")
    batch = prefix_lens.shape[0]
    _require(cu_seqlens.shape[0] == batch + 1, "cu_seqlens must have batch + 1 entries")
    tokens, heads, head_dim = query.shape
    gate_c = None
    gate_sh = 0
    if gate is not None:
        _require_cuda(gate, "gate", device)
        _require(gate.dtype == torch.bfloat16, "gate must be bfloat16")
        if gate.dim() == 3:  # (tokens, heads, head_dim) view, e.g. the second half of each q_proj head
            _require(gate.shape == (tokens, heads, head_dim), "gate must be (tokens, heads*head_dim) or (tokens, heads, head_dim)")
            gate_c = gate if gate.stride(-1) == 1 else gate.contiguous()
            gate_sh = gate_c.stride(1)
        else:
            _require(gate.shape == (tokens, heads * head_dim), "gate must be (tokens, heads*head_dim) or (tokens, heads, head_dim)")
            gate_c = gate.contiguous()
    tables = block_tables.contiguous()
    out = torch.empty((tokens, heads, head_dim), dtype=torch.bfloat16, device=device)
    status = lib.qa_paged_attention_prefill(
        _ptr(query), _code(query), query.stride(0), query.stride(1), _ptr(cu_seqlens.contiguous()), _ptr(prefix_lens.contiguous()),
        _code(cu_seqlens), batch, int(max_new), heads, head_dim, ctypes.byref(desc), _ptr(tables), _code(tables), tables.stride(0),
        tables.shape[1], int(block_size), float(scale or 0.0), _ptr(gate_c), 0 if gate_c is None else gate_c.stride(0), gate_sh, _ptr(out),
        _stream(device),
    )
    L.check(lib, status, "paged_attention_prefill")
    return out


_INV_FREQ: dict[tuple[int, float, str], torch.Tensor] = {}


def rope_inv_freq(rotary_dim: int, rope_theta: float, device: torch.device) -> torch.Tensor:
    """``inv_freq`` of ``rotary_embeddings`` (``src/reference_ops.py:203-213``), computed as the
    reference computes it (fp32 torch on the CPU), moved to ``device`` once per
    (rotary_dim, theta, device)."""
    key = (int(rotary_dim), float(rope_theta), str(device))
    cached = _INV_FREQ.get(key)
    if cached is None:
        inv = 1.0 / (float(rope_theta) ** (torch.arange(0, rotary_dim, 2, dtype=torch.float32) / rotary_dim))
        cached = inv.to(device)
        _INV_FREQ[key] = cached
    return cached


_COS_SIN: dict[tuple[int, float, str], torch.Tensor] = {}


def rope_cos_sin_table(rotary_dim: int, rope_theta: float, positions: int, device: torch.device) -> torch.Tensor:
    """bf16 ``(positions, 2, rotary_dim/2)`` cos and sin of ``pos * inv_freq``, computed with the
    torch CPU operations of ``rotary_embeddings`` (``src/reference_ops.py:203-213``: fp32 angles,
    fp32 cos/sin, cast to bf16) so the values are the reference's bit for bit; cached per
    (rotary_dim, theta, device) and regrown when more positions are asked for."""
    key = (int(rotary_dim), float(rope_theta), str(device))
    cached = _COS_SIN.get(key)
    if cached is None or cached.shape[0] < positions:
        freqs = torch.outer(torch.arange(positions, dtype=torch.float32), rope_inv_freq(rotary_dim, rope_theta, torch.device("cpu")))
        table = torch.stack((freqs.cos(), freqs.sin()), dim=1).to(torch.bfloat16).contiguous()
        cached = table.to(device)
        _COS_SIN[key] = cached
    return cached


def qk_norm_rope_kv_append(
    q_proj: torch.Tensor,
    k_proj: torch.Tensor,
    v_proj: torch.Tensor,
    q_norm_weight: torch.Tensor,
    k_norm_weight: torch.Tensor,
    key_pool: torch.Tensor,
    value_pool: torch.Tensor,
    block_tables: torch.Tensor,
    cu_seqlens: torch.Tensor,
    starts: torch.Tensor,
    block_size: int,
    *,
    max_new: int,
    eps: float,
    rope_theta: float,
    partial_rotary_factor: float,
    table_positions: int = 131072,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Prologue of a full-attention layer over packed new tokens, in one launch.

    ``q_proj`` ``(tokens, H, 2D)`` (or ``(tokens, H*2D)``), ``k_proj``/``v_proj`` ``(tokens, H_kv, D)``
    (or ``(tokens, H_kv*D)``), bf16, as the projections produce them; row ``b`` owns tokens
    ``cu_seqlens[b]:cu_seqlens[b+1]`` at positions ``starts[b] + n``.  Applies the reference's
    ``rms_norm`` with the ``(1 + w)`` weight and ``apply_rotary_pos_emb`` with
    ``rotary_dim = int(D * partial_rotary_factor)`` (``src/reference_ops.py:343-347``,
    ``src/tp_runtime.py:511-525``), appends k and v to the shared pool ``(P, H_kv, bs, D)`` at
    those positions (the reference's ``cache.append``, ``src/decode_state.py:271-293``, without
    repeating heads), and returns ``(query (tokens, H, D) bf16, gate (tokens, H, D) view of
    q_proj)`` ready for :func:`paged_attention_prefill` or, for one token per row, decode.
    The bf16 cos/sin of positions below ``table_positions`` come from :func:`rope_cos_sin_table`;
    the kernel computes those of later positions itself.
    """
    lib = L.load_library()
    _require_cuda(q_proj, "q_proj")
    device = q_proj.device
    for tensor, name in ((k_proj, "k_proj"), (v_proj, "v_proj"), (q_norm_weight, "q_norm_weight"), (k_norm_weight, "k_norm_weight"),
                         (key_pool, "key_pool"), (value_pool, "value_pool"), (block_tables, "block_tables"), (cu_seqlens, "cu_seqlens"),
                         (starts, "starts")):
        _require_cuda(tensor, name, device)
    _require(key_pool.dim() == 4, "qk_norm_rope_kv_append needs a shared pool (blocks, kv_heads, block_size, head_dim)")
    _, kv_heads, _, head_dim = key_pool.shape
    tokens = q_proj.shape[0]
    q3 = q_proj.view(tokens, -1, 2 * head_dim) if q_proj.dim() == 2 else q_proj
    k3 = k_proj.view(tokens, kv_heads, head_dim) if k_proj.dim() == 2 else k_proj
    v3 = v_proj.view(tokens, kv_heads, head_dim) if v_proj.dim() == 2 else v_proj
    heads = q3.shape[1]
    _require(q3.dim() == 3 and q3.shape[2] == 2 * head_dim, "q_proj must be (tokens, heads, 2*head_dim)")
    _require(k3.shape == (tokens, kv_heads, head_dim) and v3.shape == (tokens, kv_heads, head_dim), "k_proj/v_proj must be (tokens, kv_heads, head_dim)")
    for tensor, name in ((q3, "q_proj"), (k3, "k_proj"), (v3, "v_proj"), (key_pool, "key_pool")):
        _require(tensor.dtype == torch.bfloat16 and tensor.stride(-1) == 1, f"{name} must be bfloat16 with a contiguous last dimension")
    _float_dtype(q_norm_weight, "q_norm_weight")
    _require(q_norm_weight.dtype == k_norm_weight.dtype and q_norm_weight.shape == (head_dim,) and k_norm_weight.shape == (head_dim,),
             "norm weights must be (head_dim,) of one dtype")
    for tensor, name in ((cu_seqlens, "cu_seqlens"), (starts, "starts"), (block_tables, "block_tables")):
        _index_dtype(tensor, name)
    _require(cu_seqlens.dtype == starts.dtype, "cu_seqlens and starts must share a dtype")
    batch = starts.shape[0]
    _require(cu_seqlens.shape[0] == batch + 1, "cu_seqlens must have batch + 1 entries")
    tables = block_tables.contiguous() if block_tables.dim() == 2 else block_tables.contiguous().view(1, -1).expand(batch, -1)
    rotary_dim = int(head_dim * partial_rotary_factor)
    inv_freq = rope_inv_freq(rotary_dim, rope_theta, device)
    cos_sin = rope_cos_sin_table(rotary_dim, rope_theta, int(table_positions), device) if rotary_dim > 0 and table_positions > 0 else None
    qw = q_norm_weight.contiguous()
    kw = k_norm_weight.contiguous()
    desc = _pool_descriptor(key_pool, value_pool, "shared")
    query = torch.empty((tokens, heads, head_dim), dtype=torch.bfloat16, device=device)
    status = lib.qa_qk_norm_rope_append(
        _ptr(q3), q3.stride(0), q3.stride(1), _ptr(k3), k3.stride(0), k3.stride(1), _ptr(v3), v3.stride(0), v3.stride(1), _code(q3),
        _ptr(qw), _ptr(kw), _code(qw), float(eps), _ptr(inv_freq), _ptr(cos_sin), 0 if cos_sin is None else cos_sin.shape[0], rotary_dim,
        _ptr(cu_seqlens.contiguous()), _ptr(starts.contiguous()),
        _code(cu_seqlens), batch, int(max_new), heads, head_dim, ctypes.byref(desc), _ptr(tables), _code(tables), tables.stride(0),
        tables.shape[1], int(block_size), _ptr(query), _stream(device),
    )
    L.check(lib, status, "qk_norm_rope_kv_append")
    return query, q3[..., head_dim:]
