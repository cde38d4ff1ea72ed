"""The no-alloc decode entry point (``qa_paged_attention_decode_batched_noalloc``) through the C-ABI.

It must give exactly what ``qa_paged_attention_decode_batched`` gives with a caller workspace
(same kernels, same schedule, so bit for bit), on two calls in a row of which the second is
smaller (the static scratch keeps the first call's contents), on the MFMA and the generic
path, and reject sizes whose partials exceed the 32 MiB scratch before launching anything.
"""

from __future__ import annotations

import ctypes
import math

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _shared_pool_case(seed: int, batch: int, lo: int, hi: int, *, heads=16, kv_heads=2, dim=256, bs=16, dtype=torch.bfloat16):
    gen = torch.Generator().manual_seed(seed)
    ctx = torch.randint(lo, hi + 1, (batch,), generator=gen)
    need = [(int(c) + bs - 1) // bs for c in ctx]
    pool_blocks = math.ceil(sum(need) * 1.25)
    perm = torch.randperm(pool_blocks, generator=gen)
    tables = torch.full((batch, max(need) + 3), -1, dtype=torch.int32)
    cursor = 0
    for b, n in enumerate(need):
        tables[b, :n] = perm[cursor : cursor + n].to(torch.int32)
        cursor += n
    dgen = torch.Generator(device=DEV).manual_seed(seed)
    key = torch.randn((pool_blocks, kv_heads, bs, dim), generator=dgen, device=DEV, dtype=dtype)
    value = torch.randn((pool_blocks, kv_heads, bs, dim), generator=dgen, device=DEV, dtype=dtype)
    query = torch.randn((batch, heads, 1, dim), generator=dgen, device=DEV, dtype=dtype)
    lens = ctx.to(device=DEV, dtype=torch.int32)
    lens[0] = 0  # an empty row gives zeros on both paths
    return query, tables.to(DEV), key, value, lens, bs


def _noalloc(query, tables, key, value, lens, bs) -> tuple[int, torch.Tensor]:
    import hip_loader as L
    import hip_ops

    lib = L.load_library()
    desc = hip_ops._pool_descriptor(key, value, "shared")
    batch, heads, _, dim = query.shape
    out = torch.empty_like(query)
    print(f"no-alloc decode: batch {batch}, heads {heads}/{desc.kv_heads}, dim {dim}, max_blocks {tables.shape[1]}, {query.dtype}", flush=True)
    status = lib.qa_paged_attention_decode_batched_noalloc(
        ctypes.c_void_p(query.data_ptr()), hip_ops._code(query), query.stride(0), query.stride(1), batch, heads, dim, ctypes.byref(desc),
        ctypes.c_void_p(tables.data_ptr()), hip_ops._code(tables), tables.stride(0), tables.shape[1], ctypes.c_void_p(lens.data_ptr()),
        hip_ops._code(lens), bs, 0.0, ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream),
    )
    return status, out


def _with_workspace(query, tables, key, value, lens, bs) -> torch.Tensor:
    import hip_ops

    return hip_ops.paged_attention_decode_batched(query, tables, key, value, lens, bs)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_equals_workspace_entry_on_two_calls_the_second_smaller(dtype) -> None:
    import hip_loader as L

    lib = L.load_library()
    big = _shared_pool_case(201, 48, 1024, 16384, dtype=dtype) if dtype == torch.bfloat16 else _shared_pool_case(201, 12, 64, 2000, dtype=dtype)
    small = _shared_pool_case(202, 5, 16, 3000, dtype=dtype) if dtype == torch.bfloat16 else _shared_pool_case(202, 3, 1, 700, dtype=dtype)
    for case in (big, small):
        status, out = _noalloc(*case)
        assert status == 0, L.last_error(lib)
        want = _with_workspace(*case)
        torch.cuda.synchronize()
        assert torch.equal(out, want)
        assert torch.count_nonzero(out[0]) == 0 and torch.count_nonzero(out[1:]) > 0


def test_noalloc_rejects_sizes_beyond_the_static_scratch() -> None:
    import hip_loader as L

    lib = L.load_library()
    # fp32 takes the generic path: 64 rows x 16 heads x 64 splits x 258 floats = 67.6 MB of partials
    query = torch.zeros((64, 16, 1, 256), device=DEV)
    key = torch.zeros((8, 2, 16, 256), device=DEV)
    tables = torch.zeros((64, 2048), dtype=torch.int32, device=DEV)
    lens = torch.ones(64, dtype=torch.int32, device=DEV)
    status, _ = _noalloc(query, tables, key, key, lens, 16)
    assert status != 0
    assert "static scratch too small" in L.last_error(lib)
