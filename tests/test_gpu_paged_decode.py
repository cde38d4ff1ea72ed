"""GPU parity of paged GQA decode against the CPU oracle.

The first group restates the reference's own native-kernel tests
(``tests/unit/test_fp8_cuda.py:37-200``; same seeds, shapes and tolerances,
fp32).  The second group covers the bf16 GQA-native product path on the
shared pool: BASELINE config 1 (B=4, 16 q heads, 2 KV heads, D=256, ctx 512,
bs 16, table = seeded permutation of 128 blocks, seed 0) and edge cases.
Tolerance for bf16 outputs: ``atol = rtol = 2e-2``.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as oracle_attn

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _ops():
    import hip_ops

    return hip_ops


def _dense_ref(query: torch.Tensor, dense_key: torch.Tensor, dense_value: torch.Tensor) -> torch.Tensor:
    # tests/unit/test_fp8_cuda.py:1042-1045 (fp32 probabilities, no cast)
    return oracle_attn.dense_attention(query.cpu(), dense_key.cpu(), dense_value.cpu(), position_offset=dense_key.shape[2] - 1, cast_probs=False)


def _pack(dense_key, dense_value, block_table, block_size, *, physical_blocks=None, fill=0.0):
    # tests/unit/test_fp8_cuda.py:1048-1071 (reference pool layout (B, heads, P, bs, D))
    batch, heads, seq_len, head_dim = dense_key.shape
    if physical_blocks is None:
        physical_blocks = int(block_table.max().item()) + 1
    key_blocks = torch.full((batch, heads, physical_blocks, block_size, head_dim), fill, device=dense_key.device, dtype=dense_key.dtype)
    value_blocks = torch.full_like(key_blocks, fill)
    for token in range(seq_len):
        physical = int(block_table[token // block_size].item())
        key_blocks[:, :, physical, token % block_size] = dense_key[:, :, token]
        value_blocks[:, :, physical, token % block_size] = dense_value[:, :, token]
    return key_blocks, value_blocks


def test_decode_matches_dense_contiguous_blocks() -> None:
    ops = _ops()
    torch.manual_seed(101)
    batch, heads, seq_len, head_dim, block_size = 1, 3, 5, 8, 2
    query = torch.randn((batch, heads, 1, head_dim), device=DEV)
    dense_key = torch.randn((batch, heads, seq_len, head_dim), device=DEV)
    dense_value = torch.randn((batch, heads, seq_len, head_dim), device=DEV)
    table = torch.arange(3, device=DEV, dtype=torch.long)
    kb, vb = _pack(dense_key, dense_value, table, block_size)
    out = ops.paged_attention_decode(query, table, kb, vb, seq_len, block_size)
    torch.testing.assert_close(out.cpu(), _dense_ref(query, dense_key, dense_value), atol=2e-5, rtol=2e-5)


def test_decode_non_contiguous_blocks_ignore_padding() -> None:
    ops = _ops()
    torch.manual_seed(102)
    batch, heads, seq_len, head_dim, block_size = 1, 2, 5, 8, 2
    query = torch.randn((batch, heads, 1, head_dim), device=DEV)
    dense_key = torch.randn((batch, heads, seq_len, head_dim), device=DEV)
    dense_value = torch.randn((batch, heads, seq_len, head_dim), device=DEV)
    table = torch.tensor([2, 0, 3], device=DEV, dtype=torch.long)
    kb, vb = _pack(dense_key, dense_value, table, block_size, physical_blocks=4, fill=1000.0)
    out = ops.paged_attention_decode(query, table, kb, vb, seq_len, block_size)
    torch.testing.assert_close(out.cpu(), _dense_ref(query, dense_key, dense_value), atol=2e-5, rtol=2e-5)


def test_decode_rejects_float16_query() -> None:
    ops = _ops()
    query = torch.zeros((1, 1, 1, 8), device=DEV, dtype=torch.float16)
    table = torch.tensor([0], device=DEV, dtype=torch.long)
    kb = torch.zeros((1, 1, 1, 2, 8), device=DEV)
    with pytest.raises(RuntimeError, match="query must be float32"):
        ops.paged_attention_decode(query, table, kb, kb.clone(), 1, 2)


def test_batched_matches_dense_per_request_pools() -> None:
    ops = _ops()
    torch.manual_seed(103)
    heads, head_dim, block_size = 3, 8, 2
    seq_lens = (3, 5, 8)
    rows = [torch.tensor(t, device=DEV) for t in ([1, 0], [2, 0, 1], [0, 3, 1, 2])]
    block_tables = torch.full((3, 4), -1, device=DEV, dtype=torch.long)
    query = torch.randn((3, heads, 1, head_dim), device=DEV)
    kbs, vbs, refs = [], [], []
    for row, seq_len in enumerate(seq_lens):
        dk = torch.randn((1, heads, seq_len, head_dim), device=DEV)
        dv = torch.randn((1, heads, seq_len, head_dim), device=DEV)
        block_tables[row, : rows[row].numel()] = rows[row]
        k, v = _pack(dk, dv, rows[row], block_size, physical_blocks=int(rows[row].max()) + 1 + row, fill=1000.0)
        kbs.append(k)
        vbs.append(v)
        refs.append(_dense_ref(query[row : row + 1], dk, dv))
    lens = torch.tensor(seq_lens, device=DEV, dtype=torch.long)
    out = ops.paged_attention_decode_batched(query, block_tables, kbs, vbs, lens, block_size)
    torch.testing.assert_close(out.cpu(), torch.cat(refs), atol=2e-5, rtol=2e-5)


def test_batched_matches_single_request_kernel() -> None:
    ops = _ops()
    torch.manual_seed(104)
    heads, head_dim, block_size = 2, 16, 4
    seq_lens = (1, 7)
    query = torch.randn((2, heads, 1, head_dim), device=DEV)
    block_tables = torch.full((2, 2), -1, device=DEV, dtype=torch.long)
    kbs, vbs, singles = [], [], []
    for row, seq_len in enumerate(seq_lens):
        logical = (seq_len + block_size - 1) // block_size
        table = torch.arange(logical, device=DEV, dtype=torch.long)
        block_tables[row, :logical] = table
        k = torch.randn((1, heads, logical, block_size, head_dim), device=DEV)
        v = torch.randn((1, heads, logical, block_size, head_dim), device=DEV)
        kbs.append(k)
        vbs.append(v)
        singles.append(ops.paged_attention_decode(query[row : row + 1], table, k, v, seq_len, block_size))
    lens = torch.tensor(seq_lens, device=DEV, dtype=torch.long)
    out = ops.paged_attention_decode_batched(query, block_tables, kbs, vbs, lens, block_size)
    torch.testing.assert_close(out, torch.cat(singles), atol=2e-5, rtol=2e-5)


def test_batched_rejects_mismatched_pool_count() -> None:
    ops = _ops()
    query = torch.zeros((2, 1, 1, 8), device=DEV)
    tables = torch.zeros((2, 1), device=DEV, dtype=torch.long)
    pools = [torch.zeros((1, 1, 1, 2, 8), device=DEV)]
    with pytest.raises(RuntimeError, match="key_blocks list length must match batch"):
        ops.paged_attention_decode_batched(query, tables, pools, pools, torch.ones(2, device=DEV, dtype=torch.long), 2)


# ---- bf16 GQA-native shared pool ------------------------------------------------


def _config1_inputs():
    """BASELINE config 1 as the benchmark's CPU baseline draws it (``bench.config1_inputs``)."""
    import bench

    c1 = bench.config1_inputs()
    return c1["query"], c1["key_pool"], c1["value_pool"], c1["tables"], c1["lens"], c1["bs"]


def test_config1_bf16_shared_pool_matches_oracle() -> None:
    ops = _ops()
    q, kp, vp, tables, lens, bs = _config1_inputs()
    ref = oracle_attn.paged_decode(q, [kp] * 4, [vp] * 4, tables.tolist(), lens, block_size=bs, pool_layout="phbd")
    out = ops.paged_attention_decode_batched(
        q.to(DEV), tables.to(DEV, torch.int32), kp.to(DEV), vp.to(DEV), torch.tensor(lens, device=DEV, dtype=torch.int32), bs
    )
    assert out.dtype == torch.bfloat16 and out.shape == q.shape
    torch.testing.assert_close(out.cpu().float(), ref.float(), atol=2e-2, rtol=2e-2)
    # fp32-probability restatement (no bf16 cast) is closer still
    ref32 = oracle_attn.paged_decode(q, [kp] * 4, [vp] * 4, tables.tolist(), lens, block_size=bs, pool_layout="phbd", cast_probs=False)
    assert (out.cpu().float() - ref32).abs().max().item() < 1e-2


@pytest.mark.parametrize("table_dtype", [torch.int32, torch.int64])
def test_bf16_ragged_lengths_empty_rows_and_invalid_blocks(table_dtype) -> None:
    ops = _ops()
    gen = torch.Generator().manual_seed(11)
    heads, kv_heads, dim, bs, pool_blocks = 16, 2, 256, 16, 40
    lens = [0, 1, 17, 100, 255]
    kp = torch.randn(pool_blocks, kv_heads, bs, dim, generator=gen).to(torch.bfloat16)
    vp = torch.randn(pool_blocks, kv_heads, bs, dim, generator=gen).to(torch.bfloat16)
    q = torch.randn(len(lens), heads, 1, dim, generator=gen).to(torch.bfloat16)
    perm = torch.randperm(pool_blocks, generator=gen).tolist()
    max_blocks = 16
    tables = torch.full((len(lens), max_blocks), -1, dtype=torch.long)
    cursor = 0
    py_tables = []
    for row, n in enumerate(lens):
        need = (n + bs - 1) // bs
        t = perm[cursor : cursor + need]
        cursor += need
        tables[row, :need] = torch.tensor(t, dtype=torch.long)
        py_tables.append(t)
    ref = oracle_attn.paged_decode(q, [kp] * 5, [vp] * 5, py_tables, lens, block_size=bs, pool_layout="phbd")
    out = ops.paged_attention_decode_batched(
        q.to(DEV), tables.to(DEV, table_dtype), kp.to(DEV), vp.to(DEV), torch.tensor(lens, device=DEV), bs
    )
    assert torch.count_nonzero(out[0]) == 0
    torch.testing.assert_close(out.cpu().float(), ref.float(), atol=2e-2, rtol=2e-2)


def test_decode_is_invariant_to_physical_block_permutation() -> None:
    ops = _ops()
    q, kp, vp, tables, lens, bs = _config1_inputs()
    out1 = ops.paged_attention_decode_batched(q.to(DEV), tables.to(DEV), kp.to(DEV), vp.to(DEV), torch.tensor(lens, device=DEV), bs)
    # move every block to a new physical id and rewrite the tables accordingly
    perm = torch.randperm(kp.shape[0], generator=torch.Generator().manual_seed(3))
    kp2 = torch.empty_like(kp)
    vp2 = torch.empty_like(vp)
    kp2[perm] = kp
    vp2[perm] = vp
    tables2 = perm[tables]
    out2 = ops.paged_attention_decode_batched(q.to(DEV), tables2.to(DEV), kp2.to(DEV), vp2.to(DEV), torch.tensor(lens, device=DEV), bs)
    torch.testing.assert_close(out1, out2, atol=0, rtol=0)


def test_gqa_pool_equals_repeated_reference_layout() -> None:
    """GQA shared pool == the reference's repeated-head per-request pools (fp32)."""
    ops = _ops()
    gen = torch.Generator().manual_seed(12)
    heads, kv_heads, dim, bs, n = 8, 2, 64, 4, 13
    kp = torch.randn(6, kv_heads, bs, dim, generator=gen)
    vp = torch.randn(6, kv_heads, bs, dim, generator=gen)
    table = [4, 1, 5, 0]
    q = torch.randn(1, heads, 1, dim, generator=gen)
    # reference layout: (1, H, P, bs, D) with heads repeated (src/tp_runtime.py:518-525)
    ref_k = kp.permute(1, 0, 2, 3).repeat_interleave(heads // kv_heads, dim=0).unsqueeze(0).contiguous()
    ref_v = vp.permute(1, 0, 2, 3).repeat_interleave(heads // kv_heads, dim=0).unsqueeze(0).contiguous()
    t = torch.tensor(table, device=DEV)
    out_ref_layout = ops.paged_attention_decode(q.to(DEV), t, ref_k.to(DEV), ref_v.to(DEV), n, bs)
    out_shared = ops.paged_attention_decode(q.to(DEV), t, kp.to(DEV), vp.to(DEV), n, bs)
    torch.testing.assert_close(out_ref_layout, out_shared, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("ctx", [3700, 4000, 4200, 140_000])
@pytest.mark.parametrize("heads,dim", [(16, 256), (8, 128)])
def test_long_context_split_merge(ctx, heads, dim) -> None:
    """Long contexts split over many waves of the balanced schedule: 3700, 4000 and 4200 tokens give
    30, 32 and 34 partials per row group (under, at and over the 32 rows the combine loads before its
    merge weights), 140000 give hundreds; a repeated call must give the same result.  Both head
    dims: D = 256 (four columns per combine lane) and D = 128 (two per lane)."""
    ops = _ops()
    gen = torch.Generator().manual_seed(13)
    kv_heads, bs = 2, 16
    print(f"long-context decode: ctx {ctx}, heads {heads}/{kv_heads}, D {dim}", flush=True)
    blocks = (ctx + bs - 1) // bs
    kp = torch.randn(blocks + 3, kv_heads, bs, dim, generator=gen).to(torch.bfloat16)
    vp = torch.randn(blocks + 3, kv_heads, bs, dim, generator=gen).to(torch.bfloat16)
    table = torch.randperm(blocks + 3, generator=gen)[:blocks]
    q = torch.randn(1, heads, 1, dim, generator=gen).to(torch.bfloat16)
    ref = oracle_attn.paged_decode(q, [kp], [vp], [table.tolist()], [ctx], block_size=bs, pool_layout="phbd", cast_probs=False)
    for _ in range(2):  # the second call reuses a workspace the first one left dirty
        out = ops.paged_attention_decode_batched(q.to(DEV), table.unsqueeze(0).to(DEV), kp.to(DEV), vp.to(DEV), torch.tensor([ctx], device=DEV), bs)
        torch.testing.assert_close(out.cpu().float(), ref, atol=2e-2, rtol=2e-2)


def test_kernel_timing_counts_decode_launches() -> None:
    """The opt-in event timer sees one partial and one combine launch per batched decode call."""
    import hip_loader

    ops = _ops()
    gen = torch.Generator().manual_seed(21)
    kp = torch.randn(40, 2, 16, 256, generator=gen).to(torch.bfloat16).to(DEV)
    vp = torch.randn(40, 2, 16, 256, generator=gen).to(torch.bfloat16).to(DEV)
    tables = torch.arange(40).view(2, 20).to(DEV)
    q = torch.randn(2, 16, 1, 256, generator=gen).to(torch.bfloat16).to(DEV)
    lens = torch.tensor([300, 17], device=DEV)
    with hip_loader.KernelTiming() as timing:
        for _ in range(3):
            ops.paged_attention_decode_batched(q, tables, kp, vp, lens, 16)
        torch.cuda.synchronize()
        ms, n = timing.read("decode_partial_mfma")
        cms, cn = timing.read("decode_combine")
    assert n == 3 and cn == 3
    assert ms > 0.0 and cms > 0.0


def test_raw_ctypes_binding_matches_hip_ops() -> None:
    """The C-ABI used with nothing but ctypes (as a reference-side binding would) gives hip_ops' result."""
    import ctypes

    import hip_loader

    ops = _ops()
    gen = torch.Generator().manual_seed(5)
    P, Hkv, bs, D, B, H = 64, 2, 16, 256, 3, 16
    pool_k = torch.randn(P, Hkv, bs, D, generator=gen).to(torch.bfloat16).to(DEV)
    pool_v = torch.randn(P, Hkv, bs, D, generator=gen).to(torch.bfloat16).to(DEV)
    tables = torch.randperm(P, generator=gen)[:60].view(B, 20).to(DEV)
    lens = torch.tensor([320, 1, 77], device=DEV)
    query = torch.randn(B, H, 1, D, generator=gen).to(torch.bfloat16).to(DEV)
    max_tokens = int(lens.max())

    class PagedKV(ctypes.Structure):
        _fields_ = [("key", ctypes.c_void_p), ("value", ctypes.c_void_p),
                    ("row_key_ptrs", ctypes.c_void_p), ("row_value_ptrs", ctypes.c_void_p), ("row_blocks", ctypes.c_void_p),
                    ("num_blocks", ctypes.c_int64), ("stride_batch", ctypes.c_int64), ("stride_block", ctypes.c_int64),
                    ("stride_head", ctypes.c_int64), ("stride_token", ctypes.c_int64),
                    ("kv_heads", ctypes.c_int32), ("dtype", ctypes.c_int32)]

    lib = ctypes.CDLL(str(hip_loader.LIBRARY_PATH), mode=ctypes.RTLD_GLOBAL)
    lib.qa_last_error.restype = ctypes.c_char_p
    lib.qa_paged_attention_decode_workspace.restype = ctypes.c_int64
    lib.qa_paged_attention_decode_workspace.argtypes = [ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_int64, ctypes.c_int32]
    kv = PagedKV(pool_k.data_ptr(), pool_v.data_ptr(), None, None, None, P, 0, Hkv * bs * D, bs * D, D, Hkv, 1)
    ws = torch.empty(lib.qa_paged_attention_decode_workspace(B, H, D, max_tokens, bs), dtype=torch.uint8, device=DEV)
    out = torch.empty_like(query)
    status = lib.qa_paged_attention_decode_batched(
        ctypes.c_void_p(query.data_ptr()), 1, ctypes.c_int64(H * D), ctypes.c_int64(D), ctypes.c_int64(B), H, D,
        ctypes.byref(kv), ctypes.c_void_p(tables.data_ptr()), 4, ctypes.c_int64(tables.stride(0)), ctypes.c_int64(tables.shape[1]),
        ctypes.c_void_p(lens.data_ptr()), 4, bs, ctypes.c_float(D ** -0.5),
        ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(ws.data_ptr()), ctypes.c_int64(ws.numel()),
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert status == 0, lib.qa_last_error().decode()
    expected = ops.paged_attention_decode_batched(query, tables, pool_k, pool_v, lens, bs)
    torch.testing.assert_close(out, expected, atol=0, rtol=0)


@pytest.mark.parametrize("dim,heads,kv_heads", [(128, 8, 2), (256, 16, 2), (128, 16, 1), (256, 4, 4)])
def test_bf16_head_dims_groups_and_invalid_blocks_inside_rows(dim, heads, kv_heads) -> None:
    """Both MFMA head dims and group sizes 1..16; a table entry outside the pool (or -1) inside a row's
    valid range is skipped, so the row attends over its remaining tokens (decode has no positional term)."""
    ops = _ops()
    gen = torch.Generator().manual_seed(17 + dim + heads)
    bs, pool_blocks = 16, 200
    lens = [0, 1, 17, 300, 512, 1000]
    kp = torch.randn(pool_blocks, kv_heads, bs, dim, generator=gen).to(torch.bfloat16)
    vp = torch.randn(pool_blocks, kv_heads, bs, dim, generator=gen).to(torch.bfloat16)
    q = torch.randn(len(lens), heads, 1, dim, generator=gen).to(torch.bfloat16)
    perm = torch.randperm(pool_blocks, generator=gen).tolist()
    max_blocks = 64
    tables = torch.full((len(lens), max_blocks), -1, dtype=torch.long)
    cursor, kept_tables, kept_lens = 0, [], []
    for row, n in enumerate(lens):
        need = (n + bs - 1) // bs
        t = perm[cursor : cursor + need]
        cursor += need
        tables[row, :need] = torch.tensor(t, dtype=torch.long)
        kept_tables.append(list(t))
        kept_lens.append(n)
    tables[3, 5] = pool_blocks + 7  # out of the pool
    tables[5, 20] = -1              # padding marker inside the row
    for row, blk in ((3, 5), (5, 20)):
        del kept_tables[row][blk]
        kept_lens[row] -= bs
    ref = oracle_attn.paged_decode(q, [kp] * len(lens), [vp] * len(lens), kept_tables, kept_lens, block_size=bs, pool_layout="phbd",
                                   cast_probs=False)
    out = ops.paged_attention_decode_batched(q.to(DEV), tables.to(DEV), kp.to(DEV), vp.to(DEV), torch.tensor(lens, device=DEV), bs)
    assert torch.count_nonzero(out[0]) == 0
    torch.testing.assert_close(out.cpu().float(), ref.float(), atol=2e-2, rtol=2e-2)
