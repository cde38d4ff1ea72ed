"""GPU chunked paged prefill (causal, gated) against ``oracle.attention.paged_prefill``.

bf16 outputs within 2e-2 absolute/relative.  Also: query-chunked prefill ==
one-shot prefill; the last prefill row == the decode kernel at that position.
"""

from __future__ import annotations

import pytest
import torch

from oracle import attention as oracle_attn

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _setup(seed: int, prefixes: list[int], news: list[int], *, heads: int, kv_heads: int, dim: int, bs: int = 16):
    gen = torch.Generator().manual_seed(seed)
    totals = [p + n for p, n in zip(prefixes, news)]
    need = [(t + bs - 1) // bs for t in totals]
    pool_blocks = sum(need) + 5
    perm = torch.randperm(pool_blocks, generator=gen).tolist()
    tables, cursor = [], 0
    max_blocks = max(need)
    table_t = torch.full((len(totals), max_blocks), -1, dtype=torch.int32)
    for row, n in enumerate(need):
        tables.append(perm[cursor : cursor + n])
        table_t[row, :n] = torch.tensor(tables[-1], dtype=torch.int32)
        cursor += n
    key_pool = torch.randn(pool_blocks, kv_heads, bs, dim, generator=gen).to(torch.bfloat16)
    value_pool = torch.randn(pool_blocks, kv_heads, bs, dim, generator=gen).to(torch.bfloat16)
    q = torch.randn(sum(news), heads, dim, generator=gen).to(torch.bfloat16)
    gate = torch.randn(sum(news), heads * dim, generator=gen).to(torch.bfloat16)
    return key_pool, value_pool, tables, table_t, q, gate


def _run(q, cu, prefixes, kp, vp, table_t, *, max_new, gate=None):
    import hip_ops

    return hip_ops.paged_attention_prefill(
        q.to(DEV), torch.tensor(cu, device=DEV, dtype=torch.int32), torch.tensor(prefixes, device=DEV, dtype=torch.int32), kp.to(DEV), vp.to(DEV),
        table_t.to(DEV), 16, max_new=max_new, gate=None if gate is None else gate.to(DEV),
    )


def test_prefill_ragged_prefixes_with_gate_matches_oracle() -> None:
    prefixes, news = [0, 5, 37], [20, 1, 70]
    kp, vp, tables, table_t, q, gate = _setup(51, prefixes, news, heads=16, kv_heads=2, dim=256)
    cu = [0, 20, 21, 91]
    out = _run(q, cu, prefixes, kp, vp, table_t, max_new=70, gate=gate)
    refs = oracle_attn.paged_prefill(q, kp, vp, tables, prefixes, news, block_size=16, gate=gate)
    torch.testing.assert_close(out.cpu().float(), torch.cat(refs).float(), atol=2e-2, rtol=2e-2)


def test_prefill_head_dim_128_group_4_without_gate() -> None:
    prefixes, news = [100, 0], [33, 64]
    kp, vp, tables, table_t, q, _ = _setup(52, prefixes, news, heads=8, kv_heads=2, dim=128)
    out = _run(q, [0, 33, 97], prefixes, kp, vp, table_t, max_new=64)
    refs = oracle_attn.paged_prefill(q, kp, vp, tables, prefixes, news, block_size=16)
    torch.testing.assert_close(out.cpu().float(), torch.cat(refs).float(), atol=2e-2, rtol=2e-2)


def test_query_chunked_prefill_equals_one_shot() -> None:
    prefixes, news = [19], [150]
    kp, vp, tables, table_t, q, gate = _setup(53, prefixes, news, heads=16, kv_heads=2, dim=256)
    full = _run(q, [0, 150], prefixes, kp, vp, table_t, max_new=150, gate=gate)
    parts = []
    for start in range(0, 150, 64):
        end = min(150, start + 64)
        # the cache may already hold later tokens: causality must hide them
        parts.append(_run(q[start:end], [0, end - start], [prefixes[0] + start], kp, vp, table_t, max_new=end - start, gate=gate[start:end]))
    torch.testing.assert_close(torch.cat(parts), full, atol=0, rtol=0)


def test_last_prefill_row_equals_decode_kernel() -> None:
    import hip_ops

    prefixes, news = [45], [30]
    kp, vp, tables, table_t, q, _ = _setup(54, prefixes, news, heads=16, kv_heads=2, dim=256)
    out = _run(q, [0, 30], prefixes, kp, vp, table_t, max_new=30)
    dec = hip_ops.paged_attention_decode_batched(
        q[-1:].unsqueeze(2).to(DEV), table_t.to(DEV), kp.to(DEV), vp.to(DEV), torch.tensor([75], device=DEV), 16
    )
    torch.testing.assert_close(out[-1].float(), dec[0, :, 0].float(), atol=1e-2, rtol=1e-2)


def test_prefill_past_the_lds_table_reads_the_table_from_global_memory() -> None:
    """A row whose block table is longer than the 4,096 entries the kernel keeps in LDS (a
    66,000-token prefix and 64 new tokens: 4,129 blocks) takes the kernel's global-memory table
    path; a short row beside it keeps the LDS path.  Both against the oracle."""
    prefixes, news = [66000, 10], [64, 17]
    print("prefill: prefix 66000 + 64 new, prefix 10 + 17 new (GQA 16/2, D=256)", flush=True)
    kp, vp, tables, table_t, q, gate = _setup(55, prefixes, news, heads=16, kv_heads=2, dim=256)
    assert table_t.shape[1] > 4096
    out = _run(q, [0, 64, 81], prefixes, kp, vp, table_t, max_new=64, gate=gate)
    refs = oracle_attn.paged_prefill(q, kp, vp, tables, prefixes, news, block_size=16, gate=gate)
    torch.testing.assert_close(out.cpu().float(), torch.cat(refs).float(), atol=2e-2, rtol=2e-2)
