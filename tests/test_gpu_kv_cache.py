"""GPU slot writes and gathers are bit-exact against the oracle (``oracle/paged_kv.py``)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import paged_kv

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _as_np(t: torch.Tensor) -> np.ndarray:
    t = t.cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy()
    return t.numpy()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("table_dtype", [torch.int32, torch.int64])
def test_append_matches_oracle_bit_exact(dtype, table_dtype) -> None:
    import hip_ops

    gen = torch.Generator().manual_seed(21)
    batch, kv_heads, dim, bs, pool_blocks, max_blocks = 3, 2, 256, 16, 30, 8
    key_pool = torch.randn(pool_blocks, kv_heads, bs, dim, generator=gen).to(dtype)
    value_pool = torch.randn(pool_blocks, kv_heads, bs, dim, generator=gen).to(dtype)
    perm = torch.randperm(pool_blocks, generator=gen)[: batch * max_blocks].reshape(batch, max_blocks)
    starts = [0, 7, 31]
    seq = 20
    counts = [20, 9, 20]
    new_k = torch.randn(batch, kv_heads, seq, dim, generator=gen).to(dtype)
    new_v = torch.randn(batch, kv_heads, seq, dim, generator=gen).to(dtype)
    # oracle on numpy copies
    ok, ov = _as_np(key_pool).copy(), _as_np(value_pool).copy()
    for b in range(batch):
        paged_kv.append_tokens(ok, perm[b].numpy(), starts[b], _as_np(new_k[b, :, : counts[b]]), block_size=bs, pool_layout="phbd")
        paged_kv.append_tokens(ov, perm[b].numpy(), starts[b], _as_np(new_v[b, :, : counts[b]]), block_size=bs, pool_layout="phbd")
    kp, vp = key_pool.to(DEV), value_pool.to(DEV)
    hip_ops.paged_kv_append(
        new_k.to(DEV), new_v.to(DEV), kp, vp, perm.to(DEV, table_dtype), torch.tensor(starts, device=DEV), bs,
        counts=torch.tensor(counts, device=DEV, dtype=torch.int32),
    )
    np.testing.assert_array_equal(_as_np(kp), ok)
    np.testing.assert_array_equal(_as_np(vp), ov)


def test_append_reference_layout_scalar_start_matches_oracle() -> None:
    import hip_ops

    gen = torch.Generator().manual_seed(22)
    heads, dim, bs, blocks = 4, 8, 2, 6
    pool_k = torch.randn(1, heads, blocks, bs, dim, generator=gen)
    pool_v = torch.randn(1, heads, blocks, bs, dim, generator=gen)
    table = torch.tensor([3, 1, 4, 0])
    new_k = torch.randn(1, heads, 5, dim, generator=gen)
    new_v = torch.randn(1, heads, 5, dim, generator=gen)
    ok, ov = pool_k[0].numpy().copy(), pool_v[0].numpy().copy()
    paged_kv.append_tokens(ok, table.numpy(), 2, new_k[0].numpy(), block_size=bs, pool_layout="hpbd")
    paged_kv.append_tokens(ov, table.numpy(), 2, new_v[0].numpy(), block_size=bs, pool_layout="hpbd")
    kp, vp = pool_k.to(DEV), pool_v.to(DEV)
    hip_ops.paged_kv_append(new_k.to(DEV), new_v.to(DEV), kp, vp, table.to(DEV), 2, bs)
    np.testing.assert_array_equal(kp[0].cpu().numpy(), ok)
    np.testing.assert_array_equal(vp[0].cpu().numpy(), ov)


def test_gather_matches_oracle_and_zero_fills_invalid() -> None:
    import hip_ops

    gen = torch.Generator().manual_seed(23)
    kv_heads, dim, bs, blocks = 2, 256, 16, 12
    kp = torch.randn(blocks, kv_heads, bs, dim, generator=gen).to(torch.bfloat16)
    vp = torch.randn(blocks, kv_heads, bs, dim, generator=gen).to(torch.bfloat16)
    tables = torch.tensor([[5, 2, 9, -1], [0, 11, 3, 7]])
    valid = 50
    k_out, v_out = hip_ops.paged_kv_gather(kp.to(DEV), vp.to(DEV), tables.to(DEV), valid, bs)
    for b in range(2):
        expect_k = paged_kv.gather_tokens_bruteforce(_as_np(kp), [max(x, 0) for x in tables[b].tolist()], valid, block_size=bs, pool_layout="phbd")
        got = _as_np(k_out[b])
        if b == 0:
            np.testing.assert_array_equal(got[:, :48], expect_k[:, :48])
            assert (got[:, 48:] == 0).all()
        else:
            np.testing.assert_array_equal(got, expect_k)
    expect_v = paged_kv.gather_tokens(_as_np(vp), tables[1].tolist(), valid, block_size=bs, pool_layout="phbd")
    np.testing.assert_array_equal(_as_np(v_out[1]), expect_v)


def test_append_then_decode_equals_dense_reference() -> None:
    """Round trip: appended tokens are exactly what decode and gather read back."""
    import hip_ops
    from oracle import attention

    gen = torch.Generator().manual_seed(24)
    heads, kv_heads, dim, bs = 16, 2, 256, 16
    lens = [33, 64]
    pool_blocks = 16
    kp = torch.zeros(pool_blocks, kv_heads, bs, dim, dtype=torch.bfloat16, device=DEV)
    vp = torch.zeros_like(kp)
    tables = torch.tensor([[7, 1, 12, -1], [3, 14, 0, 9]], device=DEV)
    dense_k = torch.randn(2, kv_heads, 64, dim, generator=gen).to(torch.bfloat16)
    dense_v = torch.randn(2, kv_heads, 64, dim, generator=gen).to(torch.bfloat16)
    hip_ops.paged_kv_append(dense_k.to(DEV), dense_v.to(DEV), kp, vp, tables, 0, bs, counts=torch.tensor(lens, device=DEV))
    k_back, _ = hip_ops.paged_kv_gather(kp, vp, tables, 33, bs)
    assert torch.equal(k_back[0].cpu(), dense_k[0, :, :33])
    q = torch.randn(2, heads, 1, dim, generator=gen).to(torch.bfloat16)
    out = hip_ops.paged_attention_decode_batched(q.to(DEV), tables, kp, vp, torch.tensor(lens, device=DEV), bs)
    for b in range(2):
        ref = attention.dense_attention(q[b : b + 1], dense_k[b : b + 1, :, : lens[b]], dense_v[b : b + 1, :, : lens[b]], position_offset=lens[b] - 1)
        torch.testing.assert_close(out[b : b + 1].cpu().float(), ref.float(), atol=2e-2, rtol=2e-2)
