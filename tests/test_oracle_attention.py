"""Pins ``oracle/attention.py`` against an fp64 textbook loop and invariants."""

from __future__ import annotations

import numpy as np
import torch

from oracle import attention


def _rand(*shape: int, seed: int, dtype=torch.float32) -> torch.Tensor:
    gen = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=gen).to(dtype)


def test_dense_attention_matches_textbook_fp64_with_prefix_and_gqa() -> None:
    heads, kv_heads, seq, prefix, dim = 4, 2, 5, 3, 8
    q = _rand(1, heads, seq, dim, seed=1)
    k = _rand(1, kv_heads, prefix + seq, dim, seed=2)
    v = _rand(1, kv_heads, prefix + seq, dim, seed=3)
    out = attention.dense_attention(q, k, v, position_offset=prefix, cast_probs=False)
    ref = attention.textbook_attention_fp64(
        q[0].numpy(), k[0].numpy(), v[0].numpy(), query_positions=np.arange(prefix, prefix + seq), valid=np.ones(prefix + seq, bool), scale=dim**-0.5
    )
    np.testing.assert_allclose(out[0].numpy(), ref, rtol=2e-6, atol=2e-6)


def test_dense_attention_batched_positions_and_padding_mask_match_textbook() -> None:
    heads, kv_heads, total, dim = 4, 1, 6, 8
    q = _rand(2, heads, 1, dim, seed=4)
    k = _rand(2, kv_heads, total, dim, seed=5)
    v = _rand(2, kv_heads, total, dim, seed=6)
    positions = torch.tensor([2, 5])
    valid = torch.tensor([[True, True, True, False, False, False], [True] * 6])
    out = attention.dense_attention(q, k, v, position_offset=positions, valid_mask=valid, cast_probs=False)
    for b in range(2):
        ref = attention.textbook_attention_fp64(
            q[b].numpy(), k[b].numpy(), v[b].numpy(), query_positions=np.array([int(positions[b])]), valid=valid[b].numpy(), scale=dim**-0.5
        )
        np.testing.assert_allclose(out[b].numpy(), ref, rtol=2e-6, atol=2e-6)


def test_gqa_equals_mha_on_repeated_kv() -> None:
    q = _rand(1, 8, 3, 16, seed=7)
    k = _rand(1, 2, 3, 16, seed=8)
    v = _rand(1, 2, 3, 16, seed=9)
    gqa = attention.dense_attention(q, k, v, cast_probs=False)
    # head h must read kv head h // 4 (src/reference_ops.py:414-419)
    k_rep = torch.cat([k[:, h // 4 : h // 4 + 1] for h in range(8)], dim=1)
    v_rep = torch.cat([v[:, h // 4 : h // 4 + 1] for h in range(8)], dim=1)
    mha = attention.dense_attention(q, k_rep, v_rep, cast_probs=False)
    torch.testing.assert_close(gqa, mha, rtol=0, atol=0)


def test_causality_future_token_does_not_change_past_rows() -> None:
    q = _rand(1, 2, 4, 8, seed=10)
    k = _rand(1, 2, 4, 8, seed=11)
    v = _rand(1, 2, 4, 8, seed=12)
    out = attention.dense_attention(q, k, v, cast_probs=False)
    k2, v2 = k.clone(), v.clone()
    k2[:, :, 3] += 5.0
    v2[:, :, 3] -= 5.0
    out2 = attention.dense_attention(q, k2, v2, cast_probs=False)
    torch.testing.assert_close(out[:, :, :3], out2[:, :, :3], rtol=0, atol=0)
    assert not torch.allclose(out[:, :, 3], out2[:, :, 3])


def test_zero_query_gives_mean_of_visible_values() -> None:
    q = torch.zeros(1, 1, 1, 4)
    k = _rand(1, 1, 5, 4, seed=13)
    v = _rand(1, 1, 5, 4, seed=14)
    out = attention.dense_attention(q, k, v, position_offset=4, cast_probs=False)
    torch.testing.assert_close(out[0, 0, 0], v[0, 0].mean(0), rtol=1e-6, atol=1e-6)


def test_paged_decode_invariant_under_block_permutation_and_matches_prefill_last_row() -> None:
    bs, heads, kv_heads, dim, seq = 4, 4, 2, 8, 11
    dense_k = _rand(kv_heads, seq, dim, seed=15)
    dense_v = _rand(kv_heads, seq, dim, seed=16)
    q = _rand(1, heads, 1, dim, seed=17)
    outs = []
    for perm_seed in (0, 1):
        rng = np.random.default_rng(perm_seed)
        table = list(rng.permutation(6)[:3])
        pool_k = torch.full((6, kv_heads, bs, dim), 99.0)
        pool_v = torch.full((6, kv_heads, bs, dim), -99.0)
        for pos in range(seq):
            pool_k[table[pos // bs], :, pos % bs] = dense_k[:, pos]
            pool_v[table[pos // bs], :, pos % bs] = dense_v[:, pos]
        outs.append(attention.paged_decode(q, [pool_k], [pool_v], [table], [seq], block_size=bs, pool_layout="phbd", cast_probs=False))
    torch.testing.assert_close(outs[0], outs[1], rtol=0, atol=0)
    # decode at position seq-1 == last row of a full causal prefill with that query last
    q_full = torch.cat([_rand(1, heads, seq - 1, dim, seed=18), q], dim=2)
    full = attention.dense_attention(q_full, dense_k.unsqueeze(0), dense_v.unsqueeze(0), cast_probs=False)
    torch.testing.assert_close(outs[0][:, :, 0], full[:, :, -1], rtol=1e-6, atol=1e-6)


def test_paged_decode_empty_row_is_zero() -> None:
    q = _rand(2, 2, 1, 4, seed=19)
    pool = _rand(2, 2, 2, 4, seed=20)
    out = attention.paged_decode(q, [pool, pool], [pool, pool], [[0], [0, 1]], [0, 3], block_size=2, pool_layout="phbd")
    assert torch.count_nonzero(out[0]) == 0
    assert torch.count_nonzero(out[1]) > 0


def test_gate_applies_sigmoid_per_head_channel() -> None:
    q = _rand(1, 2, 1, 4, seed=21)
    k = _rand(1, 2, 3, 4, seed=22)
    v = _rand(1, 2, 3, 4, seed=23)
    gate = _rand(1, 1, 8, seed=24)
    plain = attention.dense_attention(q, k, v, position_offset=2, cast_probs=False)
    gated = attention.dense_attention(q, k, v, position_offset=2, cast_probs=False, gate=gate)
    expected = plain * torch.sigmoid(gate.reshape(1, 1, 2, 4).transpose(1, 2))
    torch.testing.assert_close(gated, expected, rtol=0, atol=0)
