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


def _scatter_into_pool(dense: torch.Tensor, table: list[int], pool: torch.Tensor, bs: int, layout: str) -> None:
    """Write dense ``(H_kv, T, D)`` tokens into their slots ``(table[t // bs], t % bs)``."""
    for t in range(dense.shape[1]):
        if layout == "phbd":
            pool[table[t // bs], :, t % bs] = dense[:, t]
        else:  # "hpbd": the reference's per-request (heads, P, bs, D) pool
            pool[:, table[t // bs], t % bs] = dense[:, t]


def test_paged_prefill_matches_textbook_fp64_on_ragged_prefixes_gqa_and_gate() -> None:
    """``paged_prefill`` (prefix offsets, per-row query slicing, gate reshape) against an independent
    fp64 loop: a shuffled shared pool whose unused slots hold garbage, prefixes 0 / 5 / 21 (not
    multiples of the block size), new lengths 7 / 16 / 3, GQA 16 query heads on 2 KV heads."""
    bs, heads, kv_heads, dim = 4, 16, 2, 8
    prefixes, news = [0, 5, 21], [7, 16, 3]
    totals = [p + n for p, n in zip(prefixes, news)]
    need = [(t + bs - 1) // bs for t in totals]
    pool_blocks = sum(need) + 5
    rng = np.random.default_rng(40)
    perm = [int(x) for x in rng.permutation(pool_blocks)]
    tables, cursor = [], 0
    for n in need:
        tables.append(perm[cursor : cursor + n])
        cursor += n
    pool_k = torch.full((pool_blocks, kv_heads, bs, dim), 1e4)  # garbage everywhere a token is not written
    pool_v = torch.full((pool_blocks, kv_heads, bs, dim), -1e4)
    dense_k = [_rand(kv_heads, t, dim, seed=41 + b) for b, t in enumerate(totals)]
    dense_v = [_rand(kv_heads, t, dim, seed=51 + b) for b, t in enumerate(totals)]
    for b in range(3):
        _scatter_into_pool(dense_k[b], tables[b], pool_k, bs, "phbd")
        _scatter_into_pool(dense_v[b], tables[b], pool_v, bs, "phbd")
    query = _rand(sum(news), heads, dim, seed=61)
    gate = _rand(sum(news), heads * dim, seed=62)
    outs = attention.paged_prefill(query, pool_k, pool_v, tables, prefixes, news, block_size=bs, gate=gate)
    offset = 0
    for b in range(3):
        q = query[offset : offset + news[b]].transpose(0, 1).numpy()  # (H, new, D)
        ref = attention.textbook_attention_fp64(
            q, dense_k[b].numpy(), dense_v[b].numpy(), query_positions=np.arange(prefixes[b], totals[b]),
            valid=np.ones(totals[b], bool), scale=dim**-0.5,
        )
        g = gate[offset : offset + news[b]].double().reshape(news[b], heads, dim).transpose(0, 1).numpy()
        ref = ref * (1.0 / (1.0 + np.exp(-g)))
        assert outs[b].shape == (news[b], heads, dim)
        np.testing.assert_allclose(outs[b].transpose(0, 1).numpy(), ref, rtol=2e-6, atol=2e-6)
        offset += news[b]


def test_paged_prefill_mistakes_are_caught_by_the_textbook_check() -> None:
    """The checks above can fail: a query offset by one position or a gate on the wrong head axis differs."""
    heads, kv_heads, dim, total, new = 4, 2, 8, 9, 4
    k = _rand(kv_heads, total, dim, seed=70)
    v = _rand(kv_heads, total, dim, seed=71)
    q = _rand(heads, new, dim, seed=72)
    right = attention.textbook_attention_fp64(q.numpy(), k.numpy(), v.numpy(), query_positions=np.arange(5, 9), valid=np.ones(total, bool),
                                              scale=dim**-0.5)
    off_by_one = attention.textbook_attention_fp64(q.numpy(), k.numpy(), v.numpy(), query_positions=np.arange(4, 8),
                                                   valid=np.ones(total, bool), scale=dim**-0.5)
    assert np.abs(right - off_by_one).max() > 1e-3
    gate = _rand(new, heads * dim, seed=73)
    good = gate.reshape(new, heads, dim).transpose(0, 1)
    bad = gate.reshape(new, dim, heads).permute(2, 0, 1)
    assert (torch.sigmoid(good) - torch.sigmoid(bad)).abs().max() > 1e-2


def test_reference_layout_decode_equals_shared_pool_decode_and_textbook() -> None:
    """``reference_layout_decode_cpu`` (repeated heads, per-request ``(H, P, bs, D)`` pools, the
    ``"hpbd"`` branch of ``gather_dense``) == ``paged_decode`` on a shared GQA ``(P, H_kv, bs, D)``
    pool holding the same tokens == the fp64 textbook."""
    bs, heads, kv_heads, dim = 4, 8, 2, 8
    lens = [13, 1, 8]
    query = _rand(3, heads, 1, dim, seed=80)
    rng = np.random.default_rng(81)
    shared_blocks = sum((n + bs - 1) // bs for n in lens) + 3
    shared_perm = [int(x) for x in rng.permutation(shared_blocks)]
    shared_k = torch.full((shared_blocks, kv_heads, bs, dim), 7e3)
    shared_v = torch.full((shared_blocks, kv_heads, bs, dim), -7e3)
    ref_k, ref_v, ref_tables, shared_tables, cursor = [], [], [], [], 0
    for b, n in enumerate(lens):
        nb = (n + bs - 1) // bs
        dk = _rand(kv_heads, n, dim, seed=82 + b)
        dv = _rand(kv_heads, n, dim, seed=92 + b)
        shared_tables.append(shared_perm[cursor : cursor + nb])
        cursor += nb
        _scatter_into_pool(dk, shared_tables[b], shared_k, bs, "phbd")
        _scatter_into_pool(dv, shared_tables[b], shared_v, bs, "phbd")
        # the reference's per-request pool: post-repeat heads (h reads kv head h // G), own shuffled table
        table = [int(x) for x in rng.permutation(nb + 2)[:nb]]
        pk = torch.full((heads, nb + 2, bs, dim), 5e3)
        pv = torch.full((heads, nb + 2, bs, dim), -5e3)
        rep = heads // kv_heads
        _scatter_into_pool(dk.repeat_interleave(rep, dim=0), table, pk, bs, "hpbd")
        _scatter_into_pool(dv.repeat_interleave(rep, dim=0), table, pv, bs, "hpbd")
        ref_k.append(pk)
        ref_v.append(pv)
        ref_tables.append(table)
        want = attention.textbook_attention_fp64(query[b].numpy(), dk.numpy(), dv.numpy(), query_positions=np.array([n - 1]),
                                                 valid=np.ones(n, bool), scale=dim**-0.5)
        got = attention.reference_layout_decode_cpu(query[b : b + 1], [pk], [pv], [table], [n], block_size=bs)
        np.testing.assert_allclose(got[0].numpy(), want, rtol=2e-6, atol=2e-6)
    ref_out = attention.reference_layout_decode_cpu(query, ref_k, ref_v, ref_tables, lens, block_size=bs)
    shared_out = attention.paged_decode(query, [shared_k] * 3, [shared_v] * 3, shared_tables, lens, block_size=bs, pool_layout="phbd")
    torch.testing.assert_close(ref_out, shared_out, rtol=1e-6, atol=1e-6)
    # gather_dense("hpbd") returns the tokens in logical order
    dense = attention.gather_dense(ref_k[0], ref_tables[0], lens[0], block_size=bs, pool_layout="hpbd")
    assert dense.shape == (heads, lens[0], dim)
    torch.testing.assert_close(dense[:: heads // kv_heads], _rand(kv_heads, lens[0], dim, seed=82), rtol=0, atol=0)
