"""Pins ``oracle/paged_kv.py`` against the reference's known answers and brute force.

Known answers come from the reference's own tests
(``tests/unit/test_decode_state.py``); line numbers are cited per test.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import paged_kv


def test_prefill_then_steps_table_and_capacity_known_answer() -> None:
    # tests/unit/test_decode_state.py:47-63: block_size 2, prefill 3 then 3 single
    # steps -> table [0, 1, 2, 3], capacity 8.
    free = paged_kv.FreeList()
    table: list[int] = []
    valid = 0
    for seq in (3, 1, 1, 1):
        paged_kv.grow_table(table, valid, valid + seq, 2, None, free)
        valid += seq
    assert table == [0, 1, 2, 3]
    assert len(table) * 2 == 8


def test_capacity_hint_known_answer() -> None:
    # tests/unit/test_decode_state.py:92-119: hint 8, block 4 -> 2 blocks, no free.
    free = paged_kv.FreeList()
    table: list[int] = []
    assert paged_kv.grow_table(table, 0, 3, 4, 8, free) is True
    assert table == [0, 1]
    assert free.free == []
    assert paged_kv.grow_table(table, 3, 5, 4, 8, free) is False


def test_release_then_reuse_known_answer() -> None:
    # tests/unit/test_decode_state.py:158-173: released blocks come back in order.
    free = paged_kv.FreeList()
    table: list[int] = []
    paged_kv.grow_table(table, 0, 3, 2, 4, free)
    released = list(table)
    free.release(table)
    assert free.free == released
    again: list[int] = []
    paged_kv.grow_table(again, 0, 2, 2, 4, free)
    assert again == released


def test_batch_tables_known_answer() -> None:
    # tests/unit/test_decode_state.py:388-412
    out = paged_kv.batch_tables([[0, 1], [0, 1, 2]], [3, 5], [2, 2])
    assert out.block_tables.tolist() == [[0, 1, -1], [0, 1, 2]]
    assert out.sequence_lengths.tolist() == [3, 5]
    assert out.valid_mask.tolist() == [[True, True, True, False, False], [True] * 5]
    assert out.max_blocks == 3 and out.max_sequence_length == 5


def test_batch_tables_rejects_mixed_block_sizes() -> None:
    # tests/unit/test_decode_state.py:415-422
    with pytest.raises(ValueError, match="matching block sizes"):
        paged_kv.batch_tables([[0], [0]], [1, 1], [2, 4])


def test_non_contiguous_gather_known_answer() -> None:
    # tests/unit/test_decode_state.py:194-218: table [2, 0, 1] returns logical order.
    heads, dim, bs = 2, 4, 2
    chunks = [np.arange(heads * bs * dim, dtype=np.float32).reshape(heads, bs, dim) + 1000 * i for i in range(3)]
    pool = np.zeros((heads, 3, bs, dim), dtype=np.float32)
    for logical, physical in enumerate([2, 0, 1]):
        pool[:, physical] = chunks[logical]
    out = paged_kv.gather_tokens(pool, [2, 0, 1], 6, block_size=bs, pool_layout="hpbd")
    np.testing.assert_array_equal(out, np.concatenate(chunks, axis=1))


@pytest.mark.parametrize("layout", ["hpbd", "phbd"])
def test_append_then_gather_matches_bruteforce(layout: str) -> None:
    rng = np.random.default_rng(5)
    heads, dim, bs, blocks = 3, 8, 4, 12
    shape = (heads, blocks, bs, dim) if layout == "hpbd" else (blocks, heads, bs, dim)
    pool = np.full(shape, -7, dtype=np.int16)
    table = list(rng.permutation(blocks)[:7])
    dense = rng.integers(-30000, 30000, size=(heads, 25, dim)).astype(np.int16)
    start = 0
    for seq in (5, 1, 3, 16):
        paged_kv.append_tokens(pool, table, start, dense[:, start : start + seq], block_size=bs, pool_layout=layout)
        start += seq
    got = paged_kv.gather_tokens(pool, table, start, block_size=bs, pool_layout=layout)
    brute = paged_kv.gather_tokens_bruteforce(pool, table, start, block_size=bs, pool_layout=layout)
    np.testing.assert_array_equal(got, dense[:, :start])
    np.testing.assert_array_equal(brute, dense[:, :start])


def test_slot_mapping_closed_form() -> None:
    # slot = table[pos // bs] * bs + pos % bs, written out by hand for bs = 2.
    tables = np.array([[3, 1, 5], [0, 2, 4]], dtype=np.int64)
    slots = paged_kv.slot_mapping(tables, np.array([3, 0]), np.array([2, 5]), 2)
    # row 0: pos 3 -> block 1 off 1 -> 3; pos 4 -> block 5 off 0 -> 10
    # row 1: pos 0..4 -> 0, 1, 4, 5, 8
    assert slots.tolist() == [3, 10, 0, 1, 4, 5, 8]


def _reserve_token_by_token(tables, lengths, counts, free, bs):
    """Brute force: each row appends its tokens one at a time and takes one block
    from the head of the free list whenever a token starts a new block."""
    tables = tables.copy()
    free = list(free)
    for b in range(len(lengths)):
        for pos in range(int(lengths[b]), int(lengths[b] + counts[b])):
            if pos % bs == 0:
                tables[b, pos // bs] = free.pop(0)
    return tables, free


def test_reserve_step_matches_token_by_token_growth() -> None:
    rng = np.random.default_rng(5)
    bs, batch, max_blocks = 16, 37, 12
    lengths = rng.integers(0, 100, batch)
    counts = rng.integers(0, 40, batch)
    counts[::5] = 0
    free = sorted(rng.permutation(400)[:300].tolist())
    tables = np.full((batch, max_blocks), -1, dtype=np.int64)
    status, got, pos, new_len, rest = paged_kv.reserve_step(tables, lengths, counts, free, bs)
    assert status == 0
    want, want_rest = _reserve_token_by_token(tables, lengths, counts, free, bs)
    np.testing.assert_array_equal(got, want)
    assert rest == want_rest
    np.testing.assert_array_equal(pos, lengths)
    np.testing.assert_array_equal(new_len, lengths + counts)


def test_reserve_step_is_free_list_allocate_per_row() -> None:
    # the reference's pool hands out the head of its sorted free list per request
    # (src/decode_state.py:72-78): rows of 0, 17 and 32 tokens, one new token each,
    # need 1, 0 and 1 new blocks, taken as ids 0 then 1.
    free = paged_kv.FreeList()
    free.grow(6)
    tables = np.full((3, 4), -1, dtype=np.int64)
    tables[1, :2] = [4, 5]
    tables[2, :2] = [2, 3]
    status, got, _pos, new_len, rest = paged_kv.reserve_step(tables, np.array([0, 17, 32]), 1, [0, 1], 16)
    assert status == 0
    assert got[0].tolist() == [0, -1, -1, -1] and got[2].tolist() == [2, 3, 1, -1] and got[1].tolist() == [4, 5, -1, -1]
    assert free.allocate(1) == [0] and free.allocate(1) == [1]
    assert rest == [] and new_len.tolist() == [1, 18, 33]


def test_reserve_step_all_or_nothing() -> None:
    tables = np.full((2, 2), -1, dtype=np.int64)
    lengths = np.array([0, 0])
    # exhausted: needs 2 + 1 blocks, 2 free
    status, got, _p, new_len, rest = paged_kv.reserve_step(tables, lengths, np.array([20, 5]), [7, 9], 16)
    assert status == 1 and (got == -1).all() and new_len.tolist() == [0, 0] and rest == [7, 9]
    # table too short: 40 tokens need 3 blocks of a 2-wide row
    status, got, *_ = paged_kv.reserve_step(tables, lengths, np.array([40, 0]), list(range(10)), 16)
    assert status == 2 and (got == -1).all()
    status, *_ = paged_kv.reserve_step(tables, np.array([-1, 0]), 1, list(range(10)), 16)
    assert status == 4
