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
