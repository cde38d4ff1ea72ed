"""Oracle: paged KV block bookkeeping, slot writes and gathers (bit-exact).

Restates the integer and copy semantics of the reference cache in
``src/decode_state.py``:

* block allocation from a free list, lowest ids first, and release re-sorting
  the free list -- ``PagedKVBlockPool.allocate`` / ``.release``
  (``src/decode_state.py:72-84``);
* logical capacity growth ``max(needed, hint, max(block_size, 2*capacity))``
  -- ``FullAttentionCache._ensure_logical_capacity``
  (``src/decode_state.py:365-374``);
* the slot of token ``pos``: ``(table[pos // bs], pos % bs)`` --
  ``FullAttentionCache.append_blocks`` (``src/decode_state.py:271-293``);
* the logical-order gather of the valid tokens -- ``_gather_blocks``
  (``src/decode_state.py:395-404``);
* ``-1`` padded batch tables, lengths and validity masks --
  ``batch_page_tables`` (``src/decode_state.py:545-603``).

Everything here operates on NumPy arrays of any dtype (bf16 tensors are viewed
as ``uint16``), so results are exact copies by construction.

Pinning: ``tests/test_oracle_paged_kv.py`` checks these functions against the
known answers of the reference's own tests (``tests/unit/test_decode_state.py``
tables ``[0, 1, 2, 3]``, capacity 8, ``[[0, 1, -1], [0, 1, 2]]`` padding,
release/reuse order, non-contiguous ``[2, 0, 1]`` gathers) and against a
brute-force token-by-token restatement on small random inputs.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np


def ceil_div(value: int, divisor: int) -> int:
    return (value + divisor - 1) // divisor


@dataclass
class FreeList:
    """Free-list semantics of ``PagedKVBlockPool`` (``src/decode_state.py:26,45,70-84``)."""

    block_count: int = 0
    free: list[int] = field(default_factory=list)

    def grow(self, blocks: int) -> None:
        # ensure_initialized / add_blocks append new ids in increasing order
        # (src/decode_state.py:45,70).
        self.free.extend(range(self.block_count, self.block_count + blocks))
        self.block_count += blocks

    def allocate(self, count: int) -> list[int]:
        # src/decode_state.py:72-78: grow by the shortfall, then take the head.
        if count > len(self.free):
            self.grow(count - len(self.free))
        taken = self.free[:count]
        del self.free[:count]
        return taken

    def release(self, blocks: list[int]) -> None:
        # src/decode_state.py:80-84
        if not blocks:
            return
        self.free.extend(blocks)
        self.free.sort()


def grow_table(table: list[int], valid: int, needed: int, block_size: int, hint: int | None, free: FreeList) -> bool:
    """Extend ``table`` for ``needed`` tokens; returns True on a growth event.

    Follows ``_ensure_logical_capacity`` (``src/decode_state.py:365-374``).
    """
    del valid
    capacity = len(table) * block_size
    if needed <= capacity:
        return False
    target_tokens = max(needed, hint or 0, max(block_size, capacity * 2))
    missing = ceil_div(target_tokens, block_size) - len(table)
    if missing <= 0:
        return False
    table.extend(free.allocate(missing))
    return True


def slot_of(table: np.ndarray | list[int], pos: int, block_size: int) -> tuple[int, int]:
    """Physical (block, offset) of logical token ``pos`` (``src/decode_state.py:281-284``)."""
    return int(table[pos // block_size]), pos % block_size


def append_tokens(
    pool: np.ndarray, table: np.ndarray | list[int], start: int, new: np.ndarray, *, block_size: int, pool_layout: str
) -> None:
    """Write ``new`` tokens at logical positions ``start..`` into ``pool`` in place.

    ``new`` is head-major ``(heads, seq, dim)`` as the reference's per-request
    ``key[b]`` (``src/decode_state.py:273``).  ``pool_layout`` is either
    ``"hpbd"`` (reference layout ``(heads, P, bs, dim)`` of one batch row,
    ``src/decode_state.py:39-44``) or ``"phbd"`` (GQA-native shared layout
    ``(P, heads, bs, dim)``).  The fragment loop mirrors
    ``src/decode_state.py:278-292``.
    """
    heads, seq, _dim = new.shape
    source = 0
    write_pos = start
    while source < seq:
        logical = write_pos // block_size
        offset = write_pos % block_size
        take = min(seq - source, block_size - offset)
        physical = int(table[logical])
        if pool_layout == "hpbd":
            pool[:, physical, offset : offset + take] = new[:, source : source + take]
        elif pool_layout == "phbd":
            pool[physical, :, offset : offset + take] = new[:, source : source + take]
        else:
            raise ValueError(f"unknown pool layout {pool_layout!r}")
        source += take
        write_pos += take


def gather_tokens(pool: np.ndarray, table: np.ndarray | list[int], valid: int, *, block_size: int, pool_layout: str) -> np.ndarray:
    """Dense ``(heads, valid, dim)`` view of the first ``valid`` logical tokens.

    ``index_select`` on the block axis then flatten and truncate, as
    ``_gather_blocks`` (``src/decode_state.py:395-404``).
    """
    blocks = np.asarray([int(x) for x in table[: ceil_div(valid, block_size)]], dtype=np.int64)
    if pool_layout == "hpbd":
        picked = pool[:, blocks]  # (heads, L, bs, dim)
    elif pool_layout == "phbd":
        picked = np.transpose(pool[blocks], (1, 0, 2, 3))  # (heads, L, bs, dim)
    else:
        raise ValueError(f"unknown pool layout {pool_layout!r}")
    heads, logical, bs, dim = picked.shape
    return picked.reshape(heads, logical * bs, dim)[:, :valid]


def gather_tokens_bruteforce(pool: np.ndarray, table: list[int], valid: int, *, block_size: int, pool_layout: str) -> np.ndarray:
    """Token-by-token restatement of :func:`gather_tokens` used to pin it."""
    heads = pool.shape[0] if pool_layout == "hpbd" else pool.shape[1]
    dim = pool.shape[-1]
    out = np.empty((heads, valid, dim), dtype=pool.dtype)
    for pos in range(valid):
        physical, offset = slot_of(table, pos, block_size)
        for head in range(heads):
            if pool_layout == "hpbd":
                out[head, pos] = pool[head, physical, offset]
            else:
                out[head, pos] = pool[physical, head, offset]
    return out


@dataclass(frozen=True)
class BatchTables:
    block_tables: np.ndarray  # (B, max_blocks) int64, -1 padded
    sequence_lengths: np.ndarray  # (B,) int64
    valid_mask: np.ndarray  # (B, max_valid) bool
    max_blocks: int
    max_sequence_length: int


def batch_tables(tables: list[list[int]], valids: list[int], block_sizes: list[int]) -> BatchTables:
    """Pad per-request tables with -1 (``src/decode_state.py:545-603``)."""
    if not tables:
        raise ValueError("batch_page_tables requires at least one cache")
    if len(set(block_sizes)) != 1:
        raise ValueError("batch_page_tables requires matching block sizes")
    if not any(v > 0 for v in valids):
        raise ValueError("batch_page_tables requires at least one non-empty cache")
    max_blocks = max(len(t) for t in tables)
    max_valid = max(valids)
    out = np.full((len(tables), max_blocks), -1, dtype=np.int64)
    mask = np.zeros((len(tables), max_valid), dtype=bool)
    for row, (table, valid) in enumerate(zip(tables, valids)):
        out[row, : len(table)] = table
        mask[row, :valid] = True
    return BatchTables(out, np.asarray(valids, dtype=np.int64), mask, max_blocks, max_valid)


def slot_mapping(tables: np.ndarray, starts: np.ndarray, counts: np.ndarray, block_size: int) -> np.ndarray:
    """Flat slot ids ``table[pos // bs] * bs + pos % bs`` for each appended token.

    Rows are concatenated in order; used to pin the device append kernel.
    """
    slots: list[int] = []
    for row in range(tables.shape[0]):
        for pos in range(int(starts[row]), int(starts[row]) + int(counts[row])):
            physical, offset = slot_of(tables[row], pos, block_size)
            slots.append(physical * block_size + offset)
    return np.asarray(slots, dtype=np.int64)


def reserve_step(
    tables: np.ndarray, lengths: np.ndarray, counts: np.ndarray, free: list[int], block_size: int
) -> tuple[int, np.ndarray, np.ndarray, np.ndarray, list[int]]:
    """One batched step's block reservation over a fixed-capacity shared pool.

    Each row ``b`` in order grows from ``lengths[b]`` to ``lengths[b] + counts[b]``
    tokens; its new logical blocks ``ceil(len/bs) .. ceil((len+n)/bs) - 1`` take
    ids from the head of the free list, as ``PagedKVBlockPool.allocate`` does
    (``src/decode_state.py:72-78``) when ``FullAttentionCache._grow_to`` calls it
    once per request (``src/decode_state.py:365-374``) -- except that a shared
    pool does not grow: when the rows need more blocks than are free (status 1)
    or a row would pass the table's width (status 2), or a length/count is
    negative (status 4), nothing changes.  Returns ``(status, tables, positions,
    lengths, free)`` with ``positions`` the lengths before the step.
    """
    tables = tables.copy()
    lengths = lengths.astype(np.int64)
    counts = np.broadcast_to(np.asarray(counts, dtype=np.int64), lengths.shape)
    max_blocks = tables.shape[1]
    if (lengths < 0).any() or (counts < 0).any():
        return 4, tables, lengths.copy(), lengths.copy(), list(free)
    have = [ceil_div(int(n), block_size) for n in lengths]
    want = [ceil_div(int(n + c), block_size) for n, c in zip(lengths, counts)]
    if any(w > max_blocks for w in want):
        return 2, tables, lengths.copy(), lengths.copy(), list(free)
    if sum(w - h for w, h in zip(want, have)) > len(free):
        return 1, tables, lengths.copy(), lengths.copy(), list(free)
    free = list(free)
    for b in range(lengths.shape[0]):
        k = want[b] - have[b]
        taken, free = free[:k], free[k:]
        tables[b, have[b] : want[b]] = taken
    return 0, tables, lengths.copy(), lengths + counts, free
