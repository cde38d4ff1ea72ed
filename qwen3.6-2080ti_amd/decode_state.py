"""Paged KV cache and recurrent-state containers (drop-in for the reference's ``decode_state``).

Public names, fields, methods and counters follow ``src/decode_state.py`` of
the reference so the engine and scheduler above it run unchanged:
``PagedKVBlockPool`` (``:13-84``), ``FullAttentionPageTable`` (``:87-95``),
``BatchedFullAttentionPageTables`` (``:98-107``), the stats records
(``:110-213``), ``FullAttentionCache`` (``:216-404``),
``LinearAttentionCache`` (``:420-431``), ``DecodeState`` (``:437-498``),
``batch_kv_tensors`` (``:501-542``) and ``batch_page_tables`` (``:545-603``).

What changes underneath:

* On a GPU the slot write of ``append_blocks`` and the gather of
  ``as_tensors`` run as one HIP kernel each (``hip_ops.paged_kv_append`` /
  ``hip_ops.paged_kv_gather``) instead of a Python loop of slice copies; a
  missing library raises ``RuntimeError``.  CPU tensors keep the reference's
  own CPU semantics (host bookkeeping, used by CPU callers and tests).
* ``SharedKVBlockPool`` is a preallocated device pool ``(P, H_kv, bs, D)``
  (GQA-native, no repeated heads, one per full-attention layer) shared by
  every request; caches created with ``shared_pool=`` draw blocks from it, so
  growth never reallocates and ``batch_page_tables`` hands the decode kernel a
  single pool.
* ``LinearStatePool`` keeps recurrent and conv states of many requests in
  slot-indexed device tensors updated in place (the reference stacks and
  scatters per-request states each step, ``src/tp_runtime.py:2678-2707``).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Sequence

DEFAULT_KV_BLOCK_SIZE = 16


def _ceil_div(value: int, divisor: int) -> int:
    return -(-value // divisor)


def _nbytes(tensor: Any | None) -> int:
    if tensor is None:
        return 0
    return int(tensor.numel() * tensor.element_size())


def _on_gpu(tensor: Any) -> bool:
    return bool(getattr(tensor, "is_cuda", False))


# --------------------------------------------------------------------------- pools


@dataclass
class PagedKVBlockPool:
    """Per-cache block pool ``(batch, heads, blocks, block_size, head_dim)``.

    Same contract as ``src/decode_state.py:13-84``: storage is created on first
    use, grows by appending blocks (contents preserved), ``allocate`` hands out
    the lowest free ids and ``release`` keeps the free list sorted.
    """

    block_size: int
    key_blocks: Any | None = None
    value_blocks: Any | None = None
    free_blocks: list[int] = field(default_factory=list)

    @property
    def block_count(self) -> int:
        return 0 if self.key_blocks is None else int(self.key_blocks.shape[2])

    def _storage(self, like: Any, blocks: int) -> Any:
        import torch

        batch, heads, _seq, head_dim = like.shape
        return torch.empty((batch, heads, blocks, self.block_size, head_dim), dtype=like.dtype, device=like.device)

    def ensure_initialized(self, key: Any, value: Any, blocks: int) -> None:
        if blocks <= 0 or self.key_blocks is not None:
            return
        self.key_blocks = self._storage(key, blocks)
        self.value_blocks = self._storage(value, blocks)
        self.free_blocks = list(range(blocks))

    def add_blocks(self, key: Any, value: Any, blocks: int) -> None:
        import torch

        if blocks <= 0:
            return
        if self.key_blocks is None:
            self.ensure_initialized(key, value, blocks)
            return
        old = self.block_count

        def grown(pool: Any) -> Any:
            batch, heads, _p, bs, head_dim = pool.shape
            extra = torch.empty((batch, heads, blocks, bs, head_dim), dtype=pool.dtype, device=pool.device)
            return torch.cat([pool, extra], dim=2)

        self.key_blocks = grown(self.key_blocks)
        self.value_blocks = grown(self.value_blocks)
        self.free_blocks.extend(range(old, old + blocks))

    def allocate(self, count: int, key: Any, value: Any) -> list[int]:
        self.ensure_initialized(key, value, count)
        shortfall = count - len(self.free_blocks)
        if shortfall > 0:
            self.add_blocks(key, value, shortfall)
        taken, self.free_blocks = self.free_blocks[:count], self.free_blocks[count:]
        return taken

    def release(self, blocks: list[int]) -> None:
        if blocks:
            self.free_blocks = sorted(self.free_blocks + list(blocks))


class SharedKVBlockPool:
    """One preallocated GQA-native device pool ``(num_blocks, kv_heads, block_size, head_dim)``.

    Shared by all requests of one full-attention layer.  The free list uses the
    reference's policy (lowest ids first, sorted on release,
    ``src/decode_state.py:72-84``); there is no growth -- ``allocate`` raises
    ``RuntimeError`` when the pool is exhausted, so capacity is planned up front
    (e.g. ``ceil(sum(ctx) / bs * 1.25)`` blocks).
    """

    def __init__(self, num_blocks: int, kv_heads: int, head_dim: int, *, block_size: int = DEFAULT_KV_BLOCK_SIZE, dtype: Any = None, device: Any = None) -> None:
        import torch

        if num_blocks <= 0 or block_size <= 0:
            raise ValueError("num_blocks and block_size must be positive")
        dtype = torch.bfloat16 if dtype is None else dtype
        self.block_size = block_size
        self.kv_heads = kv_heads
        self.head_dim = head_dim
        self.key_blocks = torch.zeros((num_blocks, kv_heads, block_size, head_dim), dtype=dtype, device=device)
        self.value_blocks = torch.zeros_like(self.key_blocks)
        self.free_blocks: list[int] = list(range(num_blocks))
        self.allocator: DeviceBlockAllocator | None = None

    @classmethod
    def from_tensors(cls, key_blocks: Any, value_blocks: Any, *, free_blocks: Sequence[int] | None = None) -> "SharedKVBlockPool":
        """A pool over existing ``(P, H_kv, bs, D)`` tensors (e.g. a cache restored from elsewhere);
        ``free_blocks`` lists the ids not in use (all when omitted)."""
        if key_blocks.dim() != 4 or value_blocks.shape != key_blocks.shape:
            raise ValueError("pool tensors must be (num_blocks, kv_heads, block_size, head_dim) and alike")
        pool = cls.__new__(cls)
        pool.block_size = int(key_blocks.shape[2])
        pool.kv_heads = int(key_blocks.shape[1])
        pool.head_dim = int(key_blocks.shape[3])
        pool.key_blocks = key_blocks
        pool.value_blocks = value_blocks
        pool.free_blocks = list(range(int(key_blocks.shape[0]))) if free_blocks is None else sorted(int(b) for b in free_blocks)
        pool.allocator = None
        return pool

    @property
    def block_count(self) -> int:
        return int(self.key_blocks.shape[0])

    def allocate(self, count: int, key: Any = None, value: Any = None) -> list[int]:
        del key, value
        if self.allocator is not None:
            raise RuntimeError("shared KV pool: the free list belongs to its DeviceBlockAllocator; reserve blocks on the device")
        if count > len(self.free_blocks):
            raise RuntimeError(f"shared KV pool exhausted: need {count} blocks, {len(self.free_blocks)} free")
        taken, self.free_blocks = self.free_blocks[:count], self.free_blocks[count:]
        return taken

    def release(self, blocks: list[int]) -> None:
        """Return blocks to the free list: the host list, or the device one after ``device_allocator``."""
        if not blocks:
            return
        if self.allocator is not None:
            self.allocator.release(blocks)
            return
        self.free_blocks = sorted(self.free_blocks + list(blocks))

    def device_allocator(self) -> "DeviceBlockAllocator":
        """Hand this pool's free list to a ``DeviceBlockAllocator`` (once).

        From then on blocks are reserved on the device: the host list is emptied, host
        ``allocate`` raises, and ``release`` (e.g. ``FullAttentionCache.release`` at request
        completion) merges ids into the device list, so freed blocks stay reservable.
        """
        if self.allocator is None:
            self.allocator = DeviceBlockAllocator(self.block_count, device=self.key_blocks.device, free_blocks=self.free_blocks)
            self.free_blocks = []
        return self.allocator


class DeviceBlockAllocator:
    """Device-resident free list of a shared KV pool.

    A batched step reserves the blocks its rows need with one kernel
    (``hip_ops.paged_kv_reserve``): the ids come from the head of an ascending
    int32 list, rows in order -- the reference's lowest-free-id policy
    (``src/decode_state.py:72-78``) -- and the block tables and lengths are
    updated on the device.  A decode step of reserve, K/V append and attention
    therefore never waits for the host and can be captured in a HIP graph; the
    host reads ``status`` only when it chooses to (``check``).  ``release``
    (request completion) merges ids back and re-sorts on the host, as the
    reference's ``release`` does (``src/decode_state.py:80-84``).
    """

    def __init__(self, num_blocks: int, *, device: Any, free_blocks: Sequence[int] | None = None) -> None:
        import torch

        if num_blocks <= 0:
            raise ValueError("num_blocks must be positive")
        ids = list(range(num_blocks)) if free_blocks is None else sorted(int(i) for i in free_blocks)
        if ids and (ids[0] < 0 or ids[-1] >= num_blocks or len(set(ids)) != len(ids)):
            raise ValueError("free block ids must be distinct and in [0, num_blocks)")
        self.capacity = num_blocks
        self.device = torch.device(device)
        self.free_list = torch.full((num_blocks,), -1, dtype=torch.int32, device=self.device)
        if ids:
            self.free_list[: len(ids)] = torch.tensor(ids, dtype=torch.int32, device=self.device)
        self.free_state = torch.tensor([0, len(ids)], dtype=torch.int32, device=self.device)
        self.status = torch.zeros(1, dtype=torch.int32, device=self.device)

    _STATUS = {
        1: "shared KV pool exhausted",
        2: "block table too short for the reserved blocks",
        3: "device free list state is corrupt",
        4: "negative or overflowing length/count",
    }

    def reserve(self, block_tables: Any, lengths: Any, block_size: int, *, counts: Any = 1, positions: Any = None) -> None:
        """Reserve blocks for ``counts`` new tokens per row; advances ``lengths`` in place."""
        import hip_ops

        hip_ops.paged_kv_reserve(block_tables, lengths, self.free_list, self.free_state, self.status, block_size, counts=counts, positions=positions)

    def check(self) -> None:
        """Raise ``RuntimeError`` if the last reservation failed (reads the status: a sync)."""
        code = int(self.status.item())
        if code != 0:
            raise RuntimeError(f"paged_kv_reserve failed: {self._STATUS.get(code, f'status {code}')}")

    def free_blocks(self) -> list[int]:
        head, count = (int(v) for v in self.free_state.tolist())
        return [int(v) for v in self.free_list[head : head + count].tolist()]

    @property
    def free_count(self) -> int:
        return int(self.free_state[1].item())

    def release(self, blocks: Sequence[int]) -> None:
        import torch

        blocks = [int(b) for b in blocks]
        if not blocks:
            return
        merged = sorted(self.free_blocks() + blocks)
        if merged[0] < 0 or merged[-1] >= self.capacity or len(set(merged)) != len(merged):
            raise ValueError("released block ids must be in range and not already free")
        self.free_list[: len(merged)] = torch.tensor(merged, dtype=torch.int32, device=self.device)
        self.free_state.copy_(torch.tensor([0, len(merged)], dtype=torch.int32))


class DeviceBatchPageTables:
    """Block tables and lengths of the rows of a running decode batch, kept on the device.

    The reference rebuilds ``-1``-padded ``(B, max_blocks)`` tables on the host for every
    full-attention layer of every step and copies them to the device (``batch_page_tables``,
    ``src/decode_state.py:545-603``; its engine probe counts those rebuilds,
    ``src/engine.py:489-516``).  Here a running batch keeps one ``(rows, max_blocks)`` int32
    table, ``(rows,)`` int32 lengths and per-row step token counts on the device:
    ``reserve_step`` grows every active row by its step count with one kernel (ids from the
    pool's device free list, lowest first, rows in order: ``PagedKVBlockPool.allocate``'s
    policy, ``:72-78``) and leaves the append positions in ``positions``; ``append`` writes a
    layer's step K/V there.  The full-attention layers of a model grow their caches identically
    (every layer appends the same tokens), so layers whose pools have the same block count share
    one table and a step reserves once for all of them.  ``reserve_step``, ``append`` and the
    decode neither read back to the host nor copy host to device, so a whole decode step can be
    captured in a HIP graph; the host touches the tables only when a request joins
    (``add_request``) or finishes (``release_request``).
    """

    def __init__(self, pool: SharedKVBlockPool, rows: int, max_blocks: int) -> None:
        import torch

        if rows <= 0 or max_blocks <= 0:
            raise ValueError("rows and max_blocks must be positive")
        self.pool = pool
        self.block_size = pool.block_size
        self.num_blocks = pool.block_count
        self.allocator = pool.device_allocator()
        device = pool.key_blocks.device
        self.block_tables = torch.full((rows, max_blocks), -1, dtype=torch.int32, device=device)
        self.sequence_lengths = torch.zeros(rows, dtype=torch.int32, device=device)
        self.positions = torch.zeros(rows, dtype=torch.int32, device=device)
        # the append positions of an admission reserve: kept apart from `positions`, so a request
        # admitted between a step's reserve and its per-layer appends leaves that step's positions
        self._admit_positions = torch.zeros(rows, dtype=torch.int32, device=device)
        self.step_counts = torch.zeros(rows, dtype=torch.int32, device=device)
        self.active = [False] * rows

    @property
    def rows(self) -> int:
        return len(self.active)

    def add_request(self, prompt_tokens: int = 0) -> int:
        """Take the lowest free row for a new request and reserve blocks for ``prompt_tokens``
        tokens (whose K/V the caller then writes at positions 0 ..).  The row joins later steps
        with one token each.  ``positions`` (the append positions of the current step) is left
        as it is, so a request may be admitted between a step's ``reserve_step`` and its
        appends.  A prompt that is to run through :func:`attention_runtime.full_attention_prefill_device`
        is admitted with ``prompt_tokens=0`` and reserved by :meth:`reserve_prefill` instead."""
        import torch

        if prompt_tokens < 0:
            raise ValueError("prompt_tokens must be non-negative")
        try:
            row = self.active.index(False)
        except ValueError:
            raise RuntimeError("device page tables: every row holds a request") from None
        self.active[row] = True
        if prompt_tokens:
            counts = torch.zeros_like(self.step_counts)
            counts[row] = prompt_tokens
            self.allocator.reserve(self.block_tables, self.sequence_lengths, self.block_size, counts=counts, positions=self._admit_positions)
            self.allocator.check()
        self.step_counts[row] = 1
        return row

    def reserve_prefill(self, rows: Sequence[int], counts: Sequence[int]) -> "PrefillStep":
        """Reserve blocks for a multi-token step (a prompt, or one chunk of it) of some rows.

        Row ``rows[i]`` grows by ``counts[i]`` tokens; the step's tokens are packed in that
        order (row ``rows[i]`` owns ``cu_seqlens[i]:cu_seqlens[i + 1]``).  Like ``reserve_step``
        it runs once for all full-attention layers sharing these tables, and the returned record
        feeds each layer's :func:`attention_runtime.full_attention_prefill_device`.  Other rows
        keep their lengths and the step positions of ``reserve_step``.  Reads the reservation
        status back (one sync), so a failed reservation raises here rather than in a layer."""
        import torch

        rows = [int(r) for r in rows]
        counts = [int(c) for c in counts]
        if not rows or len(rows) != len(counts):
            raise ValueError("reserve_prefill needs one count per row")
        if len(set(rows)) != len(rows) or min(rows) < 0 or max(rows) >= self.rows:
            raise ValueError("reserve_prefill rows must be distinct table rows")
        if min(counts) <= 0:
            raise ValueError("reserve_prefill counts must be positive")
        for r in rows:
            if not self.active[r]:
                raise ValueError(f"row {r} holds no request")
        device = self.block_tables.device
        index = torch.tensor(rows, dtype=torch.int64, device=device)
        full = torch.zeros_like(self.step_counts)
        full[index] = torch.tensor(counts, dtype=torch.int32, device=device)
        self.allocator.reserve(self.block_tables, self.sequence_lengths, self.block_size, counts=full, positions=self._admit_positions)
        self.allocator.check()
        cu = [0]
        for c in counts:
            cu.append(cu[-1] + c)
        return PrefillStep(
            rows=tuple(rows), counts=tuple(counts), index=index,
            cu_seqlens=torch.tensor(cu, dtype=torch.int32, device=device),
            starts=self._admit_positions.index_select(0, index),
            block_tables=self.block_tables.index_select(0, index),
            max_new=max(counts), total_tokens=cu[-1], block_size=self.block_size,
        )

    def adopt_rows(self, block_tables: Any, lengths: Any) -> None:
        """Take over requests whose blocks are already written: row ``r`` gets ``block_tables[r]``
        (``-1`` padded) and ``lengths[r]`` tokens.  Their ids must not be in the pool's free list
        (``SharedKVBlockPool.from_tensors(..., free_blocks=...)``)."""
        import torch

        rows, width = block_tables.shape
        if rows > self.rows or width > self.block_tables.shape[1]:
            raise ValueError("adopted tables do not fit the device tables")
        self.block_tables[:rows].fill_(-1)
        self.block_tables[:rows, :width] = block_tables.to(device=self.block_tables.device, dtype=torch.int32)
        self.sequence_lengths[:rows] = lengths.to(device=self.block_tables.device, dtype=torch.int32)
        self.step_counts[:rows] = 1
        for r in range(rows):
            self.active[r] = True

    def reserve_step(self) -> None:
        """Blocks for one step of every active row (device only; ``check`` reads the status)."""
        self.allocator.reserve(self.block_tables, self.sequence_lengths, self.block_size, counts=self.step_counts, positions=self.positions)

    def append(self, key: Any, value: Any, key_blocks: Any, value_blocks: Any, *, counts: Any = None) -> None:
        """Write a layer's new K/V ``(rows, H_kv, S, D)`` at the reserved positions of its pool."""
        import hip_ops

        hip_ops.paged_kv_append(key, value, key_blocks, value_blocks, self.block_tables, self.positions, self.block_size,
                                counts=self.step_counts if counts is None else counts)

    def check(self) -> None:
        self.allocator.check()

    def release_request(self, row: int) -> list[int]:
        """The request in ``row`` finished: its blocks return to the device free list (one read of
        the row) and the row is emptied.  Returns the released block ids."""
        if not self.active[row]:
            raise ValueError(f"row {row} holds no request")
        ids = [int(b) for b in self.block_tables[row].tolist() if b >= 0]
        self.allocator.release(ids)
        self.block_tables[row].fill_(-1)
        self.sequence_lengths[row] = 0
        self.step_counts[row] = 0
        self.active[row] = False
        return ids


@dataclass(frozen=True)
class PrefillStep:
    """The reservation of one multi-token step (``DeviceBatchPageTables.reserve_prefill``):
    rows in packing order, their new token counts, ``cu_seqlens`` ``(n + 1,)`` and the first
    new position ``starts`` ``(n,)`` of each row (its length before the step), and the rows'
    block tables ``(n, max_blocks)`` after the reservation, all int32 on the device."""

    rows: tuple[int, ...]
    counts: tuple[int, ...]
    index: Any
    cu_seqlens: Any
    starts: Any
    block_tables: Any
    max_new: int
    total_tokens: int
    block_size: int


# --------------------------------------------------------------------------- records


@dataclass(frozen=True)
class FullAttentionPageTable:
    block_table: Any
    sequence_length: int
    block_size: int
    logical_blocks: int
    capacity_tokens: int
    key_blocks: Any
    value_blocks: Any


@dataclass(frozen=True)
class BatchedFullAttentionPageTables:
    block_tables: Any
    sequence_lengths: Any
    valid_mask: Any
    block_size: int
    max_blocks: int
    max_sequence_length: int
    key_blocks: tuple[Any, ...]
    value_blocks: tuple[Any, ...]


@dataclass(frozen=True)
class FullAttentionCacheStats:
    block_size: int
    valid_tokens: int
    capacity_tokens: int
    logical_blocks: int
    allocated_blocks: int
    free_blocks: int
    append_calls: int
    appended_tokens: int
    growth_events: int
    release_calls: int
    released_blocks: int
    contiguous_view_calls: int
    gather_view_calls: int
    gather_copied_tokens: int
    page_table_tensor_calls: int
    page_metadata_calls: int
    batched_page_table_calls: int
    page_table_entries_total: int
    non_contiguous: bool
    estimated_key_bytes: int
    estimated_value_bytes: int
    estimated_total_bytes: int

    def to_dict(self) -> dict[str, int | bool]:
        return dict(vars(self))


@dataclass(frozen=True)
class KVCacheStats:
    full_attention_layers: int
    block_size: int | None
    valid_tokens_total: int
    capacity_tokens_total: int
    logical_blocks_total: int
    allocated_blocks_total: int
    free_blocks_total: int
    append_calls_total: int
    appended_tokens_total: int
    growth_events_total: int
    release_calls_total: int
    released_blocks_total: int
    contiguous_view_calls_total: int
    gather_view_calls_total: int
    gather_copied_tokens_total: int
    page_table_tensor_calls_total: int
    page_metadata_calls_total: int
    batched_page_table_calls_total: int
    page_table_entries_total: int
    non_contiguous_layers: int
    estimated_total_bytes: int
    max_valid_tokens: int
    max_capacity_tokens: int

    def to_dict(self) -> dict[str, int | None]:
        return dict(vars(self))


# --------------------------------------------------------------------------- caches


@dataclass
class FullAttentionCache:
    """Paged per-layer KV cache of one request.

    ``append`` / ``append_blocks`` take post-rotary K/V ``(1 or batch, heads,
    seq, head_dim)``; ``block_table`` maps logical blocks to physical ones.
    With ``shared_pool`` set, ``heads`` is the KV head count of the shared
    GQA-native pool and the cache's batch dimension must be 1.
    """

    capacity_hint: int | None = None
    block_size: int = DEFAULT_KV_BLOCK_SIZE
    valid: int = 0
    block_table: list[int] = field(default_factory=list)
    shared_pool: SharedKVBlockPool | None = None
    pool: Any = field(init=False)
    _table_cache: Any = field(default=None, init=False, repr=False, compare=False)
    append_calls: int = 0
    appended_tokens: int = 0
    growth_events: int = 0
    release_calls: int = 0
    released_blocks: int = 0
    contiguous_view_calls: int = 0
    gather_view_calls: int = 0
    gather_copied_tokens: int = 0
    page_table_tensor_calls: int = 0
    page_metadata_calls: int = 0
    batched_page_table_calls: int = 0
    page_table_entries_total: int = 0

    def __post_init__(self) -> None:
        if self.block_size <= 0:
            raise ValueError("block_size must be positive")
        if self.shared_pool is not None:
            if self.shared_pool.block_size != self.block_size:
                raise ValueError("shared pool block size differs from the cache block size")
            self.pool = self.shared_pool
        else:
            self.pool = PagedKVBlockPool(self.block_size)

    @property
    def key_blocks(self) -> Any | None:
        return self.pool.key_blocks

    @property
    def value_blocks(self) -> Any | None:
        return self.pool.value_blocks

    @property
    def length(self) -> int:
        return self.valid

    @property
    def capacity(self) -> int:
        return len(self.block_table) * self.block_size

    def append(self, key: Any, value: Any) -> tuple[Any, Any]:
        self.append_blocks(key, value)
        return self.as_tensors()

    def append_blocks(self, key: Any, value: Any) -> None:
        """Write new K/V into slots ``(table[pos // bs], pos % bs)`` (``src/decode_state.py:271-293``)."""
        seq = int(key.shape[2])
        self.append_calls += 1
        self.appended_tokens += seq
        target = self.valid + seq
        self._grow_to(target, key, value)
        if seq:
            if _on_gpu(key):
                self._device_append(key, value)
            else:
                self._host_append(key, value)
        self.valid = target

    def _host_append(self, key: Any, value: Any) -> None:
        """CPU slot copies, one fragment (run of tokens inside one block) at a time."""
        bs = self.block_size
        seq = int(key.shape[2])
        done = 0
        while done < seq:
            pos = self.valid + done
            physical, offset = self.block_table[pos // bs], pos % bs
            take = min(seq - done, bs - offset)
            src = slice(done, done + take)
            dst = slice(offset, offset + take)
            if self.shared_pool is not None:
                self.pool.key_blocks[physical, :, dst] = key[0, :, src]
                self.pool.value_blocks[physical, :, dst] = value[0, :, src]
            else:
                self.pool.key_blocks[:, :, physical, dst] = key[:, :, src]
                self.pool.value_blocks[:, :, physical, dst] = value[:, :, src]
            done += take

    def _device_append(self, key: Any, value: Any) -> None:
        import torch

        import hip_ops

        table = torch.tensor(self.block_table, dtype=torch.int32, device=key.device)
        if self.shared_pool is not None:
            if key.shape[0] != 1:
                raise ValueError("caches on a shared pool hold one request (batch 1)")
            hip_ops.paged_kv_append(key, value, self.pool.key_blocks, self.pool.value_blocks, table, self.valid, self.block_size)
            return
        # reference-layout pool (batch, heads, P, bs, D): every batch row shares the table
        for row in range(key.shape[0]):
            hip_ops.paged_kv_append(
                key[row : row + 1], value[row : row + 1], self.pool.key_blocks[row : row + 1], self.pool.value_blocks[row : row + 1],
                table, self.valid, self.block_size,
            )

    def as_tensors(self) -> tuple[Any, Any]:
        """Dense ``(batch, heads, valid, D)`` K/V (``src/decode_state.py:295-303``)."""
        if self.valid == 0:
            raise ValueError("FullAttentionCache has no valid tokens")
        if self.shared_pool is None and self._is_contiguous_table():
            self.contiguous_view_calls += 1
            return self._contiguous_view(self.pool.key_blocks), self._contiguous_view(self.pool.value_blocks)
        self.gather_view_calls += 1
        self.gather_copied_tokens += self.valid
        return self._gather()

    def page_table_tensor(self, *, device: Any | None = None) -> Any:
        import torch

        if device is None and self.pool.key_blocks is not None:
            device = self.pool.key_blocks.device
        self.page_table_tensor_calls += 1
        key = (str(device), tuple(self.block_table))
        cached = self._table_cache
        if cached is None or cached[0] != key:
            # the device copy is rebuilt only when the table changed (the reference
            # copies it host to device on every call, src/decode_state.py:87-95)
            cached = (key, torch.tensor(self.block_table, dtype=torch.long, device=device))
            self._table_cache = cached
        return cached[1]

    def page_metadata(self) -> FullAttentionPageTable:
        if self.pool.key_blocks is None or self.pool.value_blocks is None:
            raise ValueError("FullAttentionCache page metadata requires allocated block storage")
        table = self.page_table_tensor(device=self.pool.key_blocks.device)
        self.page_metadata_calls += 1
        self.page_table_entries_total += len(self.block_table)
        return FullAttentionPageTable(
            block_table=table,
            sequence_length=self.valid,
            block_size=self.block_size,
            logical_blocks=len(self.block_table),
            capacity_tokens=self.capacity,
            key_blocks=self.pool.key_blocks,
            value_blocks=self.pool.value_blocks,
        )

    def release(self) -> None:
        self.release_calls += 1
        self.released_blocks += len(self.block_table)
        self.pool.release(self.block_table)
        self.block_table = []
        self.valid = 0

    def stats(self) -> FullAttentionCacheStats:
        key_bytes = _nbytes(self.pool.key_blocks)
        value_bytes = _nbytes(self.pool.value_blocks)
        return FullAttentionCacheStats(
            block_size=self.block_size,
            valid_tokens=self.valid,
            capacity_tokens=self.capacity,
            logical_blocks=len(self.block_table),
            allocated_blocks=self.pool.block_count,
            free_blocks=len(self.pool.free_blocks),
            append_calls=self.append_calls,
            appended_tokens=self.appended_tokens,
            growth_events=self.growth_events,
            release_calls=self.release_calls,
            released_blocks=self.released_blocks,
            contiguous_view_calls=self.contiguous_view_calls,
            gather_view_calls=self.gather_view_calls,
            gather_copied_tokens=self.gather_copied_tokens,
            page_table_tensor_calls=self.page_table_tensor_calls,
            page_metadata_calls=self.page_metadata_calls,
            batched_page_table_calls=self.batched_page_table_calls,
            page_table_entries_total=self.page_table_entries_total,
            non_contiguous=not self._is_contiguous_table(),
            estimated_key_bytes=key_bytes,
            estimated_value_bytes=value_bytes,
            estimated_total_bytes=key_bytes + value_bytes,
        )

    # -- internals ------------------------------------------------------------

    def _grow_to(self, needed: int, key: Any, value: Any) -> None:
        """Logical capacity policy of ``src/decode_state.py:365-374``."""
        if needed <= self.capacity:
            return
        target_tokens = max(needed, self.capacity_hint or 0, max(self.block_size, 2 * self.capacity))
        missing = _ceil_div(target_tokens, self.block_size) - len(self.block_table)
        if missing <= 0:
            return
        self.growth_events += 1
        self.block_table.extend(self.pool.allocate(missing, key, value))

    def _is_contiguous_table(self) -> bool:
        table = self.block_table
        return all(b - a == 1 for a, b in zip(table, table[1:]))

    def _contiguous_view(self, blocks: Any) -> Any:
        batch, heads, _p, bs, head_dim = blocks.shape
        logical = len(self.block_table)
        start = self.block_table[0]
        flat = blocks.as_strided(
            (batch, heads, logical * bs, head_dim),
            (blocks.stride(0), blocks.stride(1), blocks.stride(3), blocks.stride(4)),
            storage_offset=blocks.storage_offset() + start * blocks.stride(2),
        )
        return flat[:, :, : self.valid]

    def _gather(self) -> tuple[Any, Any]:
        import torch

        keys, values = self.pool.key_blocks, self.pool.value_blocks
        if _on_gpu(keys):
            import hip_ops

            table = torch.tensor(self.block_table, dtype=torch.int32, device=keys.device)
            if self.shared_pool is not None:
                return hip_ops.paged_kv_gather(keys, values, table, self.valid, self.block_size)
            return hip_ops.paged_kv_gather(keys, values, table, self.valid, self.block_size)
        index = torch.tensor(self.block_table, dtype=torch.long)
        if self.shared_pool is not None:
            picked_k = keys.index_select(0, index).transpose(0, 1).unsqueeze(0)
            picked_v = values.index_select(0, index).transpose(0, 1).unsqueeze(0)
        else:
            picked_k = keys.index_select(2, index)
            picked_v = values.index_select(2, index)
        b, h, n, bs, d = picked_k.shape
        return picked_k.reshape(b, h, n * bs, d)[:, :, : self.valid], picked_v.reshape(b, h, n * bs, d)[:, :, : self.valid]


@dataclass
class LinearAttentionCache:
    """Recurrent ``state`` ``(batch, H_v, dk, dv)`` fp32 and ``conv_tail`` ``(batch, C, K-1)``.

    Lazily created, as ``src/decode_state.py:420-431``.  With ``slot`` set the
    request's state lives in row ``slot`` of a :class:`LinearStatePool`.
    """

    state: Any | None = None
    conv_tail: Any | None = None
    slot: int | None = None


class LinearStatePool:
    """Slot-indexed device storage for the recurrent and conv states of many requests.

    ``state`` ``(slots, H_v, dk, dv)`` fp32 and ``conv`` ``(slots, C, K-1)`` fp32
    are updated in place by the fused decode kernel; ``acquire`` zero-fills a
    slot for a new request.
    """

    def __init__(self, slots: int, value_heads: int, key_dim: int, value_dim: int, channels: int, conv_kernel: int, *, device: Any = None) -> None:
        import torch

        self.state = torch.zeros((slots, value_heads, key_dim, value_dim), dtype=torch.float32, device=device)
        self.conv = torch.zeros((slots, channels, conv_kernel - 1), dtype=torch.float32, device=device)
        self.free_slots: list[int] = list(range(slots))

    def acquire(self) -> int:
        if not self.free_slots:
            raise RuntimeError("linear state pool exhausted")
        slot = self.free_slots.pop(0)
        self.state[slot].zero_()
        self.conv[slot].zero_()
        return slot

    def release(self, slot: int) -> None:
        self.free_slots = sorted(self.free_slots + [slot])


LayerCache = FullAttentionCache | LinearAttentionCache


@dataclass
class DecodeState:
    """Per-layer decode caches plus the number of consumed tokens (``src/decode_state.py:437-498``)."""

    layers: list[LayerCache]
    position_offset: int = 0

    @classmethod
    def empty(
        cls,
        mapping: Any,
        config: Any = None,
        max_seq_len: int | None = None,
        *,
        kv_block_size: int = DEFAULT_KV_BLOCK_SIZE,
        shared_pools: dict[int, SharedKVBlockPool] | None = None,
    ) -> "DecodeState":
        del config
        layers: list[LayerCache] = []
        for layer in mapping.layers:
            if layer.layer_type == "full_attention":
                pool = None if shared_pools is None else shared_pools.get(layer.index)
                layers.append(FullAttentionCache(capacity_hint=max_seq_len, block_size=kv_block_size, shared_pool=pool))
            else:
                layers.append(LinearAttentionCache())
        return cls(layers=layers, position_offset=0)

    def advance(self, tokens: int) -> None:
        self.position_offset += tokens

    def release(self) -> None:
        for layer in self.layers:
            if isinstance(layer, FullAttentionCache):
                layer.release()

    def kv_stats(self) -> KVCacheStats:
        stats = [layer.stats() for layer in self.layers if isinstance(layer, FullAttentionCache)]
        sizes = {s.block_size for s in stats}

        def total(name: str) -> int:
            return sum(getattr(s, name) for s in stats)

        return KVCacheStats(
            full_attention_layers=len(stats),
            block_size=next(iter(sizes)) if len(sizes) == 1 else None,
            valid_tokens_total=total("valid_tokens"),
            capacity_tokens_total=total("capacity_tokens"),
            logical_blocks_total=total("logical_blocks"),
            allocated_blocks_total=total("allocated_blocks"),
            free_blocks_total=total("free_blocks"),
            append_calls_total=total("append_calls"),
            appended_tokens_total=total("appended_tokens"),
            growth_events_total=total("growth_events"),
            release_calls_total=total("release_calls"),
            released_blocks_total=total("released_blocks"),
            contiguous_view_calls_total=total("contiguous_view_calls"),
            gather_view_calls_total=total("gather_view_calls"),
            gather_copied_tokens_total=total("gather_copied_tokens"),
            page_table_tensor_calls_total=total("page_table_tensor_calls"),
            page_metadata_calls_total=total("page_metadata_calls"),
            batched_page_table_calls_total=total("batched_page_table_calls"),
            page_table_entries_total=total("page_table_entries_total"),
            non_contiguous_layers=sum(1 for s in stats if s.non_contiguous),
            estimated_total_bytes=total("estimated_total_bytes"),
            max_valid_tokens=max((s.valid_tokens for s in stats), default=0),
            max_capacity_tokens=max((s.capacity_tokens for s in stats), default=0),
        )


# --------------------------------------------------------------------------- batch helpers


def batch_kv_tensors(caches: Sequence[FullAttentionCache]) -> tuple[Any, Any, Any]:
    """Zero-padded dense K/V of several requests plus a validity mask (``src/decode_state.py:501-542``)."""
    import torch

    if not caches:
        raise ValueError("batch_kv_tensors requires at least one cache")
    longest = max(cache.valid for cache in caches)
    if longest == 0:
        raise ValueError("batch_kv_tensors requires at least one non-empty cache")
    dense = [cache.as_tensors() if cache.valid else None for cache in caches]
    sample = next(k for k in dense if k is not None)[0]
    shape = (len(caches), sample.shape[1], longest, sample.shape[3])
    keys = torch.zeros(shape, dtype=sample.dtype, device=sample.device)
    values = torch.zeros(shape, dtype=sample.dtype, device=sample.device)
    mask = torch.zeros((len(caches), longest), dtype=torch.bool, device=sample.device)
    for row, (cache, kv) in enumerate(zip(caches, dense)):
        if kv is None:
            continue
        keys[row : row + 1, :, : cache.valid] = kv[0]
        values[row : row + 1, :, : cache.valid] = kv[1]
        mask[row, : cache.valid] = True
    return keys, values, mask


def batch_page_tables(caches: Sequence[FullAttentionCache]) -> BatchedFullAttentionPageTables:
    """``-1``-padded ``(B, max_blocks)`` int64 tables, lengths and mask (``src/decode_state.py:545-603``).

    The padded table is assembled on the host and copied once; per-cache
    counters advance exactly as in the reference.
    """
    import torch

    if not caches:
        raise ValueError("batch_page_tables requires at least one cache")
    if len({cache.block_size for cache in caches}) != 1:
        raise ValueError("batch_page_tables requires matching block sizes")
    if not any(cache.valid > 0 for cache in caches):
        raise ValueError("batch_page_tables requires at least one non-empty cache")
    storage = next((c for c in caches if c.valid > 0 and c.key_blocks is not None and c.value_blocks is not None), None)
    if storage is None:
        raise ValueError("batch_page_tables requires allocated block storage")
    device = storage.key_blocks.device
    max_blocks = max(len(cache.block_table) for cache in caches)
    longest = max(cache.valid for cache in caches)
    host = torch.full((len(caches), max_blocks), -1, dtype=torch.long)
    for row, cache in enumerate(caches):
        if cache.valid > 0 and (cache.key_blocks is None or cache.value_blocks is None):
            raise ValueError("batch_page_tables requires allocated block storage for non-empty caches")
        cache.batched_page_table_calls += 1
        cache.page_table_entries_total += len(cache.block_table)
        cache.page_table_tensor_calls += 1
        if cache.block_table:
            host[row, : len(cache.block_table)] = torch.tensor(cache.block_table, dtype=torch.long)
    lengths_host = torch.tensor([cache.valid for cache in caches], dtype=torch.long)
    mask_host = torch.arange(longest).unsqueeze(0) < lengths_host.unsqueeze(1)
    return BatchedFullAttentionPageTables(
        block_tables=host.to(device),
        sequence_lengths=lengths_host.to(device),
        valid_mask=mask_host.to(device),
        block_size=caches[0].block_size,
        max_blocks=max_blocks,
        max_sequence_length=longest,
        key_blocks=tuple(cache.key_blocks for cache in caches),
        value_blocks=tuple(cache.value_blocks for cache in caches),
    )
