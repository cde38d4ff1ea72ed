"""Host logic of ``decode_state`` against the reference's known answers.

Each test restates a test of the reference's ``tests/unit/test_decode_state.py``
(line numbers cited) on this package's ``decode_state``, plus the shared-pool
additions.  CPU tensors only.
"""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

from decode_state import (
    DEFAULT_KV_BLOCK_SIZE,
    DecodeState,
    FullAttentionCache,
    LinearAttentionCache,
    SharedKVBlockPool,
    batch_kv_tensors,
    batch_page_tables,
)


def _kv(step: int, *, batch: int = 1, heads: int = 2, seq: int = 1, head_dim: int = 4):
    """Token tensors tagged with their step: element i of step s is s * 4096 + i (keys) and its
    negation (values), so a token written to the wrong slot or returned in the wrong order
    changes the compared tensors."""
    shape = (batch, heads, seq, head_dim)
    tagged = torch.arange(batch * heads * seq * head_dim, dtype=torch.float32).reshape(shape) + float(4096 * step)
    return tagged, -tagged - 1.0


def _mapping(layer_types):
    """A model-layer mapping with only the fields ``DecodeState.empty`` reads (index, layer_type)."""
    layers = [SimpleNamespace(index=i, layer_type=kind) for i, kind in enumerate(layer_types)]
    return SimpleNamespace(layers=tuple(layers))


def test_append_returns_views_equal_to_manual_concat() -> None:  # :33-44
    cache = FullAttentionCache(block_size=2)
    keys, values = [], []
    for step in range(5):
        key, value = _kv(step)
        keys.append(key)
        values.append(value)
        out_key, out_value = cache.append(key, value)
        torch.testing.assert_close(out_key, torch.cat(keys, dim=2))
        torch.testing.assert_close(out_value, torch.cat(values, dim=2))


def test_prefill_chunk_then_single_steps_across_blocks() -> None:  # :47-63
    cache = FullAttentionCache(block_size=2)
    pk, pv = _kv(0, seq=3)
    keys, values = [pk], [pv]
    cache.append(pk, pv)
    for step in range(1, 4):
        key, value = _kv(step)
        keys.append(key)
        values.append(value)
        out_key, out_value = cache.append(key, value)
    torch.testing.assert_close(out_key, torch.cat(keys, dim=2))
    torch.testing.assert_close(out_value, torch.cat(values, dim=2))
    assert cache.block_table == [0, 1, 2, 3]
    assert cache.capacity == 8


def test_append_blocks_without_dense_view_then_metadata() -> None:  # :66-89
    cache = FullAttentionCache(capacity_hint=4, block_size=2)
    key, value = _kv(0, seq=3)
    cache.append_blocks(key, value)
    assert (cache.length, cache.capacity, cache.block_table) == (3, 4, [0, 1])
    stats = cache.stats()
    assert (stats.append_calls, stats.appended_tokens, stats.contiguous_view_calls, stats.gather_view_calls) == (1, 3, 0, 0)
    metadata = cache.page_metadata()
    assert metadata.block_table.tolist() == [0, 1]
    assert metadata.sequence_length == 3
    assert metadata.key_blocks is cache.key_blocks
    out_key, out_value = cache.as_tensors()
    torch.testing.assert_close(out_key, key)
    torch.testing.assert_close(out_value, value)


def test_capacity_hint_and_contiguous_view_alias_storage() -> None:  # :92-138
    cache = FullAttentionCache(capacity_hint=8, block_size=4)
    assert cache.length == 0 and cache.capacity == 0
    out_key, _ = cache.append(*_kv(0, seq=3))
    assert cache.pool.block_count == 2 and cache.block_table == [0, 1] and cache.pool.free_blocks == []
    assert out_key.shape == (1, 2, 3, 4)
    ptr = cache.key_blocks.data_ptr()
    assert out_key.data_ptr() == ptr
    out_key, _ = cache.append(*_kv(1, seq=2))
    assert cache.key_blocks.data_ptr() == ptr and out_key.shape[2] == 5


def test_growth_beyond_hint_preserves_contents() -> None:  # :141-155
    cache = FullAttentionCache(capacity_hint=2, block_size=2)
    keys = []
    for step in range(6):
        key, value = _kv(step)
        keys.append(key)
        out_key, _ = cache.append(key, value)
    assert cache.pool.block_count >= len(cache.block_table)
    torch.testing.assert_close(out_key, torch.cat(keys, dim=2))


def test_release_reuses_blocks() -> None:  # :158-173
    cache = FullAttentionCache(capacity_hint=4, block_size=2)
    cache.append(*_kv(0, seq=3))
    released = list(cache.block_table)
    ptr = cache.key_blocks.data_ptr()
    cache.release()
    assert cache.length == 0 and cache.block_table == [] and cache.pool.free_blocks == released
    out_key, _ = cache.append(*_kv(1, seq=2))
    assert cache.block_table == released and cache.key_blocks.data_ptr() == ptr
    torch.testing.assert_close(out_key, _kv(1, seq=2)[0])


def test_stats_track_append_and_views() -> None:  # :176-190
    cache = FullAttentionCache(capacity_hint=4, block_size=2)
    cache.append(*_kv(0, seq=3))
    cache.as_tensors()
    stats = cache.stats()
    assert (stats.append_calls, stats.appended_tokens, stats.growth_events) == (1, 3, 1)
    assert (stats.contiguous_view_calls, stats.gather_view_calls, stats.valid_tokens, stats.capacity_tokens) == (2, 0, 3, 4)
    assert stats.estimated_total_bytes > 0


def test_non_contiguous_gather_matches_logical_order() -> None:  # :194-218
    cache = FullAttentionCache(capacity_hint=6, block_size=2)
    chunks = [_kv(i, seq=2) for i in range(3)]
    for k, v in chunks:
        cache.append(k, v)
    cache.block_table = [2, 0, 1]
    for physical, (k, v) in zip([2, 0, 1], chunks):
        cache.pool.key_blocks[:, :, physical] = k
        cache.pool.value_blocks[:, :, physical] = v
    out_key, out_value = cache.as_tensors()
    torch.testing.assert_close(out_key, torch.cat([c[0] for c in chunks], dim=2))
    torch.testing.assert_close(out_value, torch.cat([c[1] for c in chunks], dim=2))
    stats = cache.stats()
    assert (stats.gather_view_calls, stats.gather_copied_tokens, stats.non_contiguous) == (1, 6, True)


def test_dtype_and_device_preserved() -> None:  # :221-230
    cache = FullAttentionCache(capacity_hint=4)
    out_key, out_value = cache.append(torch.zeros((1, 2, 1, 4), dtype=torch.float64), torch.ones((1, 2, 1, 4), dtype=torch.float64))
    assert out_key.dtype == torch.float64 and out_value.dtype == torch.float64


def test_decode_state_empty_and_release() -> None:  # :233-296
    state = DecodeState.empty(_mapping(("full_attention", "linear_attention", "full_attention")), None, max_seq_len=16, kv_block_size=4)
    full = [c for c in state.layers if isinstance(c, FullAttentionCache)]
    assert len(full) == 2 and all(c.capacity_hint == 16 and c.block_size == 4 for c in full)
    assert sum(isinstance(c, LinearAttentionCache) for c in state.layers) == 1
    default = DecodeState.empty(_mapping(("full_attention",)))
    assert default.layers[0].block_size == DEFAULT_KV_BLOCK_SIZE and default.layers[0].key_blocks is None
    small = DecodeState.empty(_mapping(("full_attention", "linear_attention", "full_attention")), None, max_seq_len=4, kv_block_size=2)
    for layer in small.layers:
        if isinstance(layer, FullAttentionCache):
            layer.append(*_kv(layer.block_size, seq=2))
    stats = small.kv_stats()
    assert (stats.full_attention_layers, stats.block_size, stats.valid_tokens_total, stats.capacity_tokens_total) == (2, 2, 4, 8)
    assert (stats.append_calls_total, stats.contiguous_view_calls_total, stats.max_valid_tokens) == (2, 2, 2)
    small.release()
    for layer in small.layers:
        if isinstance(layer, FullAttentionCache):
            assert layer.length == 0 and layer.block_table == [] and layer.pool.free_blocks == [0, 1]
        else:
            assert layer.state is None and layer.conv_tail is None


def test_batch_kv_tensors_pads_and_masks() -> None:  # :306-340
    a, b = FullAttentionCache(block_size=4), FullAttentionCache(block_size=4)
    for step in range(3):
        a.append(*_kv(step))
    for step in range(5):
        b.append(*_kv(step + 10))
    keys, values, mask = batch_kv_tensors([a, b])
    assert keys.shape == (2, 2, 5, 4)
    assert mask.tolist() == [[True, True, True, False, False], [True] * 5]
    torch.testing.assert_close(keys[0:1, :, :3], a.as_tensors()[0])
    assert (keys[0, :, 3:] == 0).all() and (values[0, :, 3:] == 0).all()
    torch.testing.assert_close(values[1:2], b.as_tensors()[1])


def test_page_metadata_and_tables() -> None:  # :359-385
    cache = FullAttentionCache(capacity_hint=4, block_size=2)
    cache.append(*_kv(0, seq=3))
    meta = cache.page_metadata()
    assert meta.block_table.tolist() == [0, 1]
    assert (meta.sequence_length, meta.block_size, meta.logical_blocks, meta.capacity_tokens) == (3, 2, 2, 4)
    stats = cache.stats()
    assert (stats.page_table_tensor_calls, stats.page_metadata_calls, stats.page_table_entries_total) == (1, 1, 2)
    other = FullAttentionCache(capacity_hint=6, block_size=2)
    other.append(*_kv(0, seq=6))
    other.block_table = [2, 0, 1]
    assert other.page_table_tensor().tolist() == [2, 0, 1]


def test_batch_page_tables_pads_and_counts() -> None:  # :388-412
    a, b = FullAttentionCache(block_size=2), FullAttentionCache(block_size=2)
    a.append(*_kv(0, seq=3))
    b.append(*_kv(1, seq=5))
    meta = batch_page_tables([a, b])
    assert (meta.block_size, meta.max_blocks, meta.max_sequence_length) == (2, 3, 5)
    assert meta.block_tables.tolist() == [[0, 1, -1], [0, 1, 2]]
    assert meta.sequence_lengths.tolist() == [3, 5]
    assert meta.valid_mask.tolist() == [[True, True, True, False, False], [True] * 5]
    assert meta.key_blocks == (a.key_blocks, b.key_blocks)
    assert (a.stats().batched_page_table_calls, b.stats().batched_page_table_calls) == (1, 1)
    assert (a.stats().page_table_entries_total, b.stats().page_table_entries_total) == (2, 3)


def test_batch_page_tables_rejects_mixed_block_sizes() -> None:  # :415-422
    a, b = FullAttentionCache(block_size=2), FullAttentionCache(block_size=4)
    a.append(*_kv(0))
    b.append(*_kv(1))
    with pytest.raises(ValueError, match="matching block sizes"):
        batch_page_tables([a, b])


def test_kv_stats_aggregate_page_counters() -> None:  # :425-439
    state = DecodeState.empty(_mapping(("full_attention", "full_attention")), None, max_seq_len=4, kv_block_size=2)
    for index, cache in enumerate(state.layers):
        cache.append(*_kv(index, seq=2))
        cache.page_metadata()
    batch_page_tables(state.layers)
    stats = state.kv_stats()
    assert (stats.page_table_tensor_calls_total, stats.page_metadata_calls_total) == (4, 2)
    assert (stats.batched_page_table_calls_total, stats.page_table_entries_total) == (2, 8)


def test_shared_pool_caches_share_storage_and_gather_in_order() -> None:
    pool = SharedKVBlockPool(8, kv_heads=2, head_dim=4, block_size=2, dtype=torch.float32)
    a = FullAttentionCache(block_size=2, shared_pool=pool)
    b = FullAttentionCache(block_size=2, shared_pool=pool)
    ka, va = _kv(1, seq=3)
    kb, vb = _kv(2, seq=5)
    a.append_blocks(ka, va)
    b.append_blocks(kb, vb)
    assert a.key_blocks is b.key_blocks is pool.key_blocks
    assert a.block_table == [0, 1] and b.block_table == [2, 3, 4]
    torch.testing.assert_close(a.as_tensors()[0], ka)
    torch.testing.assert_close(b.as_tensors()[1], vb)
    meta = batch_page_tables([a, b])
    assert meta.key_blocks[0] is meta.key_blocks[1]
    a.release()
    assert pool.free_blocks == [0, 1, 5, 6, 7]
    with pytest.raises(RuntimeError, match="exhausted"):
        FullAttentionCache(block_size=2, shared_pool=pool).append_blocks(*_kv(3, seq=20))


def test_shared_pool_release_after_device_hand_off_goes_to_the_device_list() -> None:
    """After ``device_allocator()`` the host list is empty, host ``allocate`` refuses, and a cache's
    ``release`` merges its blocks into the allocator's sorted free list (they stay reservable)."""
    pool = SharedKVBlockPool(8, kv_heads=2, head_dim=4, block_size=2, dtype=torch.float32)
    a = FullAttentionCache(block_size=2, shared_pool=pool)
    b = FullAttentionCache(block_size=2, shared_pool=pool)
    a.append_blocks(*_kv(1, seq=3))
    b.append_blocks(*_kv(2, seq=2))
    assert a.block_table == [0, 1] and b.block_table == [2]
    alloc = pool.device_allocator()
    assert pool.device_allocator() is alloc
    assert pool.free_blocks == [] and alloc.free_blocks() == [3, 4, 5, 6, 7] and alloc.free_count == 5
    with pytest.raises(RuntimeError, match="DeviceBlockAllocator"):
        FullAttentionCache(block_size=2, shared_pool=pool).append_blocks(*_kv(3, seq=1))
    a.release()
    assert alloc.free_blocks() == [0, 1, 3, 4, 5, 6, 7] and pool.free_blocks == []
    b.release()
    assert alloc.free_blocks() == list(range(8))
    with pytest.raises(ValueError, match="already free"):
        pool.release([4])


def test_page_table_tensor_is_reused_until_the_table_changes() -> None:
    cache = FullAttentionCache(block_size=2)
    cache.append_blocks(torch.zeros(1, 1, 3, 4), torch.zeros(1, 1, 3, 4))
    first = cache.page_table_tensor()
    assert cache.page_table_tensor() is first
    assert first.tolist() == cache.block_table
    cache.append_blocks(torch.zeros(1, 1, 2, 4), torch.zeros(1, 1, 2, 4))
    second = cache.page_table_tensor()
    assert second is not first and second.tolist() == cache.block_table and len(cache.block_table) >= 3
    assert cache.page_table_tensor_calls == 3
