"""Dispatch ladder and counters against the reference's own tests (CPU).

Restates ``tests/unit/test_tp_runtime.py:627-751`` of the reference on this
package's ``attention_runtime``; the config dict is the reference's
``_config()`` (``tests/unit/test_tp_runtime.py:1123-1149``).
"""

from __future__ import annotations

from dataclasses import replace
from types import SimpleNamespace

import pytest
import torch

import attention_runtime as ar
from decode_state import FullAttentionCache, batch_page_tables


def _config(**full_overrides) -> ar.AttentionConfig:
    text = {
        "linear_num_key_heads": 1,
        "linear_num_value_heads": 1,
        "linear_key_head_dim": 1,
        "linear_value_head_dim": 1,
        "linear_conv_kernel_dim": 4,
        "num_attention_heads": 2,
        "num_key_value_heads": 1,
        "head_dim": 1,
        "attn_output_gate": True,
    }
    cfg = ar.parse_attention_config({"text_config": text})
    return replace(cfg, full_attention=replace(cfg.full_attention, **full_overrides)) if full_overrides else cfg


def _enabled() -> ar.AttentionConfig:
    return _config(paged_kv_metadata=True, native_paged_attention=True)


def _fake_cuda(shape):
    return SimpleNamespace(shape=shape, is_cuda=True)


def _stats_after(config, query, key, value, *, seq_len, batched):
    runtime = ar.HotPathRuntime()
    ar.record_paged_attention_dispatch(runtime, config, query, key, value, seq_len=seq_len, batched=batched)
    return runtime.paged_attention_stats


def test_disabled_by_default() -> None:  # :627-645
    stats = _stats_after(_config(), torch.zeros(1, 1, 1, 1), torch.zeros(1, 1, 1, 1), torch.zeros(1, 1, 1, 1), seq_len=1, batched=False)
    assert (stats.calls, stats.dense_fallbacks, stats.fallback_disabled, stats.eligible, stats.native_hits) == (1, 1, 1, 0, 0)


def test_cpu_fallback_when_enabled() -> None:  # :648-666
    stats = _stats_after(_enabled(), torch.zeros(1, 1, 1, 1), torch.zeros(1, 1, 1, 1), torch.zeros(1, 1, 1, 1), seq_len=1, batched=False)
    assert (stats.calls, stats.dense_fallbacks, stats.fallback_cpu, stats.eligible) == (1, 1, 1, 0)


def test_prefill_or_multitoken_fallback() -> None:  # :669-687
    f = _fake_cuda((1, 1, 2, 1))
    stats = _stats_after(_enabled(), f, f, f, seq_len=2, batched=False)
    assert (stats.dense_fallbacks, stats.fallback_prefill_or_multitoken, stats.eligible) == (1, 1, 0)


def test_per_request_pool_fallback_for_batches() -> None:  # :690-708
    f = _fake_cuda((2, 1, 1, 1))
    stats = _stats_after(_enabled(), f, f, f, seq_len=1, batched=True)
    assert (stats.dense_fallbacks, stats.fallback_per_request_pools, stats.eligible) == (1, 1, 0)


def test_native_hit() -> None:  # :711-720
    runtime = ar.HotPathRuntime()
    ar.record_native_paged_dispatch(runtime, "no_kernel", native=True)
    s = runtime.paged_attention_stats
    assert (s.calls, s.eligible, s.native_hits, s.dense_fallbacks, s.fallback_no_kernel) == (1, 1, 1, 0, 0)


def test_native_exception_counts_as_no_kernel_fallback() -> None:
    runtime = ar.HotPathRuntime()
    ar.record_native_paged_dispatch(runtime, "no_kernel", native=False)
    s = runtime.paged_attention_stats
    assert (s.eligible, s.dense_fallbacks, s.fallback_no_kernel) == (1, 1, 1)


def test_batched_reason_disabled_without_page_tables() -> None:  # :723-733
    cache = FullAttentionCache(block_size=2)
    cache.append_blocks(torch.zeros(1, 2, 1, 4), torch.zeros(1, 2, 1, 4))
    assert ar.batched_paged_attention_fallback_reason(_enabled(), torch.zeros(1, 2, 1, 4), [cache], None, seq_len=1) == "disabled"


def test_batched_reason_cpu_for_cpu_caches() -> None:  # :736-746
    cache = FullAttentionCache(block_size=2)
    cache.append_blocks(torch.zeros(1, 2, 1, 4), torch.zeros(1, 2, 1, 4))
    tables = batch_page_tables([cache])
    assert ar.batched_paged_attention_fallback_reason(_enabled(), torch.zeros(1, 2, 1, 4), [cache], tables, seq_len=1) == "cpu"


@pytest.mark.parametrize(
    "dtype,expected",
    [("torch.float32", "no_kernel"), ("torch.bfloat16", "no_kernel"), ("torch.float16", "shape")],
)
def test_dtype_eligibility(dtype, expected) -> None:
    q = SimpleNamespace(shape=(1, 16, 1, 256), is_cuda=True, dtype=dtype)
    kv = SimpleNamespace(shape=(1, 2, 8, 16, 256), is_cuda=True, dtype=dtype)
    assert ar.paged_attention_fallback_reason(_enabled(), q, kv, kv, seq_len=1, batched=False) == expected


def test_shape_mismatch_reports_shape() -> None:
    q = _fake_cuda((1, 16, 1, 128))
    kv = _fake_cuda((1, 2, 8, 16, 256))
    assert ar.paged_attention_fallback_reason(_enabled(), q, kv, kv, seq_len=1, batched=False) == "shape"


def test_full_attention_paged_returns_none_on_cpu_and_counts() -> None:
    runtime = ar.HotPathRuntime()
    cache = FullAttentionCache(block_size=2)
    cache.append_blocks(torch.zeros(1, 2, 3, 4), torch.zeros(1, 2, 3, 4))
    assert ar.full_attention_paged(torch.zeros(1, 2, 1, 4), None, cache, _enabled(), runtime) is None
    assert runtime.paged_attention_stats.fallback_cpu == 1


def test_missing_native_library_is_raised_not_a_dense_fallback(monkeypatch) -> None:
    """A kernel-side rejection falls back to the caller's dense path; a missing library never does."""
    import hip_loader
    import hip_ops

    def missing(*args, **kwargs):
        raise hip_loader.NativeLibraryMissing("not built")

    def rejected(*args, **kwargs):
        raise RuntimeError("paged decode: shape rejected")

    monkeypatch.setattr(ar, "paged_attention_fallback_reason", lambda *a, **k: "no_kernel")
    cache = FullAttentionCache(block_size=2)
    cache.append_blocks(torch.zeros(1, 2, 3, 4), torch.zeros(1, 2, 3, 4))
    runtime = ar.HotPathRuntime()
    monkeypatch.setattr(hip_ops, "paged_attention_decode", missing)
    with pytest.raises(hip_loader.NativeLibraryMissing):
        ar.full_attention_paged(torch.zeros(1, 2, 1, 4), None, cache, _enabled(), runtime)
    monkeypatch.setattr(hip_ops, "paged_attention_decode", rejected)
    assert ar.full_attention_paged(torch.zeros(1, 2, 1, 4), None, cache, _enabled(), runtime) is None
    assert runtime.paged_attention_stats.fallback_no_kernel == 1


def test_linear_native_ladder_counts_like_the_reference_on_cpu_tensors() -> None:
    # src/reference_ops.py:444-494: CPU tensors and non-fp8 weights fall back with the same counters
    import torch

    from attention_runtime import LinearDispatchStats, linear_native

    stats = LinearDispatchStats()
    w8 = torch.zeros((256, 128)).to(torch.float8_e4m3fn)
    scale = torch.ones((2, 1), dtype=torch.bfloat16)
    x = torch.zeros((3, 128))
    assert linear_native(x, w8, scale, stats=stats) is None
    assert linear_native(x, torch.zeros((256, 128)), None, stats=stats) is None
    assert linear_native(x, w8, None, use_cuda_kernel=False, stats=stats) is None
    assert linear_native(torch.zeros((3, 100)), torch.zeros((200, 100)).to(torch.float8_e4m3fn), scale.float(), stats=stats) is None
    d = stats.to_dict()
    assert d["calls"] == 4 and d["fallback_calls"] == 4 and d["cuda_kernel_hits"] == 0 and d["fp8_weight_calls"] == 3
    assert d["fallback_hidden_not_cuda"] == 3 and d["fallback_weight_not_cuda"] == 3 and d["fallback_scale_not_cuda"] == 2
    assert d["fallback_weight_dtype"] == 1 and d["fallback_missing_scale"] == 1 and d["fallback_disabled_cuda_kernel"] == 1
    assert d["fallback_scale_dtype"] == 1 and d["fallback_hidden_alignment"] == 1 and d["fallback_weight_alignment"] == 1


def test_device_page_tables_row_bookkeeping_and_cpu_dispatch_reason() -> None:
    """Rows of a DeviceBatchPageTables are taken lowest first and reused after release; on CPU
    tensors the device decode entry reports reason "cpu" and returns None (the caller's dense path)."""
    import torch

    from decode_state import DeviceBatchPageTables, SharedKVBlockPool

    pool = SharedKVBlockPool(8, kv_heads=2, head_dim=4, block_size=2, dtype=torch.float32)
    tables = DeviceBatchPageTables(pool, rows=3, max_blocks=4)
    assert pool.free_blocks == [] and tables.allocator.free_blocks() == list(range(8))
    assert [tables.add_request(), tables.add_request()] == [0, 1]
    assert tables.step_counts.tolist() == [1, 1, 0] and tables.active == [True, True, False]
    assert tables.release_request(0) == []
    assert tables.step_counts.tolist() == [0, 1, 0] and tables.add_request() == 0
    with pytest.raises(ValueError, match="holds no request"):
        tables.release_request(2)
    config = ar.parse_attention_config({"text_config": {
        "linear_num_key_heads": 1, "linear_num_value_heads": 1, "linear_key_head_dim": 4, "linear_value_head_dim": 4,
        "linear_conv_kernel_dim": 4, "num_attention_heads": 2, "num_key_value_heads": 2, "head_dim": 4, "attn_output_gate": False,
        "native_paged_attention": True}})
    runtime = ar.HotPathRuntime()
    q = torch.zeros(3, 2, 1, 4)
    kv = torch.zeros(3, 2, 1, 4)
    assert ar.full_attention_decode_device(q, None, kv, kv, pool.key_blocks, pool.value_blocks, tables, config, runtime) is None
    assert runtime.paged_attention_stats.fallback_cpu == 1 and runtime.paged_attention_stats.native_hits == 0


def _tables_on_cpu(rows=3):
    from decode_state import DeviceBatchPageTables, SharedKVBlockPool

    pool = SharedKVBlockPool(8, kv_heads=2, head_dim=4, block_size=2)
    return pool, DeviceBatchPageTables(pool, rows=rows, max_blocks=4)


def _small_enabled(**overrides) -> ar.AttentionConfig:
    text = {"linear_num_key_heads": 1, "linear_num_value_heads": 1, "linear_key_head_dim": 4, "linear_value_head_dim": 4,
            "linear_conv_kernel_dim": 4, "num_attention_heads": 2, "num_key_value_heads": 2, "head_dim": 4, "attn_output_gate": True,
            "native_paged_attention": True}
    cfg = ar.parse_attention_config({"text_config": text})
    return replace(cfg, full_attention=replace(cfg.full_attention, **overrides)) if overrides else cfg


def test_native_prefill_counter_is_reported_and_starts_at_zero() -> None:
    stats = ar.HotPathRuntime().paged_attention_stats
    assert stats.to_dict()["native_prefill_hits"] == 0
    assert stats.snapshot().native_prefill_hits == 0


@pytest.mark.parametrize("overrides,counter", [({"native_paged_attention": False}, "fallback_disabled"), ({}, "fallback_cpu")])
def test_prefill_and_decode_step_entries_follow_the_ladder_on_cpu(overrides, counter) -> None:
    """The projection-output entries return None before writing anything when the reference's
    ladder says no (disabled, CPU tensors), and count the fallback as the reference does."""
    from decode_state import PrefillStep

    pool, tables = _tables_on_cpu()
    config = _small_enabled(**overrides)
    runtime = ar.HotPathRuntime()
    q_proj = torch.zeros(3, 2 * 2 * 4, dtype=torch.bfloat16)
    kv = torch.zeros(3, 2 * 4, dtype=torch.bfloat16)
    w = torch.zeros(4, dtype=torch.bfloat16)
    step = PrefillStep(rows=(0,), counts=(3,), index=torch.tensor([0]), cu_seqlens=torch.tensor([0, 3], dtype=torch.int32),
                       starts=torch.zeros(1, dtype=torch.int32), block_tables=torch.full((1, 4), -1, dtype=torch.int32), max_new=3,
                       total_tokens=3, block_size=2)
    assert ar.full_attention_prefill_device(q_proj, kv, kv, w, w, pool.key_blocks, pool.value_blocks, step, config, runtime) is None
    assert ar.full_attention_decode_step_device(q_proj, kv, kv, w, w, pool.key_blocks, pool.value_blocks, tables, config, runtime) is None
    stats = runtime.paged_attention_stats.to_dict()
    assert stats[counter] == 2 and stats["dense_fallbacks"] == 2 and stats["native_prefill_hits"] == 0 and stats["native_hits"] == 0
    assert torch.count_nonzero(pool.key_blocks) == 0


@pytest.mark.parametrize("overrides,counter", [({"native_paged_attention": False}, "fallback_disabled"), ({}, "fallback_cpu")])
def test_projection_entries_take_the_ladder_on_misshaped_projections(overrides, counter) -> None:
    """A q_proj whose width is not H*2D goes down the same ladder (no view error): the reasons
    before the shape check still decide, and nothing is written."""
    from decode_state import PrefillStep

    pool, tables = _tables_on_cpu()
    config = _small_enabled(**overrides)
    runtime = ar.HotPathRuntime()
    q_proj = torch.zeros(3, 2 * 2 * 4 + 1, dtype=torch.bfloat16)
    kv = torch.zeros(3, 2 * 4, dtype=torch.bfloat16)
    w = torch.zeros(4, dtype=torch.bfloat16)
    step = PrefillStep(rows=(0,), counts=(3,), index=torch.tensor([0]), cu_seqlens=torch.tensor([0, 3], dtype=torch.int32),
                       starts=torch.zeros(1, dtype=torch.int32), block_tables=torch.full((1, 4), -1, dtype=torch.int32), max_new=3,
                       total_tokens=3, block_size=2)
    assert ar.full_attention_prefill_device(q_proj, kv, kv, w, w, pool.key_blocks, pool.value_blocks, step, config, runtime) is None
    assert ar.full_attention_decode_step_device(q_proj, kv, kv, w, w, pool.key_blocks, pool.value_blocks, tables, config, runtime) is None
    assert runtime.paged_attention_stats.to_dict()[counter] == 2
    assert torch.count_nonzero(pool.key_blocks) == 0


def test_query_probe_is_the_query_half_or_the_projection_itself() -> None:
    q_proj = torch.arange(2 * 3 * 2 * 4, dtype=torch.float32).reshape(2, 3 * 2 * 4)
    probe = ar._query_probe(q_proj, 3, 4)
    assert tuple(probe.shape) == (2, 3, 1, 4)
    # head h's query is the first D of its 2D-wide slice of the row
    assert torch.equal(probe[1, 2, 0], q_proj[1, 2 * 8 : 2 * 8 + 4])
    assert ar._query_probe(q_proj[:, :-1], 3, 4) is not None and tuple(ar._query_probe(q_proj[:, :-1], 3, 4).shape) == (2, 23)


def test_reserve_prefill_rejects_bad_steps_before_touching_the_device() -> None:
    _pool, tables = _tables_on_cpu()
    tables.add_request()
    with pytest.raises(ValueError, match="one count per row"):
        tables.reserve_prefill([0], [1, 2])
    with pytest.raises(ValueError, match="distinct"):
        tables.reserve_prefill([0, 0], [1, 2])
    with pytest.raises(ValueError, match="positive"):
        tables.reserve_prefill([0], [0])
    with pytest.raises(ValueError, match="holds no request"):
        tables.reserve_prefill([1], [4])


def test_linear_prefill_needs_z_and_norm_weight_together() -> None:
    with pytest.raises(ValueError, match="go together"):
        ar.linear_attention_prefill(None, None, None, None, None, None, _small_enabled(), z=torch.zeros(1))
