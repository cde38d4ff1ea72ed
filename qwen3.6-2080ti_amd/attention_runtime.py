"""Attention entry points of the hybrid runtime at TP = 1, on the gfx950 kernels.

Mirrors the attention side of the reference's ``src/tp_runtime.py`` so the
engine and scheduler above it keep their calls:

* ``PagedAttentionDispatchStats`` (``:90-107``) and the dispatch reason ladder
  ``paged_attention_fallback_reason`` (``:770-805``),
  ``batched_paged_attention_fallback_reason`` (``:646-669``),
  ``record_native_paged_dispatch`` (``:747-767``) and
  ``record_paged_attention_dispatch`` (``:733-744``) -- same reason strings and
  counters.  One difference: bfloat16 tensors are eligible (the gfx950 decode
  kernel computes bf16 natively; the reference kernel was fp32-only, so it
  reported them as ``"shape"``).
* ``full_attention_paged`` / ``full_attention_paged_batch``: the native branch
  of ``_tp_full_attention_paged_or_dense`` (``:551-610``) and its batched twin
  (``:2498-2555``) including the sigmoid output gate (``:673-695``) but not the
  output projection.  When the ladder says the native kernel does not apply,
  they return ``None`` and the caller runs its own dense path, as the
  reference does; a native ``RuntimeError`` is recorded as a fallback and also
  returns ``None``.
* ``recurrent_gated_delta_rule`` (``:2744-2787``) on the HIP recurrent core,
  ``linear_attention_decode_batch`` (the state plumbing of ``:2613-2717``) on a
  slot-indexed state pool, and ``linear_attention_prefill`` on the chunked
  kernel.

Host-side tensor preparation (L2 norm, transposes) is PyTorch on the same
device; every hot loop is a HIP kernel.  There is no CPU or dense fallback in
this module.
"""

from __future__ import annotations

import contextlib
from dataclasses import dataclass, field
from typing import Any, Iterator, Sequence

from decode_state import DeviceBatchPageTables, FullAttentionCache, LinearStatePool, PrefillStep, batch_page_tables

# --------------------------------------------------------------------------- config


@dataclass(frozen=True)
class FullAttentionConfig:
    """Full-attention fields of ``src/runtime_config.py:33-52`` that the hot path reads."""

    num_heads: int
    num_key_value_heads: int
    head_dim: int
    output_gate: bool = True
    paged_kv_metadata: bool = True
    native_paged_attention: bool = False

    @property
    def attn_dim(self) -> int:
        return self.num_heads * self.head_dim


@dataclass(frozen=True)
class LinearAttentionConfig:
    """``LinearAttentionConfig`` of ``src/runtime_config.py:15-30``."""

    key_heads: int
    value_heads: int
    key_head_dim: int
    value_head_dim: int
    conv_kernel_dim: int

    @property
    def qkv_dim(self) -> int:
        return self.key_heads * self.key_head_dim * 2 + self.value_heads * self.value_head_dim

    @property
    def value_state_dim(self) -> int:
        return self.value_heads * self.value_head_dim


@dataclass(frozen=True)
class AttentionConfig:
    full_attention: FullAttentionConfig
    linear_attention: LinearAttentionConfig


def parse_attention_config(config: dict[str, Any]) -> AttentionConfig:
    """Read the hot-path fields of an HF ``config.json`` (``src/runtime_config.py:92-131``)."""
    text = config.get("text_config", config)

    def need(key: str) -> Any:
        if key not in text:
            raise ValueError(f"missing text_config.{key}")
        return text[key]

    return AttentionConfig(
        full_attention=FullAttentionConfig(
            num_heads=int(need("num_attention_heads")),
            num_key_value_heads=int(need("num_key_value_heads")),
            head_dim=int(need("head_dim")),
            output_gate=bool(need("attn_output_gate")),
            paged_kv_metadata=bool(text.get("paged_kv_metadata", True)),
            native_paged_attention=bool(text.get("native_paged_attention", False)),
        ),
        linear_attention=LinearAttentionConfig(
            key_heads=int(need("linear_num_key_heads")),
            value_heads=int(need("linear_num_value_heads")),
            key_head_dim=int(need("linear_key_head_dim")),
            value_head_dim=int(need("linear_value_head_dim")),
            conv_kernel_dim=int(need("linear_conv_kernel_dim")),
        ),
    )


# --------------------------------------------------------------------------- dispatch accounting


@dataclass
class PagedAttentionDispatchStats:
    calls: int = 0
    eligible: int = 0
    dense_fallbacks: int = 0
    native_hits: int = 0
    fallback_disabled: int = 0
    fallback_no_kernel: int = 0
    fallback_prefill_or_multitoken: int = 0
    fallback_cpu: int = 0
    fallback_per_request_pools: int = 0
    fallback_shape: int = 0
    # multi-token steps served by the native chunked prefill (``full_attention_prefill_device``).
    # The reference has no native prefill, so its ladder counts every such call in
    # ``fallback_prefill_or_multitoken``; here they count as calls and native prefill hits only,
    # which leaves the reference's fields meaning what they mean there.
    native_prefill_hits: int = 0

    def snapshot(self) -> "PagedAttentionDispatchStats":
        return PagedAttentionDispatchStats(**vars(self))

    def to_dict(self) -> dict[str, int]:
        return dict(vars(self))


@dataclass
class HotPathRuntime:
    """The slice of ``TpRuntime`` the attention entry points use at TP = 1: counters and profile scopes."""

    paged_attention_stats: PagedAttentionDispatchStats = field(default_factory=PagedAttentionDispatchStats)
    scope_calls: dict[str, int] = field(default_factory=dict)

    @contextlib.contextmanager
    def profile_scope(self, name: str) -> Iterator[None]:
        self.scope_calls[name] = self.scope_calls.get(name, 0) + 1
        yield


_FLOAT_DTYPES = ("torch.float32", "torch.bfloat16")


def paged_attention_fallback_reason(config: AttentionConfig, query: Any, key: Any, value: Any, *, seq_len: int, batched: bool) -> str:
    """Reason ladder of ``src/tp_runtime.py:770-805`` (``"no_kernel"`` = eligible)."""
    full = config.full_attention
    if not full.paged_kv_metadata or not full.native_paged_attention:
        return "disabled"
    if not all(getattr(t, "is_cuda", False) for t in (query, key, value)):
        return "cpu"
    if seq_len != 1:
        return "prefill_or_multitoken"
    if batched:
        return "per_request_pools"
    q_shape = tuple(getattr(query, "shape", ()))
    k_shape = tuple(getattr(key, "shape", ()))
    v_shape = tuple(getattr(value, "shape", ()))
    if len(q_shape) != 4 or len(k_shape) not in (4, 5) or len(v_shape) != len(k_shape):
        return "shape"
    if len(k_shape) == 5:
        # reference per-request layout (batch, heads, P, bs, D): batch and heads follow the query
        if q_shape[0] != k_shape[0] or q_shape[0] != v_shape[0]:
            return "shape"
        if q_shape[1] % k_shape[1] or k_shape[1] != v_shape[1]:
            return "shape"
    elif k_shape[1] != v_shape[1] or q_shape[1] % k_shape[1]:
        return "shape"
    if q_shape[3] != k_shape[-1] or q_shape[3] != v_shape[-1]:
        return "shape"
    q_dtype = getattr(query, "dtype", None)
    if q_dtype is not None:
        k_dtype = getattr(key, "dtype", q_dtype)
        v_dtype = getattr(value, "dtype", q_dtype)
        if str(q_dtype) not in _FLOAT_DTYPES or str(k_dtype) not in _FLOAT_DTYPES or str(k_dtype) != str(v_dtype):
            return "shape"
    return "no_kernel"


def batched_paged_attention_fallback_reason(config: AttentionConfig, query: Any, caches: Sequence[FullAttentionCache], page_tables: Any, *, seq_len: int) -> str:
    """``src/tp_runtime.py:646-669``: every row must be eligible on its own."""
    if page_tables is None:
        return "disabled"
    if not caches:
        return "shape"
    for row, cache in enumerate(caches):
        reason = paged_attention_fallback_reason(config, query[row : row + 1], cache.key_blocks, cache.value_blocks, seq_len=seq_len, batched=False)
        if reason != "no_kernel":
            return reason
    return "no_kernel"


def record_native_paged_dispatch(runtime: HotPathRuntime, reason: str, *, native: bool) -> None:
    """``src/tp_runtime.py:747-767``."""
    stats = runtime.paged_attention_stats
    stats.calls += 1
    if reason == "no_kernel":
        stats.eligible += 1
    if native:
        stats.native_hits += 1
        return
    stats.dense_fallbacks += 1
    counter = {
        "disabled": "fallback_disabled",
        "cpu": "fallback_cpu",
        "prefill_or_multitoken": "fallback_prefill_or_multitoken",
        "per_request_pools": "fallback_per_request_pools",
        "shape": "fallback_shape",
    }.get(reason, "fallback_no_kernel")
    setattr(stats, counter, getattr(stats, counter) + 1)


def record_paged_attention_dispatch(runtime: HotPathRuntime, config: AttentionConfig, query: Any, key: Any, value: Any, *, seq_len: int, batched: bool) -> None:
    """``src/tp_runtime.py:733-744``."""
    reason = paged_attention_fallback_reason(config, query, key, value, seq_len=seq_len, batched=batched)
    record_native_paged_dispatch(runtime, reason, native=False)


# --------------------------------------------------------------------------- full attention


def _gate_heads(heads: Any, gate: Any) -> Any:
    """``out * sigmoid(gate)`` on ``(B, H, 1, D)`` heads with ``gate`` ``(B, 1, H*D)`` (``src/tp_runtime.py:689-691``)."""
    import torch

    batch, num_heads, seq, dim = heads.shape
    out = heads.transpose(1, 2).reshape(batch, seq, num_heads * dim)
    return out * torch.sigmoid(gate.to(out.dtype))


def full_attention_paged(query: Any, gate: Any | None, cache: FullAttentionCache, config: AttentionConfig, runtime: HotPathRuntime) -> Any | None:
    """Native branch of ``_tp_full_attention_paged_or_dense`` (``src/tp_runtime.py:551-610``).

    ``query`` ``(B, H, 1, D)`` after RoPE, with the step's K/V already appended
    to ``cache``.  Returns the gated attention output ``(B, 1, H*D)`` (before
    ``o_proj``), or ``None`` when the caller must take its dense path.
    """
    page_table = cache.page_metadata() if config.full_attention.paged_kv_metadata else None
    reason = paged_attention_fallback_reason(
        config, query, None if page_table is None else page_table.key_blocks, None if page_table is None else page_table.value_blocks,
        seq_len=int(query.shape[2]), batched=False,
    )
    if reason != "no_kernel" or page_table is None:
        record_native_paged_dispatch(runtime, reason, native=False)
        return None
    import hip_loader
    import hip_ops

    try:
        with runtime.profile_scope("full_attention.native_paged"):
            heads = hip_ops.paged_attention_decode(
                query, page_table.block_table, page_table.key_blocks, page_table.value_blocks, page_table.sequence_length, page_table.block_size
            )
    except hip_loader.NativeLibraryMissing:
        raise
    except RuntimeError:
        # a kernel-side rejection (shape, dtype, workspace): the caller's dense path runs,
        # as src/tp_runtime.py:591 and :2537 do
        record_native_paged_dispatch(runtime, "no_kernel", native=False)
        return None
    record_native_paged_dispatch(runtime, reason, native=True)
    return heads if gate is None else _gate_heads(heads, gate)


def full_attention_paged_batch(query: Any, gate: Any | None, caches: Sequence[FullAttentionCache], config: AttentionConfig, runtime: HotPathRuntime) -> Any | None:
    """Native branch of ``_tp_full_attention_batch_paged_or_dense`` (``src/tp_runtime.py:2498-2555``).

    Caches may each own a reference-layout pool or share one
    ``SharedKVBlockPool``; either way one kernel launch serves the batch.
    """
    page_tables = batch_page_tables(caches) if config.full_attention.paged_kv_metadata else None
    reason = batched_paged_attention_fallback_reason(config, query, caches, page_tables, seq_len=int(query.shape[2]))
    if reason != "no_kernel" or page_tables is None:
        record_native_paged_dispatch(runtime, reason, native=False)
        return None
    import hip_loader
    import hip_ops

    try:
        with runtime.profile_scope("batch.full_attention.native_paged"):
            heads = hip_ops.paged_attention_decode_batched(
                query, page_tables.block_tables, list(page_tables.key_blocks), list(page_tables.value_blocks), page_tables.sequence_lengths,
                page_tables.block_size,
            )
    except hip_loader.NativeLibraryMissing:
        raise
    except RuntimeError:
        # a kernel-side rejection (shape, dtype, workspace): the caller's dense path runs,
        # as src/tp_runtime.py:591 and :2537 do
        record_native_paged_dispatch(runtime, "no_kernel", native=False)
        return None
    record_native_paged_dispatch(runtime, reason, native=True)
    return heads if gate is None else _gate_heads(heads, gate)


def full_attention_decode_device(
    query: Any, gate: Any | None, key: Any, value: Any, key_blocks: Any, value_blocks: Any, tables: DeviceBatchPageTables,
    config: AttentionConfig, runtime: HotPathRuntime, *, no_alloc: bool = False,
) -> Any | None:
    """One decode token of a full-attention layer for every row of a running batch, on
    device-resident page tables: the batched native branch of
    ``_tp_full_attention_batch_paged_or_dense`` (``src/tp_runtime.py:2498-2555``) without its
    per-step host work (the table rebuild and copy of ``batch_page_tables``,
    ``src/decode_state.py:545-603``).

    ``tables.reserve_step()`` must have run for this step (once for all layers sharing the
    tables).  ``key``/``value`` ``(rows, H_kv, 1, D)`` are the step's post-rotary K/V; they go
    to the reserved slots of this layer's shared pool ``key_blocks``/``value_blocks``
    ``(P, H_kv, bs, D)``, then ``query`` ``(rows, H, 1, D)`` attends over each row's cache.
    Rows without a request give zeros.  Same dispatch ladder and counters as the cache form;
    ``None`` means the caller runs its dense path.  With ``no_alloc`` the attention runs on the
    library's static scratch (``qa_paged_attention_decode_batched_noalloc``) instead of a
    workspace.  Nothing here reads back to the host or copies host to device.
    """
    reason = _device_pool_reason(config, query, key_blocks, value_blocks, tables)
    if reason != "no_kernel":
        record_native_paged_dispatch(runtime, reason, native=False)
        return None
    import hip_ops

    # Once the append has written this step's K/V into the pool the cache has advanced, so a
    # later kernel error propagates: a dense fallback would attend over a cache that already
    # holds the step (and under graph capture would record a step without attention).
    with runtime.profile_scope("batch.full_attention.native_paged_device"):
        tables.append(key, value, key_blocks, value_blocks)
        decode = hip_ops.paged_attention_decode_batched_noalloc if no_alloc else hip_ops.paged_attention_decode_batched
        heads = decode(query, tables.block_tables, key_blocks, value_blocks, tables.sequence_lengths, tables.block_size)
    record_native_paged_dispatch(runtime, reason, native=True)
    return heads if gate is None else _gate_heads(heads, gate)


def _device_pool_reason(config: AttentionConfig, query: Any, key_blocks: Any, value_blocks: Any, tables: DeviceBatchPageTables) -> str:
    """The dispatch ladder for a step on device page tables, checked before anything is written:
    the reference's reasons (one token per row), then what the native kernels need of the pool
    (a shared ``(P, H_kv, bs, D)`` bf16 pool with the tables' block size and block count)."""
    seq_len = int(query.shape[2]) if len(tuple(getattr(query, "shape", ()))) == 4 else 1
    reason = paged_attention_fallback_reason(config, query, key_blocks, value_blocks, seq_len=seq_len, batched=False)
    if reason != "no_kernel":
        return reason
    if key_blocks.dim() != 4 or tuple(value_blocks.shape) != tuple(key_blocks.shape):
        return "shape"
    if int(key_blocks.shape[2]) != tables.block_size or int(key_blocks.shape[0]) != tables.num_blocks:
        return "shape"
    return "no_kernel"


def _qk_norm_rope(q_proj: Any, k_proj: Any, v_proj: Any, q_norm_weight: Any, k_norm_weight: Any, key_blocks: Any, value_blocks: Any,
                  block_tables: Any, cu_seqlens: Any, starts: Any, block_size: int, max_new: int, rope: "RopeConfig") -> tuple[Any, Any]:
    import hip_ops

    return hip_ops.qk_norm_rope_kv_append(
        q_proj, k_proj, v_proj, q_norm_weight, k_norm_weight, key_blocks, value_blocks, block_tables, cu_seqlens, starts, block_size,
        max_new=max_new, eps=rope.rms_norm_eps, rope_theta=rope.rope_theta, partial_rotary_factor=rope.partial_rotary_factor,
    )


@dataclass(frozen=True)
class RopeConfig:
    """The fields of ``RuntimeConfig`` the full-attention prologue reads (``src/runtime_config.py:55-90``;
    ``rms_norm``, ``rotary_embeddings`` and ``apply_rotary_pos_emb`` of ``src/reference_ops.py:166-224``)."""

    rms_norm_eps: float = 1e-6
    rope_theta: float = 10_000_000.0
    partial_rotary_factor: float = 0.25


def full_attention_decode_step_device(
    q_proj: Any, k_proj: Any, v_proj: Any, q_norm_weight: Any, k_norm_weight: Any, key_blocks: Any, value_blocks: Any,
    tables: DeviceBatchPageTables, config: AttentionConfig, runtime: HotPathRuntime, rope: RopeConfig = RopeConfig(), *,
    no_alloc: bool = False,
) -> Any | None:
    """One decode token of a full-attention layer for every row of a running batch, from the
    projection outputs: ``tp_full_attention``'s norm/RoPE/append (``src/tp_runtime.py:511-525``)
    and paged decode with the output gate (``:551-610``, ``:673-695``), at TP = 1.

    ``q_proj`` ``(rows, H*2D)`` (query and gate halves of each head, as the projection writes
    them), ``k_proj``/``v_proj`` ``(rows, H_kv*D)``, bf16; ``tables.reserve_step()`` has run for
    the step.  One launch applies the q/k RMSNorm with the ``(1 + w)`` weights and the partial
    rotary embedding at each row's position and writes k and v to the reserved slots of this
    layer's shared pool; the batched decode follows, and the gate (read in place from
    ``q_proj``) multiplies its output.  Returns ``(rows, 1, H*D)`` in bf16 (rows without a
    request give zeros), or ``None`` -- counted by the reference's ladder -- when the caller must
    run its dense path; that is decided before anything is written.  Once the step's K/V are
    appended, errors raise instead of returning ``None``: with ``no_alloc`` a batch whose partials
    exceed the library's 32 MiB scratch raises ``RuntimeError`` with the token already in the
    cache, so the caller must not append it again.
    """
    rows = int(q_proj.shape[0])
    full = config.full_attention
    heads, head_dim, kv_heads = full.num_heads, full.head_dim, full.num_key_value_heads
    probe = _query_probe(q_proj, heads, head_dim)
    reason = _device_pool_reason(config, probe, key_blocks, value_blocks, tables)
    if reason == "no_kernel" and (rows != tables.rows or int(key_blocks.shape[1]) != kv_heads or int(key_blocks.shape[3]) != head_dim
                                  or str(key_blocks.dtype) != "torch.bfloat16" or str(q_proj.dtype) != "torch.bfloat16"):
        reason = "shape"
    if reason != "no_kernel":
        record_native_paged_dispatch(runtime, reason, native=False)
        return None
    import hip_ops

    cu = _row_offsets(rows, q_proj.device)
    with runtime.profile_scope("batch.full_attention.native_paged_device"):
        query, gate = _qk_norm_rope(q_proj, k_proj, v_proj, q_norm_weight, k_norm_weight, key_blocks, value_blocks, tables.block_tables,
                                    cu, tables.positions, tables.block_size, 1, rope)
        decode = hip_ops.paged_attention_decode_batched_noalloc if no_alloc else hip_ops.paged_attention_decode_batched
        heads_out = decode(query.view(rows, heads, 1, head_dim), tables.block_tables, key_blocks, value_blocks, tables.sequence_lengths,
                           tables.block_size)
    record_native_paged_dispatch(runtime, reason, native=True)
    if not full.output_gate:
        return heads_out.view(rows, 1, heads * head_dim)
    return _gate_heads(heads_out, gate.reshape(rows, 1, heads * head_dim))


_ROW_OFFSETS: dict[tuple[int, str], Any] = {}


def _row_offsets(rows: int, device: Any) -> Any:
    """``cu_seqlens`` of one token per row, ``[0, 1, .., rows]`` int32, cached per (rows, device)
    so a captured decode step reads a tensor that outlives the capture."""
    import torch

    key = (rows, str(device))
    cached = _ROW_OFFSETS.get(key)
    if cached is None:
        cached = torch.arange(rows + 1, dtype=torch.int32, device=device)
        _ROW_OFFSETS[key] = cached
    return cached


def _query_probe(q_proj: Any, heads: int, head_dim: int) -> Any:
    """The query half of ``q_proj`` ``(rows, H*2D)`` as ``(rows, H, 1, D)`` for the reason ladder;
    ``q_proj`` itself when it has another shape (the ladder then reports ``"shape"`` after its
    ``"disabled"`` and ``"cpu"`` checks, instead of a view error)."""
    shape = tuple(getattr(q_proj, "shape", ()))
    if len(shape) != 2 or shape[1] != heads * 2 * head_dim or q_proj.stride(-1) != 1:
        return q_proj
    return q_proj.view(shape[0], heads, 1, 2 * head_dim)[..., :head_dim]


def full_attention_prefill_device(
    q_proj: Any, k_proj: Any, v_proj: Any, q_norm_weight: Any, k_norm_weight: Any, key_blocks: Any, value_blocks: Any,
    step: PrefillStep, config: AttentionConfig, runtime: HotPathRuntime, rope: RopeConfig = RopeConfig(),
) -> Any | None:
    """A multi-token step (a prompt or one chunk of it) of a full-attention layer, from the
    projection outputs, on the native chunked prefill: ``tp_full_attention``
    (``src/tp_runtime.py:499-548``) at TP = 1 with the step's K/V appended to the layer's shared
    pool and causal attention over each row's cache and new tokens
    (``_tp_full_attention_paged_or_dense``, ``:551-610``, whose native branch is decode-only: the
    reference runs every prefill through the dense gather + masked softmax of ``:698-730``).

    ``q_proj`` ``(tokens, H*2D)``, ``k_proj``/``v_proj`` ``(tokens, H_kv*D)`` bf16, packed in the
    row order of ``step`` (``DeviceBatchPageTables.reserve_prefill``, run once per step for all
    layers); new token ``n`` of a row sits at position ``starts[row] + n``.  One launch applies
    the q/k RMSNorm and partial RoPE and writes k and v to the reserved slots; the prefill kernel
    then attends over the row's prefix and its new tokens causally and applies the output gate,
    read in place from ``q_proj``.  Returns ``(tokens, H*D)`` bf16.

    Ladder: the reference's reasons first (``"disabled"``, ``"cpu"``, ``"shape"``), then what the
    native kernels need -- a shared ``(P, H_kv, bs, D)`` bf16 pool of the tables' geometry.  A
    call that does not qualify returns ``None`` and counts as ``"prefill_or_multitoken"`` (the
    reference's reason for every multi-token call) or ``"shape"``, so the caller's dense path
    runs; nothing has been written by then.  Native calls count in ``native_prefill_hits``.
    """
    import torch

    tokens = int(q_proj.shape[0])
    full = config.full_attention
    heads, head_dim, kv_heads = full.num_heads, full.head_dim, full.num_key_value_heads
    probe = _query_probe(q_proj, heads, head_dim)
    if probe.dim() == 4:
        probe = probe[:1]  # one token stands for the step: the ladder reads heads and widths, not rows
    reason = paged_attention_fallback_reason(config, probe, key_blocks, value_blocks, seq_len=1, batched=False)
    if reason == "no_kernel":
        if key_blocks.dim() != 4:
            reason = "prefill_or_multitoken"  # per-request (reference-layout) pools: the dense path
        elif (tuple(value_blocks.shape) != tuple(key_blocks.shape) or int(key_blocks.shape[2]) != step.block_size
              or int(key_blocks.shape[1]) != kv_heads or int(key_blocks.shape[3]) != head_dim or tokens != step.total_tokens
              or key_blocks.dtype != torch.bfloat16 or q_proj.dtype != torch.bfloat16):
            reason = "shape"
    if reason != "no_kernel":
        record_native_paged_dispatch(runtime, reason, native=False)
        return None
    import hip_ops

    with runtime.profile_scope("full_attention.native_paged_prefill"):
        query, gate = _qk_norm_rope(q_proj, k_proj, v_proj, q_norm_weight, k_norm_weight, key_blocks, value_blocks, step.block_tables,
                                    step.cu_seqlens, step.starts, step.block_size, step.max_new, rope)
        out = hip_ops.paged_attention_prefill(query, step.cu_seqlens, step.starts, key_blocks, value_blocks, step.block_tables,
                                              step.block_size, max_new=step.max_new, gate=gate if full.output_gate else None)
    stats = runtime.paged_attention_stats
    stats.calls += 1
    stats.eligible += 1
    stats.native_prefill_hits += 1
    return out.view(tokens, heads * head_dim)


# --------------------------------------------------------------------------- linear attention


def prepare_recurrent_inputs(query: Any, key: Any, value: Any, g: Any, beta: Any, initial_state: Any = None) -> tuple[Any, ...]:
    """``_prepare_recurrent_gated_delta_inputs`` (``src/tp_runtime.py:2790-2805``), on the inputs' device."""
    import torch

    def l2(x: Any) -> Any:
        x = x.float()
        return x * (x * x).sum(dim=-1, keepdim=True).add(1e-6).rsqrt()

    q = l2(query).transpose(1, 2).float().contiguous()
    k = l2(key).transpose(1, 2).float().contiguous()
    v = value.transpose(1, 2).float().contiguous()
    b = beta.transpose(1, 2).float().contiguous()
    gg = g.transpose(1, 2).float().contiguous()
    batch, heads, _, key_dim = k.shape
    q = (q * (key_dim**-0.5)).contiguous()
    if initial_state is None:
        state = torch.zeros(batch, heads, key_dim, v.shape[-1], device=q.device, dtype=torch.float32)
    else:
        state = initial_state.to(device=q.device, dtype=torch.float32).contiguous()
    return q, k, v, gg, b, state


def recurrent_gated_delta_rule(query: Any, key: Any, value: Any, g: Any, beta: Any, *, initial_state: Any = None, return_state: bool = False) -> Any:
    """``_recurrent_gated_delta_rule`` (``src/tp_runtime.py:2744-2787``) on the HIP recurrent core.

    Token-major ``(B, S, H, d)`` inputs; returns ``(B, S, H, dv)`` in the query
    dtype (and the fp32 final state).  CUDA tensors only: a missing library
    raises ``RuntimeError`` instead of falling back.
    """
    import hip_ops

    initial_dtype = query.dtype
    q, k, v, gg, b, state = prepare_recurrent_inputs(query, key, value, g, beta, initial_state)
    output, final_state = hip_ops.linear_attention_recurrent_core(q, k, v, gg, b, state)
    out = output.transpose(1, 2).contiguous().to(initial_dtype)
    return (out, final_state) if return_state else out


def linear_attention_decode_batch(
    mixed_qkv: Any, a: Any, b: Any, a_log: Any, dt_bias: Any, conv_weight: Any, pool: LinearStatePool, slots: Any, config: AttentionConfig, *,
    out_dtype: Any = None, z: Any = None, norm_weight: Any = None, eps: float = 1e-6
) -> Any:
    """One decode token of a linear-attention layer for a batch of requests.

    ``mixed_qkv`` ``(B, qkv_dim)``, ``a``/``b`` ``(B, Hv)`` are the
    ``in_proj_*`` outputs of the step; request ``r`` keeps its conv and
    recurrent state in row ``slots[r]`` of ``pool`` (updated in place).
    Returns the core output ``(B, Hv, dv)`` before the gated RMSNorm, or, given
    ``z`` (the ``in_proj_z`` output ``(B, Hv*dv)``) and ``norm_weight``, after it
    (``src/reference_ops.py:284-287``), fused into the same kernel.  This
    replaces the stack / run / scatter of ``src/tp_runtime.py:2613-2717``.
    With 1, 2 or 4 value heads per key head the conv update runs inside the
    step's kernel (one launch, no activation round trip through HBM);
    otherwise it is a launch of its own before the step.
    """
    import torch

    import hip_ops

    lin = config.linear_attention
    odt = torch.bfloat16 if out_dtype is None else out_dtype
    if lin.value_heads // lin.key_heads in (1, 2, 4):
        return hip_ops.gated_delta_step_conv(mixed_qkv, pool.conv, conv_weight, a, b, a_log, dt_bias, pool.state, key_heads=lin.key_heads,
                                             slots=slots, out_dtype=odt, z=z, norm_weight=norm_weight, eps=eps)
    act = hip_ops.causal_conv1d_update(mixed_qkv, pool.conv, conv_weight, slots)
    return hip_ops.gated_delta_step(act, a, b, a_log, dt_bias, pool.state, key_heads=lin.key_heads, slots=slots,
                                    out_dtype=odt, z=z, norm_weight=norm_weight, eps=eps)


def linear_attention_prefill(mixed_qkv: Any, a: Any, b: Any, a_log: Any, dt_bias: Any, conv_weight: Any, config: AttentionConfig, *,
                             conv_state: Any = None, initial_state: Any = None, z: Any = None, norm_weight: Any = None,
                             eps: float = 1e-6) -> tuple[Any, Any, Any]:
    """Prefill of a linear-attention layer on the chunked kernel (``src/reference_ops.py:240-287``).

    ``mixed_qkv`` ``(B, S, qkv_dim)`` bf16 and ``a``/``b`` ``(B, S, Hv)`` are the ``in_proj_*``
    outputs.  Returns ``(core, final_state, conv_state)``: ``core`` ``(B, S, Hv, dv)`` bf16 is the
    recurrence output, or, given ``z`` (the ``in_proj_z`` output ``(B, S, Hv*dv)``) and
    ``norm_weight`` ``(dv,)``, the layer's output stage applied to it -- the gated RMSNorm with
    SiLU(z) of ``src/reference_ops.py:284-287`` (``src/tp_runtime.py:853-857``) -- as
    ``(B, S, Hv*dv)`` bf16, ready for ``out_proj``.
    """
    import hip_ops

    lin = config.linear_attention
    if (z is None) != (norm_weight is None):
        raise ValueError("linear_attention_prefill: z and norm_weight go together")
    core, state, conv = hip_ops.chunk_gated_delta_rule(
        mixed_qkv, a, b, a_log, dt_bias, conv_weight, key_heads=lin.key_heads, value_heads=lin.value_heads, conv_state=conv_state,
        initial_state=initial_state,
    )
    if z is None:
        return core, state, conv
    return hip_ops.gated_rms_norm(core, z, norm_weight, eps), state, conv


# --------------------------------------------------------------------------- fp8 projections


@dataclass
class LinearDispatchStats:
    """Counters of ``reference_ops.LinearDispatchStats`` (``src/reference_ops.py:29-51``).

    The ``moe_*`` fields are kept so code reading them still works; this build has no MoE path,
    so they stay 0.
    """

    calls: int = 0
    fp8_weight_calls: int = 0
    eligible_cuda_calls: int = 0
    cuda_kernel_hits: int = 0
    fallback_calls: int = 0
    fallback_disabled_cuda_kernel: int = 0
    fallback_missing_scale: int = 0
    fallback_hidden_not_cuda: int = 0
    fallback_weight_not_cuda: int = 0
    fallback_scale_not_cuda: int = 0
    fallback_weight_dtype: int = 0
    fallback_scale_dtype: int = 0
    fallback_hidden_alignment: int = 0
    fallback_weight_alignment: int = 0
    moe_calls: int = 0
    moe_packed_calls: int = 0
    moe_loop_calls: int = 0
    moe_single_token_dispatch_calls: int = 0
    moe_single_token_dispatch_hits: int = 0
    moe_single_token_local_assignments: int = 0
    moe_assignments: int = 0
    moe_local_assignments: int = 0

    def to_dict(self) -> dict[str, int]:
        return dict(vars(self))


def linear_native(hidden_states: Any, weight: Any, scale_inv: Any | None = None, *, use_cuda_kernel: bool = True,
                  stats: LinearDispatchStats | None = None) -> Any | None:
    """The native branch of the reference's ``linear`` (``src/reference_ops.py:436-495``).

    Same eligibility test and counters: an fp8 E4M3 weight (row-major, or packed by
    ``hip_ops.fp8_pack_weight``) with a bf16 ``scale_inv``, all on the GPU, the hidden size and the
    weight rows multiples of 128.  Eligible calls return ``hip_ops.fp8_e4m3_bf16_linear`` of
    ``hidden_states.float()`` (fp32); others return ``None`` and the caller keeps its own
    dequantise-and-``F.linear`` path, as the reference does (``:496-497``).
    """
    import torch

    import hip_ops

    packed = isinstance(weight, hip_ops.PackedFp8Weight)
    weight_tensor = weight.data if packed else weight
    has_scale = scale_inv is not None
    hidden_is_cuda = bool(getattr(hidden_states, "is_cuda", False))
    weight_is_cuda = bool(getattr(weight_tensor, "is_cuda", False))
    scale_is_cuda = bool(has_scale and getattr(scale_inv, "is_cuda", False))
    weight_is_fp8 = packed or weight.dtype == torch.float8_e4m3fn
    scale_is_bf16 = bool(has_scale and scale_inv.dtype == torch.bfloat16)
    hidden_aligned = hidden_states.shape[-1] % 128 == 0
    weight_aligned = weight.shape[0] % 128 == 0
    eligible = (use_cuda_kernel and has_scale and hidden_is_cuda and weight_is_cuda and scale_is_cuda and weight_is_fp8
                and scale_is_bf16 and hidden_aligned and weight_aligned)
    if stats is not None:
        stats.calls += 1
        if weight_is_fp8:
            stats.fp8_weight_calls += 1
        if eligible:
            stats.eligible_cuda_calls += 1
            stats.cuda_kernel_hits += 1
        else:
            stats.fallback_calls += 1
            if not use_cuda_kernel:
                stats.fallback_disabled_cuda_kernel += 1
            if weight_is_fp8 and not has_scale:
                stats.fallback_missing_scale += 1
            if weight_is_fp8 and not hidden_is_cuda:
                stats.fallback_hidden_not_cuda += 1
            if weight_is_fp8 and not weight_is_cuda:
                stats.fallback_weight_not_cuda += 1
            if weight_is_fp8 and has_scale and not scale_is_cuda:
                stats.fallback_scale_not_cuda += 1
            if not weight_is_fp8:
                stats.fallback_weight_dtype += 1
            if weight_is_fp8 and has_scale and not scale_is_bf16:
                stats.fallback_scale_dtype += 1
            if weight_is_fp8 and not hidden_aligned:
                stats.fallback_hidden_alignment += 1
            if weight_is_fp8 and not weight_aligned:
                stats.fallback_weight_alignment += 1
    if not eligible:
        return None
    return hip_ops.fp8_e4m3_bf16_linear(hidden_states.float(), weight, scale_inv)
