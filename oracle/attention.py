"""Oracle: dense masked GQA attention, paged decode and paged prefill.

Restates the reference CPU attention math:

* GQA head expansion -- ``_repeat_kv`` (``src/reference_ops.py:414-419``,
  ``src/tp_runtime.py:2736-2741``): query head ``h`` reads KV head
  ``h // (H / H_kv)``;
* masked causal softmax attention with the ``probs.to(query.dtype)`` cast point
  and the sigmoid output gate -- ``full_attention`` core
  (``src/reference_ops.py:353-360``) and ``_tp_full_attention_dense_from_kv``
  (``src/tp_runtime.py:698-730``);
* the batched decode form with per-row query positions and a padding mask --
  ``_tp_full_attention_batch_dense_from_kv`` (``src/tp_runtime.py:2558-2609``);
* paged decode = gather of the valid tokens (``src/decode_state.py:295-303``)
  followed by the dense form, with the zero output for empty rows of the
  reference's batched kernel (``src/csrc/fp8_linear_cuda.cu:987-992``).

Floating-point work uses PyTorch CPU in the reference's own cast order.

Pinning: ``tests/test_oracle_attention.py`` checks :func:`dense_attention`
against :func:`textbook_attention_fp64` (an independent float64 loop over
rows with an explicit max-subtracted softmax), and checks invariants that a
wrong index or a transposed operand would break: output invariance under
physical-block permutation, GQA == MHA on explicitly repeated KV, causality
(changing a future token leaves earlier rows unchanged), decode of the last
position == last row of prefill, and uniform attention for a zero query.
:func:`paged_prefill` is checked against the same fp64 loop with query
positions ``prefix + n`` over a shuffled pool whose unwritten slots hold
garbage (ragged prefixes including 0, lengths that are not block multiples,
GQA 16/2, a gate); :func:`reference_layout_decode_cpu` (and the ``"hpbd"``
branch of :func:`gather_dense`) against the fp64 loop and against
:func:`paged_decode` on a shared GQA pool holding the same tokens.
"""

from __future__ import annotations

import math

import numpy as np
import torch


def repeat_kv(hidden: torch.Tensor, repeats: int) -> torch.Tensor:
    """``_repeat_kv`` (``src/reference_ops.py:414-419``)."""
    if repeats == 1:
        return hidden
    batch, kv_heads, seq, dim = hidden.shape
    hidden = hidden[:, :, None, :, :].expand(batch, kv_heads, repeats, seq, dim)
    return hidden.reshape(batch, kv_heads * repeats, seq, dim)


def dense_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    *,
    position_offset: int | torch.Tensor = 0,
    valid_mask: torch.Tensor | None = None,
    gate: torch.Tensor | None = None,
    scale: float | None = None,
    cast_probs: bool = True,
) -> torch.Tensor:
    """Masked causal attention in head-major layout.

    ``query`` ``(B, H, S, D)``; ``key``/``value`` ``(B, H_kv, T, D)`` with
    ``H % H_kv == 0`` (expanded with :func:`repeat_kv` first, as the reference
    does before its cache append, ``src/reference_ops.py:349-350``).
    ``position_offset`` is the absolute position of query row 0, either an int
    (``src/reference_ops.py:355``) or a ``(B,)`` tensor of per-row positions
    (``src/tp_runtime.py:2589-2592``).  ``valid_mask`` ``(B, T)`` masks padded
    keys (``src/tp_runtime.py:2593-2595``).  ``gate`` ``(B, S, H*D)`` applies
    ``out * sigmoid(gate)`` (``src/reference_ops.py:360``).
    ``cast_probs=False`` keeps fp32 probabilities, as the reference's native
    fp32 kernel and its dense test restatement do
    (``tests/unit/test_fp8_cuda.py:1042-1045``).

    Returns ``(B, H, S, D)`` in ``query.dtype`` (fp32 when ``cast_probs`` is
    False).
    """
    batch, heads, seq, dim = query.shape
    kv_heads = key.shape[1]
    key = repeat_kv(key, heads // kv_heads)
    value = repeat_kv(value, heads // kv_heads)
    scale = dim**-0.5 if scale is None else scale
    scores = torch.matmul(query.float(), key.float().transpose(2, 3)) * scale
    total = key.shape[2]
    key_pos = torch.arange(total)
    if isinstance(position_offset, torch.Tensor):
        query_pos = position_offset.reshape(batch, 1, 1).long() + torch.arange(seq).reshape(1, seq, 1)
        mask = key_pos.reshape(1, 1, total) > query_pos  # (B, S, T)
    else:
        query_pos = torch.arange(position_offset, position_offset + seq)
        mask = (key_pos.unsqueeze(0) > query_pos.unsqueeze(1)).unsqueeze(0).expand(batch, seq, total)
    if valid_mask is not None:
        mask = mask | (~valid_mask.bool()).unsqueeze(1)
    scores = scores.masked_fill(mask.unsqueeze(1), torch.finfo(scores.dtype).min)
    probs = torch.softmax(scores, dim=-1, dtype=torch.float32)
    if cast_probs:
        probs = probs.to(query.dtype)
        out = torch.matmul(probs, value)
    else:
        out = torch.matmul(probs, value.float())
    if gate is not None:
        gate_heads = gate.reshape(batch, seq, heads, dim).transpose(1, 2)
        out = out * torch.sigmoid(gate_heads)
    return out


def textbook_attention_fp64(
    query: np.ndarray, key: np.ndarray, value: np.ndarray, *, query_positions: np.ndarray, valid: np.ndarray, scale: float
) -> np.ndarray:
    """Independent float64 restatement used only to pin :func:`dense_attention`.

    ``query`` ``(H, S, D)``, ``key``/``value`` ``(H_kv, T, D)``; query row ``s``
    at absolute position ``query_positions[s]`` sees keys ``t`` with
    ``t <= position`` and ``valid[t]``.
    """
    heads, seq, _dim = query.shape
    kv_heads = key.shape[0]
    group = heads // kv_heads
    out = np.zeros(query.shape, dtype=np.float64)
    for h in range(heads):
        g = h // group
        for s in range(seq):
            allowed = [t for t in range(key.shape[1]) if t <= query_positions[s] and valid[t]]
            if not allowed:
                continue
            logits = np.array([float(np.dot(query[h, s].astype(np.float64), key[g, t].astype(np.float64))) * scale for t in allowed])
            peak = logits.max()
            weights = np.exp(logits - peak)
            weights /= weights.sum()
            acc = np.zeros(query.shape[-1], dtype=np.float64)
            for w, t in zip(weights, allowed):
                acc += w * value[g, t].astype(np.float64)
            out[h, s] = acc
    return out


def gather_dense(pool: torch.Tensor, table: list[int] | torch.Tensor, valid: int, *, block_size: int, pool_layout: str) -> torch.Tensor:
    """Dense ``(heads, valid, D)`` KV of one request (``src/decode_state.py:395-404``)."""
    blocks = torch.as_tensor([int(x) for x in table[: math.ceil(valid / block_size)]], dtype=torch.long)
    if pool_layout == "hpbd":
        picked = pool.index_select(1, blocks)
    elif pool_layout == "phbd":
        picked = pool.index_select(0, blocks).transpose(0, 1)
    else:
        raise ValueError(pool_layout)
    heads, logical, bs, dim = picked.shape
    return picked.reshape(heads, logical * bs, dim)[:, :valid]


def paged_decode(
    query: torch.Tensor,
    key_pools: list[torch.Tensor],
    value_pools: list[torch.Tensor],
    tables: list[list[int]],
    seq_lens: list[int],
    *,
    block_size: int,
    pool_layout: str,
    scale: float | None = None,
    cast_probs: bool = True,
    gate: torch.Tensor | None = None,
) -> torch.Tensor:
    """Single-token attention of each row over its paged KV.

    ``query`` ``(B, H, 1, D)``; row ``b`` reads ``key_pools[b]`` (a
    ``(H_kv, P, bs, D)`` reference-layout pool or a ``(P, H_kv, bs, D)`` shared
    pool) through ``tables[b]``.  The query sits at position ``seq_lens[b]-1``
    (the token just appended, ``src/tp_runtime.py:2481-2483,2589-2592``).
    Rows with ``seq_lens[b] <= 0`` produce zeros
    (``src/csrc/fp8_linear_cuda.cu:987-992``).
    """
    batch, heads, _one, dim = query.shape
    out_dtype = query.dtype if cast_probs else torch.float32
    out = torch.zeros((batch, heads, 1, dim), dtype=out_dtype)
    for b in range(batch):
        if seq_lens[b] <= 0:
            continue
        k = gather_dense(key_pools[b], tables[b], seq_lens[b], block_size=block_size, pool_layout=pool_layout)
        v = gather_dense(value_pools[b], tables[b], seq_lens[b], block_size=block_size, pool_layout=pool_layout)
        row_gate = None if gate is None else gate[b : b + 1]
        out[b : b + 1] = dense_attention(
            query[b : b + 1],
            k.unsqueeze(0),
            v.unsqueeze(0),
            position_offset=seq_lens[b] - 1,
            scale=scale,
            cast_probs=cast_probs,
            gate=row_gate,
        ).to(out_dtype)
    return out


def paged_prefill(
    query: torch.Tensor,
    key_pool: torch.Tensor,
    value_pool: torch.Tensor,
    tables: list[list[int]],
    prefix_lens: list[int],
    new_lens: list[int],
    *,
    block_size: int,
    gate: torch.Tensor | None = None,
    scale: float | None = None,
) -> list[torch.Tensor]:
    """Causal attention of each request's new tokens over prefix + new KV.

    The new tokens' K/V are already appended to the shared ``(P, H_kv, bs, D)``
    pool at positions ``prefix..prefix+new-1``.  ``query`` is a list-free packed
    ``(sum_new, H, D)`` tensor in request order; ``gate`` the matching
    ``(sum_new, H*D)`` logits.  This is the reference's multi-token path
    (``src/tp_runtime.py:551-610`` falling back to
    ``_tp_full_attention_dense_from_kv`` ``:698-730`` with
    ``position_offset = prefix``).  Returns per-request ``(new, H, D)``.
    """
    outs = []
    offset = 0
    heads = query.shape[1]
    dim = query.shape[2]
    for b, (prefix, new) in enumerate(zip(prefix_lens, new_lens)):
        total = prefix + new
        k = gather_dense(key_pool, tables[b], total, block_size=block_size, pool_layout="phbd")
        v = gather_dense(value_pool, tables[b], total, block_size=block_size, pool_layout="phbd")
        q = query[offset : offset + new].transpose(0, 1).unsqueeze(0)  # (1, H, new, D)
        row_gate = None if gate is None else gate[offset : offset + new].reshape(1, new, heads * dim)
        out = dense_attention(q, k.unsqueeze(0), v.unsqueeze(0), position_offset=prefix, gate=row_gate, scale=scale)
        outs.append(out[0].transpose(0, 1).contiguous())
        offset += new
    return outs


def reference_layout_decode_cpu(
    query: torch.Tensor, key_repeated_pools: list[torch.Tensor], value_repeated_pools: list[torch.Tensor], tables: list[list[int]], seq_lens: list[int], *, block_size: int
) -> torch.Tensor:
    """The reference's CPU decode as the engine runs it, for the timed baseline.

    Caches hold post-``_repeat_kv`` heads (``src/tp_runtime.py:518-525``), a
    non-contiguous table forces the ``index_select`` gather
    (``src/decode_state.py:395-404``) and the dense fp32-score path runs
    (``src/tp_runtime.py:698-730``).
    """
    return paged_decode(
        query, key_repeated_pools, value_repeated_pools, tables, seq_lens, block_size=block_size, pool_layout="hpbd"
    )
