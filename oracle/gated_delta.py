"""Oracle: causal conv1d, gating, L2 norm and the gated delta rule.

Restates the reference CPU math of the linear-attention (gated delta-rule)
layers:

* depthwise causal conv1d + SiLU, with and without a ``K-1`` token tail --
  ``linear_attention`` (``src/reference_ops.py:240-258``) and its batched twin
  (``src/tp_runtime.py:2635-2659``);
* the q/k/v channel split and head reshape (``src/reference_ops.py:259-270``);
* gating ``beta = sigmoid(b)``, ``g = -exp(A_log) * softplus(a + dt_bias)``
  (``src/reference_ops.py:271-275``);
* q/k head repeat for the value heads (``src/reference_ops.py:276-279``);
* ``l2_norm`` (``src/reference_ops.py:181-183``) and the input preparation
  (``src/tp_runtime.py:2790-2805``);
* the per-token gated delta recurrence ``recurrent_gated_delta_rule``
  (``src/reference_ops.py:291-322``).

Pinning: ``tests/test_oracle_gated_delta.py`` checks the recurrence against
:func:`delta_rule_scalar_fp64` (scalar float64 loops), the closed forms
``T = 1``, ``beta = 0`` (pure decay) and orthonormal-key column overwrite,
``prefill(T1) + prefill(T2) == prefill(T1 + T2)`` through the carried state,
and the chunked WY form :func:`chunked_delta_rule_fp64` (Yang et al., "Gated
Delta Networks", ICLR 2025) against the recurrence.  The conv is checked
against a direct sum over taps and streaming-with-tail == full sequence.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch
import torch.nn.functional as F


@dataclass(frozen=True)
class LinearShape:
    """Head geometry of a linear-attention layer (``src/runtime_config.py:15-30``)."""

    key_heads: int
    value_heads: int
    key_head_dim: int
    value_head_dim: int
    conv_kernel_dim: int

    @property
    def key_dim(self) -> int:
        return self.key_heads * self.key_head_dim

    @property
    def value_state_dim(self) -> int:
        return self.value_heads * self.value_head_dim

    @property
    def qkv_dim(self) -> int:
        return 2 * self.key_dim + self.value_state_dim


def l2_norm(hidden: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """``l2_norm`` (``src/reference_ops.py:181-183``)."""
    states = hidden.float()
    return states * (states * states).sum(dim=-1, keepdim=True).add(eps).rsqrt()


def causal_conv1d(conv_input: torch.Tensor, weight: torch.Tensor, tail: torch.Tensor | None) -> tuple[torch.Tensor, torch.Tensor]:
    """Depthwise causal conv1d + SiLU on ``(B, C, S)`` fp32 input.

    ``weight`` is ``(C, 1, K)`` (or ``(C, K)``).  ``tail`` ``(B, C, K-1)`` or
    None for a fresh sequence (zeros, ``src/reference_ops.py:253-254``).
    Returns ``(silu(conv), new_tail)``; the streaming form is
    ``src/reference_ops.py:255-258``.
    """
    batch, channels, _seq = conv_input.shape
    if weight.dim() == 2:
        weight = weight.unsqueeze(1)
    kernel = weight.shape[-1]
    conv_input = conv_input.float()
    weight = weight.float()
    if tail is None:
        tail = torch.zeros(batch, channels, kernel - 1, dtype=torch.float32)
    padded = torch.cat((tail.float(), conv_input), dim=2)
    new_tail = padded[:, :, -(kernel - 1) :] if kernel > 1 else tail
    out = F.conv1d(padded, weight, padding=0, groups=channels)
    return F.silu(out), new_tail.contiguous()


def causal_conv1d_direct_fp64(conv_input: np.ndarray, weight: np.ndarray, tail: np.ndarray) -> np.ndarray:
    """Direct tap sum ``y[c,t] = sum_i w[c,i] * x_pad[c, t+i]`` (no SiLU), float64."""
    padded = np.concatenate([tail.astype(np.float64), conv_input.astype(np.float64)], axis=-1)
    kernel = weight.shape[-1]
    seq = conv_input.shape[-1]
    out = np.zeros(conv_input.shape, dtype=np.float64)
    for i in range(kernel):
        out += weight[None, :, i : i + 1].astype(np.float64) * padded[:, :, i : i + seq]
    return out


def gating(a: torch.Tensor, b: torch.Tensor, a_log: torch.Tensor, dt_bias: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """``beta = sigmoid(b)``; ``g = -exp(A_log) * softplus(a + dt_bias)`` (``src/reference_ops.py:271-275``)."""
    beta = torch.sigmoid(b)
    g = -a_log.float().exp() * F.softplus(a.float() + dt_bias.float())
    return g, beta


def recurrent_gated_delta_rule(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    g: torch.Tensor,
    beta: torch.Tensor,
    *,
    initial_state: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """``recurrent_gated_delta_rule`` (``src/reference_ops.py:291-322``).

    Inputs are token-major ``(B, S, H, d)`` (``g``/``beta`` ``(B, S, H)``) before
    L2 norm.  Returns ``(out (B, S, H, dv) in query.dtype, final_state fp32)``.
    """
    initial_dtype = query.dtype
    query, key, value, g, beta, state = prepare_inputs(query, key, value, g, beta, initial_state)
    out, state = recurrent_core(query, key, value, g, beta, state)
    return out.transpose(1, 2).contiguous().to(initial_dtype), state


def prepare_inputs(query, key, value, g, beta, initial_state=None):
    """``_prepare_recurrent_gated_delta_inputs`` (``src/tp_runtime.py:2790-2805``).

    Returns head-major ``(B, H, S, d)`` fp32 tensors with L2-normalised q/k,
    ``q *= dk**-0.5`` and a zero state when none is given.
    """
    query = l2_norm(query).transpose(1, 2).float().contiguous()
    key = l2_norm(key).transpose(1, 2).float().contiguous()
    value = value.transpose(1, 2).float().contiguous()
    beta = beta.transpose(1, 2).float().contiguous()
    g = g.transpose(1, 2).float().contiguous()
    batch, heads, _seq, key_dim = key.shape
    value_dim = value.shape[-1]
    query = (query * (key_dim**-0.5)).contiguous()
    if initial_state is None:
        state = torch.zeros(batch, heads, key_dim, value_dim, dtype=torch.float32)
    else:
        state = initial_state.to(dtype=torch.float32).contiguous()
    return query, key, value, g, beta, state


def recurrent_core(query, key, value, g, beta, state):
    """Per-token loop of ``src/reference_ops.py:310-318`` on prepared ``(B, H, S, d)`` inputs.

    This is also the contract of ``linear_attention_recurrent_core``
    (``src/fp8_cuda.py:206-214``): returns ``(output (B, H, S, dv) fp32, state)``.
    """
    batch, heads, seq, _ = key.shape
    value_dim = value.shape[-1]
    state = state.clone()
    output = torch.zeros(batch, heads, seq, value_dim, dtype=torch.float32)
    for index in range(seq):
        q_t = query[:, :, index]
        k_t = key[:, :, index]
        v_t = value[:, :, index]
        state = state * g[:, :, index].exp().unsqueeze(-1).unsqueeze(-1)
        kv_mem = (state * k_t.unsqueeze(-1)).sum(dim=-2)
        delta = (v_t - kv_mem) * beta[:, :, index].unsqueeze(-1)
        state = state + k_t.unsqueeze(-1) * delta.unsqueeze(-2)
        output[:, :, index] = (state * q_t.unsqueeze(-1)).sum(dim=-2)
    return output, state


def linear_attention_core(
    mixed_qkv: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
    a_log: torch.Tensor,
    dt_bias: torch.Tensor,
    conv_weight: torch.Tensor,
    shape: LinearShape,
    *,
    conv_tail: torch.Tensor | None = None,
    initial_state: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Linear-attention layer core between ``in_proj_*`` and the output norm.

    ``mixed_qkv`` ``(B, S, qkv_dim)`` is the ``in_proj_qkv`` output; ``a``/``b``
    ``(B, S, H_v)`` the ``in_proj_a``/``in_proj_b`` outputs.  Follows
    ``src/reference_ops.py:240-283`` with a cache object's ``conv_tail`` and
    ``state``.  Returns ``(core (B, S, H_v, dv) fp32, final_state, new_tail)``.
    """
    batch, seq, _ = mixed_qkv.shape
    conv_input = mixed_qkv.transpose(1, 2).float()
    mixed, new_tail = causal_conv1d(conv_input, conv_weight, conv_tail)
    mixed = mixed.transpose(1, 2)
    query, key, value = torch.split(mixed, [shape.key_dim, shape.key_dim, shape.value_state_dim], dim=-1)
    query = query.reshape(batch, seq, shape.key_heads, shape.key_head_dim)
    key = key.reshape(batch, seq, shape.key_heads, shape.key_head_dim)
    value = value.reshape(batch, seq, shape.value_heads, shape.value_head_dim)
    g, beta = gating(a, b, a_log, dt_bias)
    repeats = shape.value_heads // shape.key_heads
    if repeats > 1:
        query = query.repeat_interleave(repeats, dim=2)
        key = key.repeat_interleave(repeats, dim=2)
    core, state = recurrent_gated_delta_rule(query, key, value, g, beta, initial_state=initial_state)
    return core, state, new_tail


def delta_rule_scalar_fp64(q: np.ndarray, k: np.ndarray, v: np.ndarray, g: np.ndarray, beta: np.ndarray, state: np.ndarray):
    """Scalar float64 restatement on prepared inputs of one (batch, head).

    ``q``/``k`` ``(S, dk)`` (already normalised and scaled), ``v`` ``(S, dv)``,
    ``g``/``beta`` ``(S,)``, ``state`` ``(dk, dv)``.  Used only to pin
    :func:`recurrent_core`.
    """
    state = state.astype(np.float64).copy()
    seq, dk = k.shape
    dv = v.shape[1]
    out = np.zeros((seq, dv), dtype=np.float64)
    for t in range(seq):
        decay = np.exp(np.float64(g[t]))
        for i in range(dk):
            for j in range(dv):
                state[i, j] *= decay
        for j in range(dv):
            mem = 0.0
            for i in range(dk):
                mem += state[i, j] * np.float64(k[t, i])
            delta = (np.float64(v[t, j]) - mem) * np.float64(beta[t])
            for i in range(dk):
                state[i, j] += np.float64(k[t, i]) * delta
        for j in range(dv):
            acc = 0.0
            for i in range(dk):
                acc += state[i, j] * np.float64(q[t, i])
            out[t, j] = acc
    return out, state


def chunked_delta_rule_fp64(q: np.ndarray, k: np.ndarray, v: np.ndarray, g: np.ndarray, beta: np.ndarray, state: np.ndarray, chunk: int):
    """Chunked (WY / UT-transform) form of the gated delta rule, float64.

    Within a chunk with cumulative log-decay ``G_t`` and initial state ``S0``:
    ``A[t,i] = beta_t * exp(G_t - G_i) * (k_t . k_i)`` for ``i < t``,
    ``T = (I + A)^-1``, ``U = T (beta * v)``, ``W = T (beta * exp(G) * k)``,
    ``delta = U - W S0``,
    ``o = exp(G) * (q S0) + ((q k^T) * exp(G_t - G_i))_{i <= t} delta``,
    ``S_end = exp(G_C) S0 + k^T (exp(G_C - G) * delta)``.
    This is the algorithm the device chunked-prefill kernel implements; it is
    pinned here against :func:`delta_rule_scalar_fp64`.
    """
    state = state.astype(np.float64).copy()
    seq = k.shape[0]
    dv = v.shape[1]
    out = np.zeros((seq, dv), dtype=np.float64)
    for start in range(0, seq, chunk):
        end = min(seq, start + chunk)
        qc = q[start:end].astype(np.float64)
        kc = k[start:end].astype(np.float64)
        vc = v[start:end].astype(np.float64)
        bc = beta[start:end].astype(np.float64)
        gcum = np.cumsum(g[start:end].astype(np.float64))
        n = end - start
        diff = gcum[:, None] - gcum[None, :]
        lower_strict = np.tril(np.ones((n, n), dtype=bool), -1)
        lower = np.tril(np.ones((n, n), dtype=bool), 0)
        decay = np.where(lower, np.exp(np.where(lower, diff, 0.0)), 0.0)
        a_mat = np.where(lower_strict, bc[:, None] * decay * (kc @ kc.T), 0.0)
        t_mat = np.linalg.inv(np.eye(n) + a_mat)
        u = t_mat @ (bc[:, None] * vc)
        w = t_mat @ (bc[:, None] * np.exp(gcum)[:, None] * kc)
        delta = u - w @ state
        out[start:end] = np.exp(gcum)[:, None] * (qc @ state) + ((qc @ kc.T) * decay) @ delta
        state = np.exp(gcum[-1]) * state + kc.T @ (np.exp(gcum[-1] - gcum)[:, None] * delta)
    return out, state
