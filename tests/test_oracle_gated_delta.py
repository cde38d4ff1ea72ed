"""Pins ``oracle/gated_delta.py``: scalar fp64 loops, closed forms, chunked form."""

from __future__ import annotations

import numpy as np
import torch

from oracle import gated_delta as gd


def _prepared(seed: int, batch=1, heads=2, seq=6, dk=4, dv=5, with_state=True):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(batch, seq, heads, dk, generator=gen)
    k = torch.randn(batch, seq, heads, dk, generator=gen)
    v = torch.randn(batch, seq, heads, dv, generator=gen)
    g = -torch.rand(batch, seq, heads, generator=gen)
    beta = torch.rand(batch, seq, heads, generator=gen)
    state = torch.randn(batch, heads, dk, dv, generator=gen) * 0.1 if with_state else None
    return gd.prepare_inputs(q, k, v, g, beta, state)


def test_recurrent_core_matches_scalar_fp64() -> None:
    q, k, v, g, beta, state = _prepared(0)
    out, final = gd.recurrent_core(q, k, v, g, beta, state)
    for h in range(q.shape[1]):
        ref_out, ref_state = gd.delta_rule_scalar_fp64(q[0, h].numpy(), k[0, h].numpy(), v[0, h].numpy(), g[0, h].numpy(), beta[0, h].numpy(), state[0, h].numpy())
        np.testing.assert_allclose(out[0, h].numpy(), ref_out, rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(final[0, h].numpy(), ref_state, rtol=1e-5, atol=1e-5)


def test_single_token_closed_form() -> None:
    q, k, v, g, beta, state = _prepared(1, seq=1)
    out, final = gd.recurrent_core(q, k, v, g, beta, state)
    s0 = state[0, 0].double() * torch.exp(g[0, 0, 0].double())
    kt = k[0, 0, 0].double()
    delta = (v[0, 0, 0].double() - s0.T @ kt) * beta[0, 0, 0].double()
    s1 = s0 + torch.outer(kt, delta)
    torch.testing.assert_close(final[0, 0].double(), s1, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(out[0, 0, 0].double(), s1.T @ q[0, 0, 0].double(), rtol=1e-5, atol=1e-6)


def test_beta_zero_is_pure_decay() -> None:
    q, k, v, g, beta, state = _prepared(2)
    beta = torch.zeros_like(beta)
    out, final = gd.recurrent_core(q, k, v, g, beta, state)
    total = torch.exp(g.sum(dim=-1))  # (B, H)
    torch.testing.assert_close(final, state * total[..., None, None], rtol=1e-5, atol=1e-7)
    # o_t = S_t^T q_t with S_t = exp(cumsum g) S0
    cum = torch.exp(torch.cumsum(g, dim=-1))
    expect = torch.einsum("bhs,bhkv,bhsk->bhsv", cum, state, q)
    torch.testing.assert_close(out, expect, rtol=1e-5, atol=1e-6)


def test_orthonormal_keys_with_beta_one_overwrite_columns() -> None:
    dk, dv = 4, 3
    basis = torch.eye(dk)
    k = basis[[2, 0]].reshape(1, 1, 2, dk)  # tokens write rows 2 then 0
    v = torch.tensor([[[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]]]).reshape(1, 1, 2, dv)
    q = basis[[2, 0]].reshape(1, 1, 2, dk)
    g = torch.zeros(1, 1, 2)
    beta = torch.ones(1, 1, 2)
    state = torch.full((1, 1, dk, dv), 9.0)
    out, final = gd.recurrent_core(q, k, v, g, beta, state)
    expect = torch.full((dk, dv), 9.0)
    expect[2] = torch.tensor([1.0, 2.0, 3.0])
    expect[0] = torch.tensor([4.0, 5.0, 6.0])
    torch.testing.assert_close(final[0, 0], expect, rtol=0, atol=1e-6)
    torch.testing.assert_close(out[0, 0, 1], torch.tensor([4.0, 5.0, 6.0]), rtol=0, atol=1e-6)


def test_split_sequence_through_state_equals_full() -> None:
    q, k, v, g, beta, state = _prepared(3, seq=9)
    full_out, full_state = gd.recurrent_core(q, k, v, g, beta, state)
    first_out, mid = gd.recurrent_core(q[:, :, :4], k[:, :, :4], v[:, :, :4], g[:, :, :4], beta[:, :, :4], state)
    second_out, end = gd.recurrent_core(q[:, :, 4:], k[:, :, 4:], v[:, :, 4:], g[:, :, 4:], beta[:, :, 4:], mid)
    torch.testing.assert_close(torch.cat([first_out, second_out], dim=2), full_out, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(end, full_state, rtol=1e-5, atol=1e-6)


def test_chunked_form_matches_scalar_recurrence() -> None:
    q, k, v, g, beta, state = _prepared(4, seq=21, dk=6, dv=5)
    for h in range(2):
        args = [x[0, h].numpy() for x in (q, k, v, g, beta)]
        ref_out, ref_state = gd.delta_rule_scalar_fp64(*args, state[0, h].numpy())
        for chunk in (1, 4, 8, 64):
            out, final = gd.chunked_delta_rule_fp64(*args, state[0, h].numpy(), chunk)
            np.testing.assert_allclose(out, ref_out, rtol=1e-9, atol=1e-10)
            np.testing.assert_allclose(final, ref_state, rtol=1e-9, atol=1e-10)


def test_conv_matches_direct_tap_sum_and_streaming() -> None:
    gen = torch.Generator().manual_seed(5)
    x = torch.randn(2, 6, 9, generator=gen)
    w = torch.randn(6, 1, 4, generator=gen)
    tail = torch.randn(2, 6, 3, generator=gen)
    out, new_tail = gd.causal_conv1d(x, w, tail)
    direct = gd.causal_conv1d_direct_fp64(x.numpy(), w[:, 0].numpy(), tail.numpy())
    np.testing.assert_allclose(out.numpy(), torch.nn.functional.silu(torch.from_numpy(direct)).numpy(), rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(new_tail, x[:, :, -3:])
    # streaming 5 + 4 tokens == 9 at once
    a, tail_a = gd.causal_conv1d(x[:, :, :5], w, tail)
    b, tail_b = gd.causal_conv1d(x[:, :, 5:], w, tail_a)
    torch.testing.assert_close(torch.cat([a, b], dim=2), out, rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(tail_b, new_tail)


def test_gating_closed_form() -> None:
    a = torch.tensor([[0.0, 1.0]])
    b = torch.tensor([[0.0, 2.0]])
    g, beta = gd.gating(a, b, torch.zeros(2), torch.zeros(2))
    torch.testing.assert_close(beta, torch.tensor([[0.5, 1.0 / (1.0 + np.exp(-2.0))]], dtype=torch.float32), rtol=1e-6, atol=1e-7)
    torch.testing.assert_close(g, torch.tensor([[-np.log(2.0), -np.log(1.0 + np.e)]], dtype=torch.float32), rtol=1e-6, atol=1e-7)


def test_layer_core_head_mapping_value_head_j_reads_qk_head_j_over_2() -> None:
    shape = gd.LinearShape(key_heads=2, value_heads=4, key_head_dim=4, value_head_dim=3, conv_kernel_dim=4)
    gen = torch.Generator().manual_seed(6)
    mixed = torch.randn(1, 5, shape.qkv_dim, generator=gen)
    a = torch.randn(1, 5, 4, generator=gen)
    b = torch.randn(1, 5, 4, generator=gen)
    w = torch.randn(shape.qkv_dim, 1, 4, generator=gen)
    core, state, tail = gd.linear_attention_core(mixed, a, b, torch.zeros(4), torch.zeros(4), w, shape)
    # recompute head 3 by hand with qk head 1
    conv, _ = gd.causal_conv1d(mixed.transpose(1, 2), w, None)
    conv = conv.transpose(1, 2)
    q = conv[..., 4:8].reshape(1, 5, 1, 4)
    k = conv[..., 12:16].reshape(1, 5, 1, 4)
    v = conv[..., 16 + 9 : 16 + 12].reshape(1, 5, 1, 3)
    g, beta = gd.gating(a[..., 3:4], b[..., 3:4], torch.zeros(1), torch.zeros(1))
    out, st = gd.recurrent_gated_delta_rule(q, k, v, g, beta)
    torch.testing.assert_close(core[:, :, 3:4], out, rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(state[:, 3:4], st, rtol=1e-6, atol=1e-6)
    assert tail.shape == (1, shape.qkv_dim, 3)
