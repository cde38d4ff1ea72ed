"""GPU parity of the gated delta-rule kernels against ``oracle/gated_delta.py``.

Tolerances: fp32 recurrent states within 1e-3 relative (Frobenius), bf16
outputs within 2e-2 absolute/relative; the restated reference test keeps its
own 2e-5 (``tests/unit/test_fp8_cuda.py:999-1029``).
"""

from __future__ import annotations

import pytest
import torch

from oracle import gated_delta as gd

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _ops():
    import hip_ops

    return hip_ops


def _rel(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def test_recurrent_core_matches_reference_small_shapes() -> None:
    # tests/unit/test_fp8_cuda.py:999-1029 (seed 2, B2 H3 dk4 dv5)
    ops = _ops()
    torch.manual_seed(2)
    for seq_len, use_state in ((1, False), (1, True), (5, False), (5, True)):
        b, h, dk, dv = 2, 3, 4, 5
        q_raw = torch.randn((b, seq_len, h, dk))
        k_raw = torch.randn((b, seq_len, h, dk))
        v_raw = torch.randn((b, seq_len, h, dv))
        g_raw = -torch.rand((b, seq_len, h))
        beta_raw = torch.rand((b, seq_len, h))
        state0 = torch.randn((b, h, dk, dv)) * 0.1 if use_state else None
        q, k, v, g, beta, state = gd.prepare_inputs(q_raw, k_raw, v_raw, g_raw, beta_raw, state0)
        out, final = ops.linear_attention_recurrent_core(*(x.to(DEV) for x in (q, k, v, g, beta, state)))
        ref_out, ref_state = gd.recurrent_core(q, k, v, g, beta, state)
        torch.testing.assert_close(out.cpu(), ref_out, atol=2e-5, rtol=2e-5)
        torch.testing.assert_close(final.cpu(), ref_state, atol=2e-5, rtol=2e-5)


def test_recurrent_core_rejects_bf16() -> None:
    ops = _ops()
    x = torch.zeros((1, 1, 1, 4), device=DEV, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="query must be float32"):
        ops.linear_attention_recurrent_core(x, x, x, x[..., 0], x[..., 0], torch.zeros((1, 1, 4, 4), device=DEV))


def test_recurrent_core_128_register_path_matches_oracle() -> None:
    ops = _ops()
    gen = torch.Generator().manual_seed(31)
    b, h, s, d = 2, 4, 37, 128
    q_raw = torch.randn(b, s, h, d, generator=gen)
    k_raw = torch.randn(b, s, h, d, generator=gen)
    v_raw = torch.randn(b, s, h, d, generator=gen)
    g_raw = -torch.rand(b, s, h, generator=gen)
    beta_raw = torch.rand(b, s, h, generator=gen)
    state0 = torch.randn(b, h, d, d, generator=gen) * 0.1
    q, k, v, g, beta, state = gd.prepare_inputs(q_raw, k_raw, v_raw, g_raw, beta_raw, state0)
    out, final = ops.linear_attention_recurrent_core(*(x.to(DEV) for x in (q, k, v, g, beta, state)))
    ref_out, ref_state = gd.recurrent_core(q, k, v, g, beta, state)
    assert _rel(final, ref_state) < 1e-5
    assert _rel(out, ref_out) < 1e-5


def test_conv1d_prefill_matches_oracle_with_and_without_state() -> None:
    ops = _ops()
    gen = torch.Generator().manual_seed(32)
    b, t, c, kk = 3, 19, 300, 4
    x = torch.randn(b, t, c, generator=gen).to(torch.bfloat16)
    w = torch.randn(c, 1, kk, generator=gen)
    tail = torch.randn(b, c, kk - 1, generator=gen)
    for state in (None, tail):
        ref, ref_tail = gd.causal_conv1d(x.transpose(1, 2).float(), w, state)
        out, new_tail = ops.causal_conv1d_prefill(x.to(DEV), w.to(DEV), None if state is None else state.to(DEV))
        torch.testing.assert_close(out.cpu(), ref.transpose(1, 2), atol=1e-5, rtol=1e-5)
        torch.testing.assert_close(new_tail.cpu(), ref_tail, atol=0, rtol=0)


def test_conv1d_update_streams_like_prefill_with_slots() -> None:
    ops = _ops()
    gen = torch.Generator().manual_seed(33)
    b, t, c, kk = 2, 6, 130, 4
    x = torch.randn(b, t, c, generator=gen)
    w = torch.randn(c, kk, generator=gen)
    full, _ = gd.causal_conv1d(x.transpose(1, 2), w, None)
    pool = torch.zeros(5, c, kk - 1, device=DEV)
    slots = torch.tensor([3, 1], device=DEV, dtype=torch.int32)
    outs = []
    for step in range(t):
        outs.append(ops.causal_conv1d_update(x[:, step].contiguous().to(DEV), pool, w.to(DEV), slots).cpu())
    torch.testing.assert_close(torch.stack(outs, dim=1), full.transpose(1, 2), atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(pool[3].cpu(), x[0, -3:].T.contiguous(), atol=0, rtol=0)
    assert torch.count_nonzero(pool[0]) == 0


def _layer_inputs(seed: int, batch: int, seq: int, shape: gd.LinearShape):
    gen = torch.Generator().manual_seed(seed)
    mixed = torch.randn(batch, seq, shape.qkv_dim, generator=gen).to(torch.bfloat16)
    a = torch.randn(batch, seq, shape.value_heads, generator=gen)
    b = torch.randn(batch, seq, shape.value_heads, generator=gen)
    a_log = torch.randn(shape.value_heads, generator=gen) * 0.5
    dt_bias = torch.randn(shape.value_heads, generator=gen) * 0.5
    w = torch.randn(shape.qkv_dim, 1, shape.conv_kernel_dim, generator=gen) * 0.5
    return mixed, a, b, a_log, dt_bias, w


def test_fused_decode_steps_match_oracle_layer_core() -> None:
    """T decode steps (conv update + fused step) == the reference layer core over T tokens."""
    ops = _ops()
    shape = gd.LinearShape(key_heads=4, value_heads=8, key_head_dim=128, value_head_dim=128, conv_kernel_dim=4)
    batch, seq = 3, 6
    mixed, a, b, a_log, dt_bias, w = _layer_inputs(34, batch, seq, shape)
    gen = torch.Generator().manual_seed(35)
    state0 = torch.randn(batch, shape.value_heads, 128, 128, generator=gen) * 0.05
    tail0 = torch.randn(batch, shape.qkv_dim, 3, generator=gen)
    ref_core, ref_state, ref_tail = gd.linear_attention_core(mixed.float(), a, b, a_log, dt_bias, w, shape, conv_tail=tail0, initial_state=state0)
    slots = torch.tensor([4, 0, 2], device=DEV)
    state_pool = torch.zeros(5, shape.value_heads, 128, 128, device=DEV)
    conv_pool = torch.zeros(5, shape.qkv_dim, 3, device=DEV)
    state_pool[slots] = state0.to(DEV)
    conv_pool[slots] = tail0.to(DEV)
    outs = []
    for step in range(seq):
        act = ops.causal_conv1d_update(mixed[:, step].contiguous().to(DEV), conv_pool, w.to(DEV), slots)
        outs.append(
            ops.gated_delta_step(
                act, a[:, step].contiguous().to(DEV), b[:, step].contiguous().to(DEV), a_log.to(DEV), dt_bias.to(DEV), state_pool,
                key_heads=shape.key_heads, slots=slots, out_dtype=torch.float32,
            ).cpu()
        )
    core = torch.stack(outs, dim=1)
    assert _rel(state_pool[slots], ref_state) < 1e-3
    torch.testing.assert_close(core, ref_core, atol=2e-3, rtol=2e-3)
    torch.testing.assert_close(conv_pool[slots].cpu(), ref_tail, atol=0, rtol=0)
    assert torch.count_nonzero(state_pool[1]) == 0 and torch.count_nonzero(state_pool[3]) == 0


def test_fused_step_bf16_output_and_bf16_gates() -> None:
    ops = _ops()
    shape = gd.LinearShape(key_heads=16, value_heads=32, key_head_dim=128, value_head_dim=128, conv_kernel_dim=4)
    batch = 4
    mixed, a, b, a_log, dt_bias, w = _layer_inputs(36, batch, 1, shape)
    ref_core, ref_state, _ = gd.linear_attention_core(mixed.float(), a.to(torch.bfloat16).float(), b.to(torch.bfloat16).float(), a_log, dt_bias, w, shape)
    act = ops.causal_conv1d_update(mixed[:, 0].contiguous().to(DEV), torch.zeros(batch, shape.qkv_dim, 3, device=DEV), w.to(DEV))
    state = torch.zeros(batch, 32, 128, 128, device=DEV)
    out = ops.gated_delta_step(
        act, a[:, 0].to(torch.bfloat16).to(DEV), b[:, 0].to(torch.bfloat16).to(DEV), a_log.to(DEV), dt_bias.to(DEV), state, key_heads=16
    )
    assert out.dtype == torch.bfloat16
    torch.testing.assert_close(out.cpu().float(), ref_core[:, 0].float(), atol=2e-2, rtol=2e-2)
    assert _rel(state, ref_state) < 1e-3


@pytest.mark.parametrize("slot_dtype", [torch.int32, torch.int64])
def test_invalid_slots_give_zeros_and_leave_the_pools_untouched(slot_dtype) -> None:
    """A -1 pad or an id past the pool in ``slots``: that row's conv and step outputs are zeros,
    no state row changes, and the valid rows match a run without the invalid rows."""
    ops = _ops()
    shape = gd.LinearShape(key_heads=2, value_heads=4, key_head_dim=128, value_head_dim=128, conv_kernel_dim=4)
    mixed, a, b, a_log, dt_bias, w = _layer_inputs(37, 4, 1, shape)
    gen = torch.Generator().manual_seed(38)
    rows = 3
    state0 = (torch.randn(rows, shape.value_heads, 128, 128, generator=gen) * 0.05).to(DEV)
    conv0 = torch.randn(rows, shape.qkv_dim, 3, generator=gen).to(DEV)
    slots = torch.tensor([2, -1, 0, rows], device=DEV, dtype=slot_dtype)
    state_pool, conv_pool = state0.clone(), conv0.clone()
    x, av, bv = mixed[:, 0].contiguous().to(DEV), a[:, 0].contiguous().to(DEV), b[:, 0].contiguous().to(DEV)
    act = ops.causal_conv1d_update(x, conv_pool, w.to(DEV), slots)
    out = ops.gated_delta_step(act, av, bv, a_log.to(DEV), dt_bias.to(DEV), state_pool, key_heads=shape.key_heads, slots=slots,
                               out_dtype=torch.float32)
    z = torch.randn(4, shape.value_heads * 128, generator=gen).to(DEV)
    nw = torch.ones(128, device=DEV)
    state_norm = state0.clone()
    out_norm = ops.gated_delta_step(act, av, bv, a_log.to(DEV), dt_bias.to(DEV), state_norm, key_heads=shape.key_heads, slots=slots,
                                    out_dtype=torch.float32, z=z, norm_weight=nw)
    for bad in (1, 3):
        assert torch.count_nonzero(act[bad]) == 0
        assert torch.count_nonzero(out[bad]) == 0
        assert torch.count_nonzero(out_norm[bad]) == 0
    # slot 1 is no valid row's slot: untouched bit for bit
    assert torch.equal(state_pool[1], state0[1]) and torch.equal(conv_pool[1], conv0[1]) and torch.equal(state_norm[1], state0[1])
    # the valid rows equal the same step with only those rows
    good = torch.tensor([0, 2], device=DEV)
    ref_state, ref_conv = state0.clone(), conv0.clone()
    ref_slots = slots[good].contiguous()
    ref_act = ops.causal_conv1d_update(x[good].contiguous(), ref_conv, w.to(DEV), ref_slots)
    ref_out = ops.gated_delta_step(ref_act, av[good].contiguous(), bv[good].contiguous(), a_log.to(DEV), dt_bias.to(DEV), ref_state,
                                   key_heads=shape.key_heads, slots=ref_slots, out_dtype=torch.float32)
    assert torch.equal(act[good], ref_act) and torch.equal(out[good], ref_out)
    assert torch.equal(state_pool, ref_state) and torch.equal(conv_pool, ref_conv)


@pytest.mark.parametrize("key_heads,value_heads", [(2, 2), (2, 4), (1, 4)])
@pytest.mark.parametrize("x_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("norm", [False, True])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_conv_fused_step_equals_conv_update_then_step(key_heads, value_heads, x_dtype, norm, out_dtype) -> None:
    """qa_gated_delta_step_conv == qa_causal_conv1d_update followed by qa_gated_delta_step(_norm),
    bit for bit (outputs, recurrent states, conv states), over two tokens, with a -1 pad and an id
    past the pool among the slots."""
    ops = _ops()
    shape = gd.LinearShape(key_heads=key_heads, value_heads=value_heads, key_head_dim=128, value_head_dim=128, conv_kernel_dim=4)
    batch, rows = 5, 6
    mixed, a, b, a_log, dt_bias, w = _layer_inputs(41 + value_heads, batch, 2, shape)
    gen = torch.Generator().manual_seed(42)
    state0 = (torch.randn(rows, value_heads, 128, 128, generator=gen) * 0.05).to(DEV)
    conv0 = torch.randn(rows, shape.qkv_dim, 3, generator=gen).to(DEV)
    slots = torch.tensor([3, -1, 0, rows, 5], device=DEV, dtype=torch.int32)
    z = torch.randn(2, batch, value_heads * 128, generator=gen).to(torch.bfloat16).to(DEV)
    nw = (1 + 0.1 * torch.randn(128, generator=gen)).to(DEV)
    s_ref, c_ref = state0.clone(), conv0.clone()
    s_fused, c_fused = state0.clone(), conv0.clone()
    for step in range(2):
        x = mixed[:, step].to(x_dtype).contiguous().to(DEV)
        av, bv = a[:, step].contiguous().to(DEV), b[:, step].contiguous().to(DEV)
        kw = dict(key_heads=key_heads, slots=slots, out_dtype=out_dtype)
        if norm:
            kw.update(z=z[step], norm_weight=nw)
        act = ops.causal_conv1d_update(x, c_ref, w.to(DEV), slots)
        ref = ops.gated_delta_step(act, av, bv, a_log.to(DEV), dt_bias.to(DEV), s_ref, **kw)
        out = ops.gated_delta_step_conv(x, c_fused, w.to(DEV), av, bv, a_log.to(DEV), dt_bias.to(DEV), s_fused, **kw)
        assert out.dtype == out_dtype and torch.equal(out, ref), f"step {step}: max diff {(out.float() - ref.float()).abs().max().item()}"
        assert torch.equal(s_fused, s_ref) and torch.equal(c_fused, c_ref)
        for bad in (1, 3):
            assert torch.count_nonzero(out[bad]) == 0
    # rows 1, 2 and 4 are no valid request's slot: untouched
    for r in (1, 2, 4):
        assert torch.equal(s_fused[r], state0[r]) and torch.equal(c_fused[r], conv0[r])


@pytest.mark.parametrize("key_heads,value_heads", [(16, 32), (16, 16)])
@pytest.mark.parametrize("norm", [False, True])
def test_conv_fused_step_large_batch_equals_conv_update_then_step(key_heads, value_heads, norm) -> None:
    """A config-5-sized batch (80 rows x 16 key heads, more workgroups than the GPU holds at once):
    the fused step stays bit-equal to qa_causal_conv1d_update + qa_gated_delta_step(_norm) over two
    tokens, with a -1 pad and an id past the pool among the slots, and leaves unused pool rows
    untouched."""
    ops = _ops()
    shape = gd.LinearShape(key_heads=key_heads, value_heads=value_heads, key_head_dim=128, value_head_dim=128, conv_kernel_dim=4)
    batch, rows = 80, 84
    mixed, a, b, a_log, dt_bias, w = _layer_inputs(70 + value_heads, batch, 2, shape)
    gen = torch.Generator(device=DEV).manual_seed(71)
    state0 = torch.randn(rows, value_heads, 128, 128, generator=gen, device=DEV) * 0.05
    conv0 = torch.randn(rows, shape.qkv_dim, 3, generator=gen, device=DEV)
    slots = torch.randperm(rows, generator=torch.Generator().manual_seed(72))[:batch].to(torch.int64)
    slots[5] = -1
    slots[17] = rows
    used = set(int(s) for s in slots.tolist() if 0 <= s < rows)
    slots = slots.to(DEV)
    z = torch.randn(2, batch, value_heads * 128, generator=gen, device=DEV).to(torch.bfloat16)
    nw = 1 + 0.1 * torch.randn(128, generator=gen, device=DEV)
    s_ref, c_ref = state0.clone(), conv0.clone()
    s_fused, c_fused = state0.clone(), conv0.clone()
    for step in range(2):
        x = mixed[:, step].to(torch.bfloat16).contiguous().to(DEV)
        av, bv = a[:, step].contiguous().to(DEV), b[:, step].contiguous().to(DEV)
        kw = dict(key_heads=key_heads, slots=slots, out_dtype=torch.bfloat16)
        if norm:
            kw.update(z=z[step], norm_weight=nw)
        act = ops.causal_conv1d_update(x, c_ref, w.to(DEV), slots)
        ref = ops.gated_delta_step(act, av, bv, a_log.to(DEV), dt_bias.to(DEV), s_ref, **kw)
        out = ops.gated_delta_step_conv(x, c_fused, w.to(DEV), av, bv, a_log.to(DEV), dt_bias.to(DEV), s_fused, **kw)
        assert torch.equal(out, ref), f"step {step}: max diff {(out.float() - ref.float()).abs().max().item()}"
        assert torch.equal(s_fused, s_ref) and torch.equal(c_fused, c_ref)
        assert torch.count_nonzero(out[5]) == 0 and torch.count_nonzero(out[17]) == 0
    for r in range(rows):
        if r not in used:
            assert torch.equal(s_fused[r], state0[r]) and torch.equal(c_fused[r], conv0[r])


def test_conv_fused_step_rejects_unsupported_head_ratio() -> None:
    ops = _ops()
    shape = gd.LinearShape(key_heads=1, value_heads=3, key_head_dim=128, value_head_dim=128, conv_kernel_dim=4)
    x = torch.zeros(1, shape.qkv_dim, device=DEV)
    ab = torch.zeros(1, 3, device=DEV)
    with pytest.raises(RuntimeError, match="1, 2 or 4"):
        ops.gated_delta_step_conv(x, torch.zeros(1, shape.qkv_dim, 3, device=DEV), torch.zeros(shape.qkv_dim, 4, device=DEV), ab, ab,
                                  torch.zeros(3, device=DEV), torch.zeros(3, device=DEV), torch.zeros(1, 3, 128, 128, device=DEV), key_heads=1)


@pytest.mark.parametrize("conv_kernel", [2, 3, 8])
def test_conv_fused_step_other_conv_kernels_and_strided_rows(conv_kernel) -> None:
    """Conv kernel sizes other than the model's 4, and x rows that are a slice of a wider
    projection output: still equal to qa_causal_conv1d_update + qa_gated_delta_step bit for bit."""
    ops = _ops()
    shape = gd.LinearShape(key_heads=2, value_heads=4, key_head_dim=128, value_head_dim=128, conv_kernel_dim=conv_kernel)
    batch, rows = 3, 4
    mixed, a, b, a_log, dt_bias, w = _layer_inputs(60 + conv_kernel, batch, 1, shape)
    gen = torch.Generator().manual_seed(61)
    state0 = (torch.randn(rows, 4, 128, 128, generator=gen) * 0.05).to(DEV)
    conv0 = torch.randn(rows, shape.qkv_dim, conv_kernel - 1, generator=gen).to(DEV)
    slots = torch.tensor([2, 0, 3], device=DEV, dtype=torch.int64)
    wide = torch.randn(batch, shape.qkv_dim + 96, generator=gen).to(torch.bfloat16).to(DEV)
    wide[:, 32 : 32 + shape.qkv_dim] = mixed[:, 0].to(DEV)
    x = wide[:, 32 : 32 + shape.qkv_dim]  # row stride qkv_dim + 96
    av, bv = a[:, 0].contiguous().to(DEV), b[:, 0].contiguous().to(DEV)
    s_ref, c_ref, s_fused, c_fused = state0.clone(), conv0.clone(), state0.clone(), conv0.clone()
    act = ops.causal_conv1d_update(x.contiguous(), c_ref, w.to(DEV), slots)
    ref = ops.gated_delta_step(act, av, bv, a_log.to(DEV), dt_bias.to(DEV), s_ref, key_heads=2, slots=slots)
    out = ops.gated_delta_step_conv(x, c_fused, w.to(DEV), av, bv, a_log.to(DEV), dt_bias.to(DEV), s_fused, key_heads=2, slots=slots)
    assert torch.equal(out, ref)
    assert torch.equal(s_fused, s_ref) and torch.equal(c_fused, c_ref)


def test_gate_inputs_on_the_host_are_rejected() -> None:
    """a / b given as host tensors raise the wrappers' error instead of reaching a kernel."""
    ops = _ops()
    shape = gd.LinearShape(key_heads=2, value_heads=4, key_head_dim=128, value_head_dim=128, conv_kernel_dim=4)
    batch = 2
    mixed, a, b, a_log, dt_bias, w = _layer_inputs(80, batch, 1, shape)
    x = mixed[:, 0].contiguous().to(DEV)
    state = torch.zeros(batch, 4, 128, 128, device=DEV)
    conv = torch.zeros(batch, shape.qkv_dim, 3, device=DEV)
    act = ops.causal_conv1d_update(x, conv.clone(), w.to(DEV))
    a_host, b_dev = a[:, 0].contiguous(), b[:, 0].contiguous().to(DEV)
    with pytest.raises(RuntimeError, match="a must be CUDA"):
        ops.gated_delta_step(act, a_host, b_dev, a_log.to(DEV), dt_bias.to(DEV), state, key_heads=2)
    with pytest.raises(RuntimeError, match="a must be CUDA"):
        ops.gated_delta_step_conv(x, conv, w.to(DEV), a_host, b_dev, a_log.to(DEV), dt_bias.to(DEV), state, key_heads=2)
    with pytest.raises(RuntimeError, match="b must be CUDA"):
        ops.gated_delta_step(act, a_host.to(DEV), b[:, 0].contiguous(), a_log.to(DEV), dt_bias.to(DEV), state, key_heads=2)
    assert torch.count_nonzero(state) == 0 and torch.count_nonzero(conv) == 0
