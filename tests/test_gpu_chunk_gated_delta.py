"""GPU chunked gated delta-rule prefill against the oracle layer core.

Checks: bf16/fp32 outputs within 2e-2, fp32 final state within 1e-3 relative
(Frobenius), final conv state bit-exact; ragged last chunk; carried conv and
recurrent state; weak decay (long memory); prefill followed by decode steps
equals one longer prefill.
"""

from __future__ import annotations

import pytest
import torch

from oracle import gated_delta as gd

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _rel(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def _inputs(seed: int, batch: int, seq: int, shape: gd.LinearShape, *, a_log_scale: float = 0.0, a_log_shift: float = 0.0):
    gen = torch.Generator().manual_seed(seed)
    mixed = torch.randn(batch, seq, shape.qkv_dim, generator=gen).to(torch.bfloat16)
    a = torch.randn(batch, seq, shape.value_heads, generator=gen)
    b = torch.randn(batch, seq, shape.value_heads, generator=gen)
    a_log = torch.randn(shape.value_heads, generator=gen) * a_log_scale + a_log_shift
    dt_bias = torch.zeros(shape.value_heads)
    w = torch.randn(shape.qkv_dim, 1, 4, generator=gen) * 0.5
    return mixed, a, b, a_log, dt_bias, w


def _run(mixed, a, b, a_log, dt_bias, w, shape, *, conv_state=None, state=None, out_dtype=torch.bfloat16):
    import hip_ops

    return hip_ops.chunk_gated_delta_rule(
        mixed.to(DEV), a.to(DEV), b.to(DEV), a_log.to(DEV), dt_bias.to(DEV), w.to(DEV), key_heads=shape.key_heads, value_heads=shape.value_heads,
        conv_state=None if conv_state is None else conv_state.to(DEV), initial_state=None if state is None else state.to(DEV), out_dtype=out_dtype,
    )


SHAPE = gd.LinearShape(key_heads=2, value_heads=4, key_head_dim=128, value_head_dim=128, conv_kernel_dim=4)


def test_chunked_prefill_zero_state_ragged_matches_oracle() -> None:
    mixed, a, b, a_log, dt_bias, w = _inputs(41, 2, 150, SHAPE)
    ref_core, ref_state, ref_tail = gd.linear_attention_core(mixed.float(), a, b, a_log, dt_bias, w, SHAPE)
    out, state, tail = _run(mixed, a, b, a_log, dt_bias, w, SHAPE)
    torch.testing.assert_close(out.cpu().float(), ref_core, atol=2e-2, rtol=2e-2)
    assert _rel(state, ref_state) < 1e-3
    torch.testing.assert_close(tail.cpu(), ref_tail, atol=0, rtol=0)


@pytest.mark.parametrize("key_heads,value_heads", [(1, 3), (1, 4), (2, 6)])
def test_value_head_groups_of_three_and_four_match_oracle(key_heads, value_heads) -> None:
    # value heads j and j + 1 of one key head share its q/k rows; groups larger than the two of
    # the baseline configurations map workgroups to key heads through the same division
    shape = gd.LinearShape(key_heads=key_heads, value_heads=value_heads, key_head_dim=128, value_head_dim=128, conv_kernel_dim=4)
    mixed, a, b, a_log, dt_bias, w = _inputs(47 + value_heads, 1, 130, shape, a_log_scale=0.5)
    ref_core, ref_state, ref_tail = gd.linear_attention_core(mixed.float(), a, b, a_log, dt_bias, w, shape)
    out, state, tail = _run(mixed, a, b, a_log, dt_bias, w, shape, out_dtype=torch.float32)
    case = f"heads {key_heads}/{value_heads}"
    torch.testing.assert_close(out.cpu(), ref_core, atol=2e-2, rtol=2e-2, msg=lambda m: f"{case}: {m}")
    assert _rel(state, ref_state) < 1e-3, case
    torch.testing.assert_close(tail.cpu(), ref_tail, atol=0, rtol=0, msg=lambda m: f"{case}: {m}")


def test_chunked_prefill_with_initial_and_conv_state_fp32_out() -> None:
    mixed, a, b, a_log, dt_bias, w = _inputs(42, 1, 200, SHAPE, a_log_scale=0.5)
    gen = torch.Generator().manual_seed(43)
    state0 = torch.randn(1, SHAPE.value_heads, 128, 128, generator=gen) * 0.1
    tail0 = torch.randn(1, SHAPE.qkv_dim, 3, generator=gen)
    ref_core, ref_state, ref_tail = gd.linear_attention_core(mixed.float(), a, b, a_log, dt_bias, w, SHAPE, conv_tail=tail0, initial_state=state0)
    out, state, tail = _run(mixed, a, b, a_log, dt_bias, w, SHAPE, conv_state=tail0, state=state0, out_dtype=torch.float32)
    assert _rel(out, ref_core) < 2e-3
    assert _rel(state, ref_state) < 1e-3
    torch.testing.assert_close(tail.cpu(), ref_tail, atol=0, rtol=0)


def test_chunked_prefill_weak_decay_long_memory_state_precision() -> None:
    # A_log = -5: g ~ -0.005 per token, the state integrates ~200 tokens
    mixed, a, b, a_log, dt_bias, w = _inputs(44, 1, 640, SHAPE, a_log_shift=-5.0)
    ref_core, ref_state, _ = gd.linear_attention_core(mixed.float(), a, b, a_log, dt_bias, w, SHAPE)
    out, state, _ = _run(mixed, a, b, a_log, dt_bias, w, SHAPE, out_dtype=torch.float32)
    assert _rel(state, ref_state) < 1e-3
    assert _rel(out, ref_core) < 5e-3


def test_chunked_prefill_strong_and_mixed_decay_matches_oracle() -> None:
    # Heads with A_log up to ~+4 (g down to ~-50 per token, so in-chunk decays exp(G_i - G_l)
    # span far beyond the fp32 range of exp(-G_l) alone) beside weakly decaying heads, and a run
    # of tokens with large a inside otherwise moderate chunks, in one sequence and one launch.
    mixed, a, b, a_log, dt_bias, w = _inputs(45, 2, 300, SHAPE, a_log_scale=2.0)
    a[:, 100:140] += 8.0
    a_log[0] = 3.5
    ref_core, ref_state, _ = gd.linear_attention_core(mixed.float(), a, b, a_log, dt_bias, w, SHAPE)
    out, state, _ = _run(mixed, a, b, a_log, dt_bias, w, SHAPE, out_dtype=torch.float32)
    assert _rel(state, ref_state) < 1e-3
    assert _rel(out, ref_core) < 5e-3
    torch.testing.assert_close(out.cpu(), ref_core, atol=2e-2, rtol=2e-2)


def test_prefill_then_decode_equals_longer_prefill() -> None:
    import hip_ops

    shape = SHAPE
    total, first = 96, 70
    mixed, a, b, a_log, dt_bias, w = _inputs(45, 2, total, shape, a_log_scale=0.5)
    full_out, full_state, _ = _run(mixed, a, b, a_log, dt_bias, w, shape, out_dtype=torch.float32)
    out1, state, tail = _run(mixed[:, :first], a[:, :first], b[:, :first], a_log, dt_bias, w, shape, out_dtype=torch.float32)
    state = state.contiguous()
    outs = [out1.cpu()]
    for step in range(first, total):
        act = hip_ops.causal_conv1d_update(mixed[:, step].contiguous().to(DEV), tail, w.to(DEV))
        o = hip_ops.gated_delta_step(act, a[:, step].contiguous().to(DEV), b[:, step].contiguous().to(DEV), a_log.to(DEV), dt_bias.to(DEV), state,
                                     key_heads=shape.key_heads, out_dtype=torch.float32)
        outs.append(o.unsqueeze(1).cpu())
    stitched = torch.cat(outs, dim=1)
    assert _rel(stitched, full_out) < 2e-3
    assert _rel(state, full_state) < 1e-3


def test_chunked_prefill_matches_recurrent_core_kernel() -> None:
    """Chunked (MFMA) == token-serial (fp32) on the same prepared inputs."""
    import hip_ops

    shape = gd.LinearShape(key_heads=1, value_heads=2, key_head_dim=128, value_head_dim=128, conv_kernel_dim=4)
    mixed, a, b, a_log, dt_bias, w = _inputs(46, 1, 256, shape, a_log_scale=1.0)
    out, state, _ = _run(mixed, a, b, a_log, dt_bias, w, shape, out_dtype=torch.float32)
    conv, _ = gd.causal_conv1d(mixed.float().transpose(1, 2), w, None)
    conv = conv.transpose(1, 2)
    q = conv[..., :128].reshape(1, 256, 1, 128).repeat_interleave(2, dim=2)
    k = conv[..., 128:256].reshape(1, 256, 1, 128).repeat_interleave(2, dim=2)
    v = conv[..., 256:].reshape(1, 256, 2, 128)
    g, beta = gd.gating(a, b, a_log, dt_bias)
    pq, pk, pv, pg, pb, ps = gd.prepare_inputs(q, k, v, g, beta, None)
    rec_out, rec_state = hip_ops.linear_attention_recurrent_core(*(x.to(DEV) for x in (pq, pk, pv, pg, pb, ps)))
    assert _rel(out.transpose(1, 2), rec_out) < 2e-3
    assert _rel(state, rec_state) < 1e-3


def test_gate_inputs_on_the_host_are_rejected() -> None:
    import hip_ops

    mixed, a, b, a_log, dt_bias, w = _inputs(46, 1, 64, SHAPE)
    with pytest.raises(RuntimeError, match="a must be CUDA"):
        hip_ops.chunk_gated_delta_rule(mixed.to(DEV), a, b.to(DEV), a_log.to(DEV), dt_bias.to(DEV), w.to(DEV),
                                       key_heads=SHAPE.key_heads, value_heads=SHAPE.value_heads)
    with pytest.raises(RuntimeError, match="b must be CUDA"):
        hip_ops.chunk_gated_delta_rule(mixed.to(DEV), a.to(DEV), b, a_log.to(DEV), dt_bias.to(DEV), w.to(DEV),
                                       key_heads=SHAPE.key_heads, value_heads=SHAPE.value_heads)
