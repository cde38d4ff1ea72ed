"""``hip_ops.gated_rms_norm`` (the linear-attention output stage: gated RMSNorm + SiLU(z)) on
the GPU against ``oracle/gated_norm.py`` and against what the reference's ``gated_rms_norm``
returned inside its ``linear_attention`` layer.

Tolerances: fp32 outputs within 1e-5 relative of the largest value (the order of the
mean-of-squares sum and libm's exp differ by an ulp or so); bf16 outputs within 2e-2 absolute
and relative, with at least 99% of the elements bit-identical (a rounding moves only where those
ulps cross a bf16 rounding boundary).
"""

from __future__ import annotations

import pytest
import torch

from golden_io import bf16, f32, load
from oracle import gated_norm as gn

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
EPS = 1e-6


def _mostly_bit_exact(out: torch.Tensor, ref: torch.Tensor) -> None:
    out = out.cpu()
    assert out.dtype == ref.dtype == torch.bfloat16
    torch.testing.assert_close(out.float(), ref.float(), atol=2e-2, rtol=2e-2)
    same = (out.view(torch.int16) == ref.view(torch.int16)).float().mean().item()
    assert same >= 0.99, f"only {same:.4f} of the elements are bit-identical"


def _fp32_close(out: torch.Tensor, ref: torch.Tensor) -> None:
    out = out.cpu().float()
    torch.testing.assert_close(out, ref.float(), atol=1e-5 * float(ref.abs().max()), rtol=1e-5)


def test_matches_reference_layer_call() -> None:
    import hip_ops

    v = load("linear_attention_output")
    batch, seq, _kh, heads, _dk, dv, _k = (int(t) for t in v["shape"])
    x = f32(v["x"]).reshape(batch, seq, heads, dv)
    gate = bf16(v["gate_bf16"]).reshape(batch, seq, heads * dv)
    norm = bf16(v["norm_bf16"])
    eps = float(v["eps"][0])
    out = hip_ops.gated_rms_norm(x.to(DEV), gate.to(DEV), norm.to(DEV), eps)
    assert out.dtype == torch.float32 and out.shape == (batch, seq, heads * dv)
    _fp32_close(out.reshape(-1, dv), f32(v["out"]))
    layer = hip_ops.gated_rms_norm(x.to(DEV), gate.to(DEV), norm.to(DEV), eps, out_dtype=torch.bfloat16)
    _mostly_bit_exact(layer, bf16(v["layer_out_bf16"]))


@pytest.mark.parametrize("dim", [64, 128, 256])
@pytest.mark.parametrize("wdtype", [torch.bfloat16, torch.float32])
def test_bf16_core_matches_oracle(dim: int, wdtype: torch.dtype) -> None:
    """A bf16 core (what the chunked prefill kernel writes): the normalised value is rounded
    to bf16 before the weight, as the reference does for a bf16 input."""
    import hip_ops

    gen = torch.Generator().manual_seed(dim)
    tokens, heads = 37, 3
    core = (torch.randn(tokens, heads, dim, generator=gen) * 3.0).to(torch.bfloat16)
    z = (torch.randn(tokens, heads * dim, generator=gen) * 2.0).to(torch.bfloat16)
    w = (1.0 + 0.2 * torch.randn(dim, generator=gen)).to(wdtype)
    out = hip_ops.gated_rms_norm(core.to(DEV), z.to(DEV), w.to(DEV), EPS)
    ref = gn.linear_attention_output(core, z, w, EPS)
    assert out.shape == ref.shape
    _mostly_bit_exact(out, ref)
    out32 = hip_ops.gated_rms_norm(core.to(DEV), z.to(DEV), w.to(DEV), EPS, out_dtype=torch.float32)
    ref32 = gn.linear_attention_output(core, z, w, EPS).float()
    torch.testing.assert_close(out32.cpu().to(torch.bfloat16).float(), ref32, atol=2e-2, rtol=2e-2)


def test_strided_views_and_fp32_gate() -> None:
    """core a head slice of a wider buffer, z a column slice of the fused projection output."""
    import hip_ops

    gen = torch.Generator().manual_seed(11)
    tokens, heads, dim = 29, 4, 128
    wide = torch.randn(tokens, heads + 2, dim, generator=gen) * 2.0
    core = wide[:, 1 : 1 + heads]  # token stride (heads + 2) * dim
    proj = torch.randn(tokens, heads * dim + 64, generator=gen)
    z = proj[:, 32 : 32 + heads * dim]  # token stride heads*dim + 64, starts 32 elements in
    w = torch.randn(dim, generator=gen)
    out = hip_ops.gated_rms_norm(core.to(DEV), z.to(DEV), w.to(DEV), EPS)
    ref = gn.linear_attention_output(core.contiguous(), z.contiguous(), w, EPS)
    _fp32_close(out, ref)


def test_chunked_prefill_output_stage_end_to_end() -> None:
    """core of the chunked delta-rule kernel (bf16) through the output stage equals the oracle's
    output stage on the same core."""
    import hip_ops

    gen = torch.Generator().manual_seed(5)
    batch, seq, hk, hv = 1, 70, 1, 2
    channels = 2 * hk * 128 + hv * 128
    mixed = torch.randn(batch, seq, channels, generator=gen).to(torch.bfloat16)
    a = torch.randn(batch, seq, hv, generator=gen).to(torch.bfloat16)
    b = torch.randn(batch, seq, hv, generator=gen).to(torch.bfloat16)
    a_log = torch.rand(hv, generator=gen) * 2.0 - 1.0
    dt_bias = torch.randn(hv, generator=gen) * 0.5
    conv_w = torch.randn(channels, 4, generator=gen) * 0.5
    z = (torch.randn(batch, seq, hv * 128, generator=gen) * 2.0).to(torch.bfloat16)
    norm = (1.0 + 0.2 * torch.randn(128, generator=gen)).to(torch.bfloat16)
    core, _state, _conv = hip_ops.chunk_gated_delta_rule(mixed.to(DEV), a.to(DEV), b.to(DEV), a_log.to(DEV), dt_bias.to(DEV), conv_w.to(DEV),
                                                         key_heads=hk, value_heads=hv)
    out = hip_ops.gated_rms_norm(core, z.to(DEV), norm.to(DEV), EPS)
    ref = gn.linear_attention_output(core.cpu(), z, norm, EPS)
    _mostly_bit_exact(out, ref)


def test_rejects_unsupported_shapes() -> None:
    import hip_ops

    z = torch.zeros(4, 96, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="head_dim"):
        hip_ops.gated_rms_norm(torch.zeros(4, 1, 96, device=DEV, dtype=torch.bfloat16), z, torch.ones(96, device=DEV), EPS)
    wide = torch.zeros(4, 2, 132, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="16-byte"):
        hip_ops.gated_rms_norm(wide[:, :, 2:130], torch.zeros(4, 256, device=DEV, dtype=torch.bfloat16), torch.ones(128, device=DEV), EPS)


def _decode_inputs(seed: int, batch: int, key_heads: int, value_heads: int):
    gen = torch.Generator().manual_seed(seed)
    channels = 2 * key_heads * 128 + value_heads * 128
    act = torch.randn(batch, channels, generator=gen)  # the conv + SiLU output of the step
    a = torch.randn(batch, value_heads, generator=gen)
    b = torch.randn(batch, value_heads, generator=gen)
    a_log = torch.rand(value_heads, generator=gen) * 2.0 - 1.0
    dt_bias = torch.randn(value_heads, generator=gen) * 0.5
    state = torch.randn(batch, value_heads, 128, 128, generator=gen) * 0.05
    z = (torch.randn(batch, value_heads * 128, generator=gen) * 2.0).to(torch.bfloat16)
    norm = (1.0 + 0.2 * torch.randn(128, generator=gen)).to(torch.bfloat16)
    return act, a, b, a_log, dt_bias, state, z, norm


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_decode_step_with_fused_output_stage(out_dtype: torch.dtype) -> None:
    """qa_gated_delta_step_norm = the plain step's fp32 core through the oracle's output stage
    (the core is fp32, as in the reference's layers); the state update is the plain step's."""
    import hip_ops

    act, a, b, a_log, dt_bias, state0, z, norm = _decode_inputs(21, 3, 2, 4)
    args = (act.to(DEV), a.to(DEV), b.to(DEV), a_log.to(DEV), dt_bias.to(DEV))
    s_plain = state0.to(DEV).clone()
    core = hip_ops.gated_delta_step(*args, s_plain, key_heads=2, out_dtype=torch.float32)
    s_fused = state0.to(DEV).clone()
    out = hip_ops.gated_delta_step(*args, s_fused, key_heads=2, out_dtype=out_dtype, z=z.to(DEV), norm_weight=norm.to(DEV), eps=EPS)
    assert torch.equal(s_fused, s_plain)
    ref = gn.gated_rms_norm(core.cpu().reshape(-1, 128), norm, z.reshape(-1, 128), EPS).reshape(3, 4, 128)
    if out_dtype == torch.float32:
        _fp32_close(out, ref)
    else:
        _mostly_bit_exact(out, ref.to(torch.bfloat16))


def test_runtime_decode_batch_output_stage_on_slots() -> None:
    """attention_runtime.linear_attention_decode_batch with z: slot-indexed states, fused stage."""
    import attention_runtime as rt
    from decode_state import LinearStatePool

    from oracle import gated_delta as gd

    shape = gd.LinearShape(key_heads=2, value_heads=4, key_head_dim=128, value_head_dim=128, conv_kernel_dim=4)
    gen = torch.Generator().manual_seed(23)
    batch = 3
    mixed = torch.randn(batch, shape.qkv_dim, generator=gen)
    a = torch.randn(batch, 4, generator=gen)
    b = torch.randn(batch, 4, generator=gen)
    a_log = torch.rand(4, generator=gen) * 2.0 - 1.0
    dt_bias = torch.randn(4, generator=gen) * 0.5
    conv_w = torch.randn(shape.qkv_dim, 4, generator=gen) * 0.5
    z = (torch.randn(batch, 4 * 128, generator=gen) * 2.0).to(torch.bfloat16)
    norm = (1.0 + 0.2 * torch.randn(128, generator=gen)).to(torch.bfloat16)
    cfg = rt.parse_attention_config({"text_config": {
        "linear_num_key_heads": 2, "linear_num_value_heads": 4, "linear_key_head_dim": 128, "linear_value_head_dim": 128,
        "linear_conv_kernel_dim": 4, "num_attention_heads": 2, "num_key_value_heads": 2, "head_dim": 4, "attn_output_gate": True}})
    slots = torch.tensor([2, 0, 3], device=DEV)
    pool_a = LinearStatePool(4, 4, 128, 128, shape.qkv_dim, 4, device=DEV)
    pool_b = LinearStatePool(4, 4, 128, 128, shape.qkv_dim, 4, device=DEV)
    core = rt.linear_attention_decode_batch(mixed.to(DEV), a.to(DEV), b.to(DEV), a_log.to(DEV), dt_bias.to(DEV), conv_w.to(DEV), pool_a, slots, cfg,
                                            out_dtype=torch.float32)
    out = rt.linear_attention_decode_batch(mixed.to(DEV), a.to(DEV), b.to(DEV), a_log.to(DEV), dt_bias.to(DEV), conv_w.to(DEV), pool_b, slots, cfg,
                                           out_dtype=torch.float32, z=z.to(DEV), norm_weight=norm.to(DEV), eps=EPS)
    assert torch.equal(pool_a.state, pool_b.state) and torch.equal(pool_a.conv, pool_b.conv)
    ref = gn.gated_rms_norm(core.cpu().reshape(-1, 128), norm, z.reshape(-1, 128), EPS).reshape(batch, 4, 128)
    _fp32_close(out, ref)
