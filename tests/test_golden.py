"""The oracle against vectors written by the reference's own CPU code.

``tests/golden/make_golden.py`` ran ``recurrent_gated_delta_rule``,
``linear_attention`` and ``full_attention`` of ``src/reference_ops.py`` on small
seeded inputs.  These are the checks that pin the bf16 rounding of the
reference's cast points (``src/reference_ops.py:319``, ``:358-359``), which the
closed forms and invariants of ``test_oracle_*.py`` leave open.

Tolerances: the recurrence and the layer core are the same torch CPU operations
in the same order, so they must agree to fp32 rounding (1e-6); bf16 outputs must
be bit-identical except where a product's fp32 accumulation order differs, where
one bf16 ulp (2^-7 relative) is allowed.
"""

from __future__ import annotations

import torch

from golden_io import bf16, f32, load
from oracle import attention as oa
from oracle import gated_delta as gd
from oracle import gated_norm as gn


def _ulp_close(out: torch.Tensor, ref: torch.Tensor) -> None:
    out = out.float()
    ref = ref.float()
    torch.testing.assert_close(out, ref, atol=1e-3, rtol=2.0**-7)


def test_recurrent_rule_bf16_output_cast_matches_reference() -> None:
    for name in ("recurrent_rule_bf16", "recurrent_rule_bf16_state"):
        v = load(name)
        init = f32(v["initial_state"]) if "initial_state" in v else None
        out, state = gd.recurrent_gated_delta_rule(bf16(v["q_bf16"]), bf16(v["k_bf16"]), bf16(v["v_bf16"]), f32(v["g"]), f32(v["beta"]),
                                                   initial_state=init)
        assert out.dtype == torch.bfloat16
        torch.testing.assert_close(out, bf16(v["out_bf16"]), atol=0, rtol=0)
        torch.testing.assert_close(state, f32(v["state"]), atol=1e-6, rtol=1e-6)


def test_linear_attention_core_matches_reference_layer() -> None:
    v = load("linear_attention_core")
    batch, seq, hk, hv, dk, dv, kernel = (int(x) for x in v["shape"])
    shape = gd.LinearShape(key_heads=hk, value_heads=hv, key_head_dim=dk, value_head_dim=dv, conv_kernel_dim=kernel)
    w = f32(v["conv_weight"]).reshape(-1, 1, kernel)
    core, state, _tail = gd.linear_attention_core(bf16(v["mixed_qkv_bf16"]).float(), bf16(v["a_bf16"]), bf16(v["b_bf16"]), f32(v["a_log"]),
                                                  f32(v["dt_bias"]), w, shape)
    torch.testing.assert_close(core.float(), f32(v["core"]), atol=1e-6, rtol=1e-5)
    torch.testing.assert_close(state, f32(v["state"]), atol=1e-6, rtol=1e-5)


def test_full_attention_probs_cast_matches_reference() -> None:
    v = load("full_attention_prefill")
    batch, seq, heads, kv_heads, dim = (int(x) for x in v["shape"])
    q = bf16(v["q_bf16"])                                 # (1, H, S, D)
    k = bf16(v["k_bf16"])                                 # (1, H_kv, S, D)
    val = bf16(v["v_bf16"]).transpose(1, 2).contiguous()  # (1, H_kv, S, D)
    gate = bf16(v["gate_bf16"]).reshape(batch, seq, heads * dim)
    out = oa.dense_attention(q, k, val, position_offset=0, gate=gate)
    _ulp_close(out.transpose(1, 2), bf16(v["out_bf16"]))


def _prologue_inputs(v: dict) -> tuple:
    batch, seq, heads, kv_heads, head_dim = (int(x) for x in v["shape"])
    theta, factor, eps, offset = (float(x) for x in v["rope"])
    q_proj = bf16(v["q_proj_bf16"]).reshape(batch * seq, heads, 2 * head_dim)
    k_proj = bf16(v["k_proj_bf16"]).reshape(batch * seq, kv_heads, head_dim)
    positions = torch.arange(int(offset), int(offset) + seq).repeat(batch)
    return q_proj, k_proj, bf16(v["q_norm_bf16"]), bf16(v["k_norm_bf16"]), positions, theta, factor, eps, (batch, seq, heads, kv_heads, head_dim)


def test_qk_norm_rope_matches_reference_bit_for_bit() -> None:
    from oracle import rope

    for name in ("full_attention_prefill", "full_attention_rope_d256"):
        v = load(name)
        q_proj, k_proj, qw, kw, positions, theta, factor, eps, (batch, seq, heads, kv_heads, head_dim) = _prologue_inputs(v)
        q, k = rope.qk_norm_rope(q_proj[..., :head_dim], k_proj, qw, kw, positions, eps=eps, rope_theta=theta, partial_rotary_factor=factor)
        # the fixture holds the reference's (B, H, S, D) q and (B, H_kv, S, D) k after RMSNorm and rotation
        q_ref = bf16(v["q_bf16"]).permute(0, 2, 1, 3).reshape(batch * seq, heads, head_dim)
        k_ref = bf16(v["k_bf16"]).permute(0, 2, 1, 3).reshape(batch * seq, kv_heads, head_dim)
        torch.testing.assert_close(q, q_ref, atol=0, rtol=0)
        torch.testing.assert_close(k, k_ref, atol=0, rtol=0)


def test_gated_rms_norm_matches_reference_layer_call() -> None:
    """``gated_rms_norm`` as ``linear_attention`` calls it: an fp32 core (its mid cast is the
    identity), bf16 ``z`` and weight; same torch CPU operations, so bit for bit in fp32, and the
    layer's bf16 output (identity ``out_proj``) is that result cast to bf16."""
    v = load("linear_attention_output")
    x, gate, norm = f32(v["x"]), bf16(v["gate_bf16"]), bf16(v["norm_bf16"])
    out = gn.gated_rms_norm(x, norm, gate, float(v["eps"][0]))
    assert out.dtype == torch.float32
    assert torch.equal(out, f32(v["out"]))
    batch, seq, _kh, value_heads, _dk, dv, _k = (int(t) for t in v["shape"])
    layer = bf16(v["layer_out_bf16"])
    assert torch.equal(layer, out.reshape(batch, seq, value_heads * dv).to(torch.bfloat16))
