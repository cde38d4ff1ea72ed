"""Write the golden fixtures in this directory by running the reference's own CPU code.

Run in a container that has the reference checkout (it is not needed afterwards):

    python tests/golden/make_golden.py /root/reference

The checks of ``tests/test_oracle_*.py`` pin every oracle function except the exact
bf16 rounding of two cast points the reference leaves to torch's CPU kernels:

* ``out.to(initial_dtype)`` at the end of ``recurrent_gated_delta_rule``
  (``src/reference_ops.py:319``) for bf16 inputs (inside ``linear_attention``,
  ``src/reference_ops.py:227-288``, the inputs are fp32 conv outputs and the cast
  is the identity; that layer path is recorded too, as the end-to-end vector of
  the conv + gating + recurrence core);
* ``probs.to(query.dtype)`` before the value product of ``full_attention``
  (``src/reference_ops.py:358-359``);
* the dtypes at which ``linear_attention`` hands its core and ``z`` to ``gated_rms_norm``
  (``src/reference_ops.py:172-178,284-287``): the recorded inputs and output of that call
  fix which of its casts are identities in the layer (the core arrives in fp32).

For those, this script calls the reference functions themselves on small seeded
inputs and stores inputs and outputs as plain arrays (``.npz``, no pickles; bf16
tensors as their uint16 bit patterns).  The reference functions take projection
weights through a weights object; here that object returns fixed, seeded tensors
for the projections that feed the hot path and the identity for the output
projection, and the inputs of the attention product (q, k after RMSNorm and RoPE)
and the linear layer's recurrence output and state are recorded by wrapping the
reference's own module functions for the duration of the call.
"""

from __future__ import annotations

import sys
from pathlib import Path
from types import SimpleNamespace

import numpy as np
import torch

HERE = Path(__file__).resolve().parent


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


class _Weights:
    """Weights object of the reference's ``linear``/``tensor`` interface over a dict."""

    def __init__(self, linear_out: dict, tensors: dict) -> None:
        self.linear_out = linear_out
        self.tensors = tensors

    def linear(self, hidden, name):
        produce = self.linear_out[name]
        return produce(hidden)

    def tensor(self, name):
        return self.tensors[name]


def linear_attention_case(ro, seed: int, batch: int, seq: int, key_heads: int, value_heads: int) -> dict:
    """``linear_attention`` (cache=None) on seeded in_proj outputs; records the core and state."""
    g = torch.Generator().manual_seed(seed)
    dk = dv = 128
    kernel = 4
    qkv_dim = 2 * key_heads * dk + value_heads * dv
    mixed = torch.randn(batch, seq, qkv_dim, generator=g).to(torch.bfloat16)
    a = torch.randn(batch, seq, value_heads, generator=g).to(torch.bfloat16)
    b = torch.randn(batch, seq, value_heads, generator=g).to(torch.bfloat16)
    a_log = (torch.rand(value_heads, generator=g) * 2.0 - 1.0).float()
    dt_bias = (torch.randn(value_heads, generator=g) * 0.5).float()
    conv_w = (torch.randn(qkv_dim, 1, kernel, generator=g) * 0.5).float()
    cfg = SimpleNamespace(
        linear_attention=SimpleNamespace(
            key_heads=key_heads, value_heads=value_heads, key_head_dim=dk, value_head_dim=dv, conv_kernel_dim=kernel,
            value_state_dim=value_heads * dv,
        ),
        rms_norm_eps=1e-6,
    )
    mapping = SimpleNamespace(in_proj_qkv="qkv", in_proj_z="z", out_proj="out", in_proj_a="a", in_proj_b="b",
                              conv1d_weight="conv", a_log="a_log", dt_bias="dt_bias", norm="norm")
    weights = _Weights(
        {"qkv": lambda h: mixed, "a": lambda h: a, "b": lambda h: b, "z": lambda h: torch.zeros(batch, seq, value_heads * dv),
         "out": lambda h: h},
        {"conv": conv_w, "a_log": a_log, "dt_bias": dt_bias, "norm": torch.zeros(dv)},
    )
    seen = {}
    original = ro.recurrent_gated_delta_rule

    def recording(query, key, value, g_, beta, *, initial_state=None, return_state=False):
        out, state = original(query, key, value, g_, beta, initial_state=initial_state, return_state=True)
        seen["core"], seen["state"] = out, state
        return (out, state) if return_state else out

    ro.recurrent_gated_delta_rule = recording
    try:
        ro.linear_attention(torch.zeros(batch, seq, 8, dtype=torch.bfloat16), mapping, cfg, weights, cache=None)
    finally:
        ro.recurrent_gated_delta_rule = original
    return {
        "mixed_qkv_bf16": bits(mixed), "a_bf16": bits(a), "b_bf16": bits(b), "a_log": a_log.numpy(), "dt_bias": dt_bias.numpy(),
        "conv_weight": conv_w.reshape(qkv_dim, kernel).numpy(), "core": seen["core"].float().numpy(),
        "state": seen["state"].numpy().astype(np.float32),
        "shape": np.array([batch, seq, key_heads, value_heads, dk, dv, kernel], dtype=np.int64),
    }


def linear_attention_output_case(ro, seed: int, batch: int, seq: int, key_heads: int, value_heads: int) -> dict:
    """``linear_attention`` (cache=None) with a non-zero ``in_proj_z`` output and norm weight;
    records what its ``gated_rms_norm`` received and returned (the core reaches it in fp32)."""
    g = torch.Generator().manual_seed(seed)
    dk = dv = 128
    kernel = 4
    qkv_dim = 2 * key_heads * dk + value_heads * dv
    mixed = torch.randn(batch, seq, qkv_dim, generator=g).to(torch.bfloat16)
    a = torch.randn(batch, seq, value_heads, generator=g).to(torch.bfloat16)
    b = torch.randn(batch, seq, value_heads, generator=g).to(torch.bfloat16)
    z = (torch.randn(batch, seq, value_heads * dv, generator=g) * 2.0).to(torch.bfloat16)
    norm = (1.0 + 0.2 * torch.randn(dv, generator=g)).to(torch.bfloat16)
    a_log = (torch.rand(value_heads, generator=g) * 2.0 - 1.0).float()
    dt_bias = (torch.randn(value_heads, generator=g) * 0.5).float()
    conv_w = (torch.randn(qkv_dim, 1, kernel, generator=g) * 0.5).float()
    cfg = SimpleNamespace(
        linear_attention=SimpleNamespace(
            key_heads=key_heads, value_heads=value_heads, key_head_dim=dk, value_head_dim=dv, conv_kernel_dim=kernel,
            value_state_dim=value_heads * dv,
        ),
        rms_norm_eps=1e-6,
    )
    mapping = SimpleNamespace(in_proj_qkv="qkv", in_proj_z="z", out_proj="out", in_proj_a="a", in_proj_b="b",
                              conv1d_weight="conv", a_log="a_log", dt_bias="dt_bias", norm="norm")
    weights = _Weights(
        {"qkv": lambda h: mixed, "a": lambda h: a, "b": lambda h: b, "z": lambda h: z, "out": lambda h: h},
        {"conv": conv_w, "a_log": a_log, "dt_bias": dt_bias, "norm": norm},
    )
    seen = {}
    original = ro.gated_rms_norm

    def recording(hidden, weight, gate, eps):
        out = original(hidden, weight, gate, eps)
        seen["x"], seen["gate"], seen["out"], seen["eps"] = hidden, gate, out, eps
        return out

    ro.gated_rms_norm = recording
    try:
        layer_out = ro.linear_attention(torch.zeros(batch, seq, 8, dtype=torch.bfloat16), mapping, cfg, weights, cache=None)
    finally:
        ro.gated_rms_norm = original
    assert seen["x"].dtype == torch.float32 and seen["out"].dtype == torch.float32
    return {
        "x": seen["x"].numpy(), "gate_bf16": bits(seen["gate"]), "norm_bf16": bits(norm), "out": seen["out"].numpy(),
        "layer_out_bf16": bits(layer_out), "eps": np.array([seen["eps"]], dtype=np.float64),
        "shape": np.array([batch, seq, key_heads, value_heads, dk, dv, kernel], dtype=np.int64),
    }


def recurrent_rule_case(ro, seed: int, batch: int, seq: int, heads: int, dk: int, dv: int, with_state: bool) -> dict:
    """``recurrent_gated_delta_rule`` on bf16 q/k/v (output cast back to bf16)."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(batch, seq, heads, dk, generator=g).to(torch.bfloat16)
    k = torch.randn(batch, seq, heads, dk, generator=g).to(torch.bfloat16)
    v = torch.randn(batch, seq, heads, dv, generator=g).to(torch.bfloat16)
    gg = -torch.rand(batch, seq, heads, generator=g) * 0.5
    beta = torch.rand(batch, seq, heads, generator=g)
    s0 = torch.randn(batch, heads, dk, dv, generator=g) * 0.1 if with_state else None
    out, state = ro.recurrent_gated_delta_rule(q, k, v, gg, beta, initial_state=s0, return_state=True)
    case = {"q_bf16": bits(q), "k_bf16": bits(k), "v_bf16": bits(v), "g": gg.numpy(), "beta": beta.numpy(),
            "out_bf16": bits(out), "state": state.numpy().astype(np.float32)}
    if s0 is not None:
        case["initial_state"] = s0.numpy()
    return case


def full_attention_case(ro, seed: int, seq: int, heads: int, kv_heads: int, head_dim: int, position_offset: int = 0) -> dict:
    """``full_attention`` (no cache, positions ``position_offset + 0..seq-1``) on seeded q/k/v/gate
    projections; also records the projections, the norm weights and the rotary parameters, which
    pin the q/k RMSNorm + rotary prologue."""
    g = torch.Generator().manual_seed(seed)
    batch = 1
    q_proj = torch.randn(batch, seq, heads * head_dim * 2, generator=g).to(torch.bfloat16)
    k_proj = torch.randn(batch, seq, kv_heads * head_dim, generator=g).to(torch.bfloat16)
    v_proj = torch.randn(batch, seq, kv_heads * head_dim, generator=g).to(torch.bfloat16)
    q_norm = (torch.randn(head_dim, generator=g) * 0.1).to(torch.bfloat16)
    k_norm = (torch.randn(head_dim, generator=g) * 0.1).to(torch.bfloat16)
    cfg = SimpleNamespace(
        full_attention=SimpleNamespace(num_heads=heads, num_key_value_heads=kv_heads, head_dim=head_dim, attn_dim=heads * head_dim),
        rms_norm_eps=1e-6, rope_theta=10000000.0, partial_rotary_factor=0.25,
    )
    mapping = SimpleNamespace(q_proj="q", k_proj="k", v_proj="v", o_proj="o", q_norm="qn", k_norm="kn")
    weights = _Weights({"q": lambda h: q_proj, "k": lambda h: k_proj, "v": lambda h: v_proj, "o": lambda h: h},
                       {"qn": q_norm, "kn": k_norm})
    seen = {}
    original = ro.apply_rotary_pos_emb

    def recording(query, key, cos, sin):
        q, k = original(query, key, cos, sin)
        seen["q"], seen["k"] = q, k
        return q, k

    ro.apply_rotary_pos_emb = recording
    try:
        out = ro.full_attention(torch.zeros(batch, seq, 8, dtype=torch.bfloat16), mapping, cfg, weights, cache=None,
                                position_offset=position_offset)
    finally:
        ro.apply_rotary_pos_emb = original
    gate = q_proj.view(batch, seq, heads, head_dim * 2)[..., head_dim:]
    return {
        # q (B, H, S, D) and k (B, H_kv, S, D) after RMSNorm and RoPE; v (B, S, H_kv, D) as projected
        "q_bf16": bits(seen["q"]), "k_bf16": bits(seen["k"]), "v_bf16": bits(v_proj.view(batch, seq, kv_heads, head_dim)),
        "gate_bf16": bits(gate), "out_bf16": bits(out.view(batch, seq, heads, head_dim)),
        "shape": np.array([batch, seq, heads, kv_heads, head_dim], dtype=np.int64),
        "q_proj_bf16": bits(q_proj.view(batch, seq, heads, head_dim * 2)), "k_proj_bf16": bits(k_proj.view(batch, seq, kv_heads, head_dim)),
        "q_norm_bf16": bits(q_norm), "k_norm_bf16": bits(k_norm),
        "rope": np.array([cfg.rope_theta, cfg.partial_rotary_factor, cfg.rms_norm_eps, position_offset], dtype=np.float64),
    }


def main(reference_root: str) -> None:
    sys.path.insert(0, str(Path(reference_root) / "src"))
    import reference_ops as ro

    torch.set_num_threads(1)
    np.savez_compressed(HERE / "linear_attention_core.npz", **linear_attention_case(ro, 20240, 1, 40, 1, 2))
    np.savez_compressed(HERE / "full_attention_prefill.npz", **full_attention_case(ro, 20241, 20, 4, 2, 128))
    np.savez_compressed(HERE / "full_attention_rope_d256.npz", **full_attention_case(ro, 20244, 12, 4, 2, 256, position_offset=3000))
    np.savez_compressed(HERE / "linear_attention_output.npz", **linear_attention_output_case(ro, 20245, 2, 9, 1, 2))
    np.savez_compressed(HERE / "recurrent_rule_bf16.npz", **recurrent_rule_case(ro, 20242, 2, 7, 3, 16, 8, False))
    np.savez_compressed(HERE / "recurrent_rule_bf16_state.npz", **recurrent_rule_case(ro, 20243, 1, 5, 2, 16, 8, True))
    for f in sorted(HERE.glob("*.npz")):
        print(f.name, f.stat().st_size, "bytes")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
