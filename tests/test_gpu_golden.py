"""HIP kernels against vectors written by the reference's own CPU code (``tests/golden``).

Tolerances as everywhere: bf16 / fp32 outputs within 2e-2 absolute and relative,
fp32 recurrent states within 1e-3 relative (Frobenius).
"""

from __future__ import annotations

import pytest
import torch

from golden_io import bf16, f32, load
from oracle import gated_delta as gd

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _rel(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def test_chunked_prefill_matches_reference_linear_attention_layer() -> None:
    import hip_ops

    v = load("linear_attention_core")
    batch, seq, hk, hv, dk, dv, kernel = (int(x) for x in v["shape"])
    out, state, _tail = hip_ops.chunk_gated_delta_rule(
        bf16(v["mixed_qkv_bf16"]).to(DEV), bf16(v["a_bf16"]).to(DEV), bf16(v["b_bf16"]).to(DEV), f32(v["a_log"]).to(DEV),
        f32(v["dt_bias"]).to(DEV), f32(v["conv_weight"]).reshape(-1, 1, kernel).to(DEV), key_heads=hk, value_heads=hv,
        out_dtype=torch.float32,
    )
    torch.testing.assert_close(out.cpu(), f32(v["core"]), atol=2e-2, rtol=2e-2)
    assert _rel(state, f32(v["state"])) < 1e-3


@pytest.mark.parametrize("name", ["recurrent_rule_bf16", "recurrent_rule_bf16_state"])
def test_recurrent_core_matches_reference_rule_with_bf16_cast(name: str) -> None:
    import hip_ops

    v = load(name)
    init = f32(v["initial_state"]) if "initial_state" in v else None
    q, k, val, g, beta, s0 = gd.prepare_inputs(bf16(v["q_bf16"]), bf16(v["k_bf16"]), bf16(v["v_bf16"]), f32(v["g"]), f32(v["beta"]), init)
    out, state = hip_ops.linear_attention_recurrent_core(q.to(DEV), k.to(DEV), val.to(DEV), g.to(DEV), beta.to(DEV), s0.to(DEV))
    out_bf16 = out.transpose(1, 2).contiguous().to(torch.bfloat16).cpu()
    torch.testing.assert_close(out_bf16.float(), bf16(v["out_bf16"]).float(), atol=2e-2, rtol=2e-2)
    assert _rel(state, f32(v["state"])) < 1e-3


def test_paged_prefill_matches_reference_full_attention() -> None:
    import hip_ops

    v = load("full_attention_prefill")
    batch, seq, heads, kv_heads, dim = (int(x) for x in v["shape"])
    bs = 16
    nblk = (seq + bs - 1) // bs
    perm = [3, 0, 2][:nblk] if nblk <= 3 else list(range(nblk))
    pool_blocks = max(perm) + 1
    kp = torch.zeros(pool_blocks, kv_heads, bs, dim, dtype=torch.bfloat16)
    vp = torch.zeros(pool_blocks, kv_heads, bs, dim, dtype=torch.bfloat16)
    k = bf16(v["k_bf16"])[0]                   # (H_kv, S, D)
    val = bf16(v["v_bf16"])[0].transpose(0, 1)  # (H_kv, S, D)
    for t in range(seq):
        kp[perm[t // bs], :, t % bs] = k[:, t]
        vp[perm[t // bs], :, t % bs] = val[:, t]
    table = torch.tensor([perm], dtype=torch.int32)
    q = bf16(v["q_bf16"])[0].transpose(0, 1).contiguous()  # (S, H, D)
    gate = bf16(v["gate_bf16"]).reshape(seq, heads * dim)
    out = hip_ops.paged_attention_prefill(
        q.to(DEV), torch.tensor([0, seq], device=DEV, dtype=torch.int32), torch.tensor([0], device=DEV, dtype=torch.int32), kp.to(DEV),
        vp.to(DEV), table.to(DEV), bs, max_new=seq, gate=gate.to(DEV),
    )
    torch.testing.assert_close(out.cpu().float(), bf16(v["out_bf16"])[0].float(), atol=2e-2, rtol=2e-2)
