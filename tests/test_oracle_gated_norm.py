"""Pins of ``oracle/gated_norm.py`` (gated RMSNorm + SiLU(z), the output stage of a
linear-attention layer) by mathematics that does not restate its formulas:

* a float64 textbook version (``w * x / rms(x) * z * sigmoid(z)``) agrees with the bf16
  restatement to bf16 rounding (a ``1 + w`` weight, a missing SiLU, a sigmoid in place of the
  SiLU or a wrong reduction axis breaks this);
* a positive scale of ``x`` leaves the output unchanged up to bf16 rounding, and a sign flip of
  ``x`` flips it exactly;
* ``z = 0`` and ``w = 0`` give exact zeros;
* for large ``z`` the SiLU is ``z`` itself, so the output is ``w * x / rms(x) * z``.

The bit patterns of the reference's cast points are pinned by ``test_golden.py``.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import gated_norm as gn

EPS = 1e-6


def _inputs(seed: int, rows: int = 33, dv: int = 128):
    gen = torch.Generator().manual_seed(seed)
    x = (torch.randn(rows, dv, generator=gen) * 3.0).to(torch.bfloat16)
    z = (torch.randn(rows, dv, generator=gen) * 2.0).to(torch.bfloat16)
    w = (1.0 + 0.2 * torch.randn(dv, generator=gen)).to(torch.bfloat16)
    return x, z, w


def test_matches_fp64_textbook() -> None:
    for dv in (64, 128, 256):
        x, z, w = _inputs(1, dv=dv)
        out = gn.gated_rms_norm(x, w, z, EPS)
        assert out.dtype == torch.bfloat16
        ref = gn.gated_rms_norm_fp64(x.float().numpy(), w.float().numpy(), z.float().numpy(), EPS)
        # two bf16 roundings (the normalised value and the output)
        torch.testing.assert_close(out.double(), torch.from_numpy(ref), atol=2.0**-6 * float(np.abs(ref).max()), rtol=2.0**-7)


def test_scale_and_sign() -> None:
    x, z, w = _inputs(2)
    base = gn.gated_rms_norm(x, w, z, 0.0)
    for c in (0.25, 8.0, 1024.0):  # powers of two keep x * c exact in bf16
        torch.testing.assert_close(gn.gated_rms_norm(x * c, w, z, 0.0).float(), base.float(), atol=1e-2, rtol=2.0**-7)
    assert torch.equal(gn.gated_rms_norm(-x, w, z, EPS), -gn.gated_rms_norm(x, w, z, EPS))


def test_zero_gate_and_zero_weight() -> None:
    x, z, w = _inputs(3)
    assert torch.count_nonzero(gn.gated_rms_norm(x, w, torch.zeros_like(z), EPS)) == 0
    assert torch.count_nonzero(gn.gated_rms_norm(x, torch.zeros_like(w), z, EPS)) == 0


def test_large_gate_is_linear_in_z() -> None:
    x, _, w = _inputs(4)
    z = torch.full_like(x, 40.0)  # sigmoid(40) == 1 in fp32
    out = gn.gated_rms_norm(x, w, z, EPS).double()
    xd = x.double()
    ref = w.double() * xd / torch.sqrt(xd.pow(2).mean(dim=-1, keepdim=True) + EPS) * 40.0
    torch.testing.assert_close(out, ref, atol=2.0**-6 * float(ref.abs().max()), rtol=2.0**-7)


def test_layer_output_reshape() -> None:
    gen = torch.Generator().manual_seed(5)
    core = torch.randn(2, 5, 3, 128, generator=gen).to(torch.bfloat16)
    z = torch.randn(2, 5, 3 * 128, generator=gen).to(torch.bfloat16)
    w = torch.randn(128, generator=gen).to(torch.bfloat16)
    out = gn.linear_attention_output(core, z, w, EPS)
    assert out.shape == (2, 5, 384)
    # head h of token (b, s) is the norm of core[b, s, h] with z[b, s, h*128:(h+1)*128]
    torch.testing.assert_close(out[1, 2, 128:256], gn.gated_rms_norm(core[1, 2, 1], w, z[1, 2, 128:256], EPS), atol=0, rtol=0)
