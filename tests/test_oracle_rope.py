"""Pins of ``oracle/rope.py`` (q/k RMSNorm with the (1 + w) weight and partial rotary
embedding) by mathematics that does not restate its formulas:

* an fp64 RMSNorm and an fp64 rotation written as complex multiplication of each
  (j, j + rd/2) pair agree with the bf16 restatement to bf16 rounding (a swapped half, a
  wrong sign of ``rotate_half`` or a wrong frequency index breaks this);
* position 0 is the identity and elements past ``rotary_dim`` pass through unchanged;
* a rotation keeps the norm of each pair, and rotating by p1 then p2 is rotating by p1 + p2
  (fp64, which pins the angle as position times frequency);
* a zero weight gives the plain RMS normalisation and the mean of squares of the output is 1.

The bit patterns of the reference's bf16 cast points are pinned by ``test_golden.py``.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import rope

THETA = 10_000_000.0
FACTOR = 0.25


def _bf16_close(out: torch.Tensor, ref: np.ndarray, rel: float = 2.0**-6) -> None:
    ref_t = torch.from_numpy(ref).float()
    torch.testing.assert_close(out.float(), ref_t, atol=rel * float(np.abs(ref).max()), rtol=rel)


def test_rms_norm_matches_fp64() -> None:
    gen = torch.Generator().manual_seed(1)
    x = torch.randn(7, 3, 256, generator=gen).to(torch.bfloat16)
    w = (torch.randn(256, generator=gen) * 0.2).to(torch.bfloat16)
    out = rope.rms_norm(x, w, 1e-6)
    assert out.dtype == torch.bfloat16
    _bf16_close(out, rope.rms_norm_fp64(x.float().numpy(), w.float().numpy(), 1e-6))
    # zero weight: unit mean square
    ms = rope.rms_norm(x.float(), torch.zeros(256), 1e-6).double().pow(2).mean(dim=-1)
    torch.testing.assert_close(ms, torch.ones_like(ms), atol=1e-5, rtol=0)


def test_rope_matches_complex_rotation_fp64() -> None:
    gen = torch.Generator().manual_seed(2)
    for head_dim in (128, 256):
        rd = int(head_dim * FACTOR)
        x = torch.randn(9, 4, head_dim, generator=gen).to(torch.bfloat16)
        pos = torch.tensor([0, 1, 2, 17, 100, 1023, 4096, 12287, 30000])
        cos, sin = rope.rotary_cos_sin(pos, rd, THETA, torch.bfloat16)
        out = rope.apply_rope(x, cos, sin)
        ref = rope.rope_textbook_fp64(x.float().numpy(), pos.numpy(), rd, THETA)
        _bf16_close(out, ref, rel=2.0**-5)
        # pass-through part is untouched, bit for bit
        assert torch.equal(out[..., rd:], x[..., rd:])


def test_rope_position_zero_is_identity() -> None:
    x = torch.randn(3, 2, 256).to(torch.bfloat16)
    cos, sin = rope.rotary_cos_sin(torch.zeros(3, dtype=torch.long), 64, THETA, torch.bfloat16)
    assert torch.equal(rope.apply_rope(x, cos, sin), x)


def test_rope_rotation_invariants_fp64() -> None:
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, 2, 256))
    rd, half = 64, 32
    p1 = np.array([3, 50, 700, 9000, 1])
    p2 = np.array([11, 1, 300, 2000, 65000])
    once = rope.rope_textbook_fp64(x, p1, rd, THETA)
    norm_in = x[..., :half] ** 2 + x[..., half:rd] ** 2
    norm_out = once[..., :half] ** 2 + once[..., half:rd] ** 2
    np.testing.assert_allclose(norm_out, norm_in, rtol=1e-12)
    twice = rope.rope_textbook_fp64(once, p2, rd, THETA)
    np.testing.assert_allclose(twice, rope.rope_textbook_fp64(x, p1 + p2, rd, THETA), rtol=1e-9, atol=1e-9)


def test_inv_freq_is_the_geometric_ladder() -> None:
    f = rope.inv_freq(64, THETA).double().numpy()
    np.testing.assert_allclose(f, THETA ** (-(2.0 * np.arange(32)) / 64), rtol=1e-6)
    assert f[0] == 1.0
