"""Oracle: the prologue of a full-attention layer -- q/k RMSNorm with the (1 + w)
weight and the partial rotary embedding -- restated from the reference's CPU code.

* ``rms_norm`` (``src/reference_ops.py:166-169``): fp32 mean of squares, ``rsqrt(var + eps)``,
  times ``1 + weight`` in fp32, cast back to the activation dtype;
* ``rotary_embeddings`` (``src/reference_ops.py:203-213``): ``rotary_dim = int(D * factor)``,
  ``inv_freq = 1 / theta ** (arange(0, rd, 2) / rd)`` in fp32, angles ``pos * inv_freq``
  duplicated over the two halves, cos/sin cast to the activation dtype;
* ``apply_rotary_pos_emb`` / ``_rotate_half`` / ``_cat_last`` (``src/reference_ops.py:216-224,
  422-433``): ``x_rot * cos + rotate_half(x_rot) * sin`` on the first ``rd`` elements in the
  activation dtype, the rest passed through;
* the order of the full-attention layer (``src/reference_ops.py:343-347``,
  ``src/tp_runtime.py:511-520``): norm q and k, then rotate both at the token positions.

Floating-point work uses PyTorch CPU in the reference's own cast order, on the packed
``(tokens, heads, head_dim)`` layout (per-token positions broadcast over heads exactly as the
reference's ``cos.unsqueeze(1)`` does over its head axis).

Pinning (``tests/test_oracle_rope.py``): :func:`rope_textbook_fp64` (each pair ``(j, j + rd/2)``
as a complex number times ``exp(i pos inv_freq_j)``, in float64) and :func:`rms_norm_fp64`
agree with the bf16 restatement to bf16 rounding; position 0 is the identity; a rotation keeps
the norm of every pair; rotating by ``p1`` then ``p2`` equals rotating by ``p1 + p2`` (fp64);
and ``tests/test_golden.py`` matches q and k bit for bit with vectors written by the
reference's own ``full_attention`` (``tests/golden/make_golden.py``).

Test infrastructure only: the product path never imports this module.
"""

from __future__ import annotations

import numpy as np
import torch


def rms_norm(hidden: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """``rms_norm`` (``src/reference_ops.py:166-169``)."""
    variance = hidden.float().pow(2).mean(dim=-1, keepdim=True)
    normalized = hidden.float() * variance.add(eps).rsqrt()
    return (normalized * (1.0 + weight.float())).to(hidden.dtype)


def inv_freq(rotary_dim: int, rope_theta: float) -> torch.Tensor:
    """The ``inv_freq`` of ``rotary_embeddings`` (``src/reference_ops.py:207-209``), fp32."""
    return 1.0 / (rope_theta ** (torch.arange(0, rotary_dim, 2, dtype=torch.float32) / rotary_dim))


def rotary_cos_sin(positions: torch.Tensor, rotary_dim: int, rope_theta: float, dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
    """``rotary_embeddings`` (``src/reference_ops.py:203-213``) for a 1-D tensor of positions:
    ``(tokens, rotary_dim)`` cos and sin in ``dtype``."""
    freqs = torch.outer(positions.to(torch.float32).reshape(-1), inv_freq(rotary_dim, rope_theta))
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype=dtype), emb.sin().to(dtype=dtype)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """``_rotate_half`` (``src/reference_ops.py:422-427``)."""
    first = x[..., : x.shape[-1] // 2]
    second = x[..., x.shape[-1] // 2 :]
    return torch.cat((-second, first), dim=-1)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """One operand of ``apply_rotary_pos_emb`` (``src/reference_ops.py:216-224``) on
    ``(tokens, heads, D)`` with ``(tokens, rd)`` cos/sin."""
    cos = cos.unsqueeze(1)
    sin = sin.unsqueeze(1)
    rd = cos.shape[-1]
    x_rot, x_pass = x[..., :rd], x[..., rd:]
    return torch.cat((x_rot * cos + rotate_half(x_rot) * sin, x_pass), dim=-1)


def qk_norm_rope(
    q: torch.Tensor,
    k: torch.Tensor,
    q_weight: torch.Tensor,
    k_weight: torch.Tensor,
    positions: torch.Tensor,
    *,
    eps: float,
    rope_theta: float,
    partial_rotary_factor: float,
) -> tuple[torch.Tensor, torch.Tensor]:
    """q ``(tokens, H, D)`` and k ``(tokens, H_kv, D)`` after the reference's norm and rotation."""
    head_dim = q.shape[-1]
    rotary_dim = int(head_dim * partial_rotary_factor)
    qn = rms_norm(q, q_weight, eps)
    kn = rms_norm(k, k_weight, eps)
    cos, sin = rotary_cos_sin(positions, rotary_dim, rope_theta, q.dtype)
    return apply_rope(qn, cos, sin), apply_rope(kn, cos, sin)


def rms_norm_fp64(x: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    """Textbook RMSNorm with the (1 + w) weight over the last axis, float64."""
    x = x.astype(np.float64)
    return x / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps) * (1.0 + weight.astype(np.float64))


def rope_textbook_fp64(x: np.ndarray, positions: np.ndarray, rotary_dim: int, rope_theta: float) -> np.ndarray:
    """``(tokens, heads, D)`` rotated in float64: pair ``(j, j + rd/2)`` of the first ``rd``
    elements is the complex number ``x_j + i x_{j+rd/2}`` multiplied by
    ``exp(i pos theta^(-2j/rd))``; the other elements are unchanged."""
    x = x.astype(np.float64).copy()
    half = rotary_dim // 2
    if half == 0:
        return x
    freq = rope_theta ** (-(2.0 * np.arange(half)) / rotary_dim)
    ang = positions.astype(np.float64)[:, None] * freq[None, :]
    z = (x[..., :half] + 1j * x[..., half:rotary_dim]) * np.exp(1j * ang)[:, None, :]
    x[..., :half] = z.real
    x[..., half:rotary_dim] = z.imag
    return x
