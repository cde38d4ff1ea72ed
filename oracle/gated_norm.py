"""Oracle: the gated RMSNorm + SiLU(z) output stage of a linear-attention layer, restated from
the reference's CPU code.

* ``gated_rms_norm`` (``src/reference_ops.py:172-178``): fp32 mean of squares over the head's
  ``value_head_dim`` elements, ``rsqrt(var + eps)``, the normalised value cast back to the input
  dtype, then ``weight.float() *`` that (plain ``w``, unlike the ``1 + w`` of ``rms_norm``) times
  ``silu(z.float())`` in fp32, cast to the input dtype;
* its use after the recurrent core (``src/reference_ops.py:284-287``, ``src/tp_runtime.py:853-857``):
  the core and ``z = in_proj_z(hidden)`` both reshaped to ``(tokens * value_heads, value_head_dim)``.

Floating-point work uses PyTorch CPU in the reference's own cast order.

Pinning (``tests/test_oracle_gated_norm.py``): :func:`gated_rms_norm_fp64` (the textbook formula in
float64) agrees with the bf16 restatement to bf16 rounding; the output is invariant to a positive
scale of ``x`` (up to the bf16 rounding of the normalised value), is zero for ``z = 0`` or
``w = 0``, is odd in ``x``, and for large ``z`` tends to ``w * x / rms(x) * z``; and
``tests/test_golden.py`` matches it bit for bit with vectors the reference's own
``linear_attention`` wrote with a non-zero ``z`` and norm weight
(``tests/golden/linear_attention_output.npz``, ``tests/golden/make_golden.py``).

Test infrastructure only: the product path never imports this module.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F


def gated_rms_norm(hidden: torch.Tensor, weight: torch.Tensor, gate: torch.Tensor, eps: float) -> torch.Tensor:
    """``gated_rms_norm`` (``src/reference_ops.py:172-178``) over the last axis."""
    variance = hidden.float().pow(2).mean(dim=-1, keepdim=True)
    normalized = hidden.float() * variance.add(eps).rsqrt()
    out = weight.float() * normalized.to(hidden.dtype)
    return (out * F.silu(gate.float())).to(hidden.dtype)


def linear_attention_output(core: torch.Tensor, z: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """The output stage of ``linear_attention`` (``src/reference_ops.py:284-287``): ``core``
    ``(..., value_heads, value_head_dim)`` and ``z`` ``(..., value_heads * value_head_dim)`` to
    ``(..., value_heads * value_head_dim)``."""
    dv = core.shape[-1]
    flat = gated_rms_norm(core.reshape(-1, dv), weight, z.reshape(-1, dv), eps)
    return flat.reshape(*core.shape[:-2], core.shape[-2] * dv)


def gated_rms_norm_fp64(x: np.ndarray, weight: np.ndarray, gate: np.ndarray, eps: float) -> np.ndarray:
    """Textbook gated RMSNorm in float64: ``w * x / sqrt(mean(x^2) + eps) * z * sigmoid(z)``."""
    x = x.astype(np.float64)
    z = gate.astype(np.float64)
    rms = np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps)
    return weight.astype(np.float64) * (x / rms) * (z / (1.0 + np.exp(-z)))
