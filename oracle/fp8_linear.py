"""Oracle: block-scaled fp8 E4M3 linear layer (test infrastructure only).

Restates the reference's ``linear`` for an fp8 weight with a bf16 ``scale_inv``
(``src/reference_ops.py:436-497``): ``F.linear(x.float(), dequantize_fp8_weight(w,
scale_inv))`` in fp32, with ``dequantize_fp8_weight`` (``:500-506``) expanding each
scale over its 128 x 128 block.  The E4M3 decode follows the reference's native
table (``src/csrc/fp8_linear_cuda.cu:66-77``: ``exp == 0`` -> ``mant/8 * 2^-6``,
else ``(1 + mant/8) * 2^(exp-7)``) except for codes 0x7F / 0xFF, which torch's
``float8_e4m3fn`` -- the arithmetic of the reference's CPU path -- decodes as NaN
where that native table gives +-480.

Pinning (``tests/test_oracle_fp8_linear.py``): the decode of all 256 codes against
torch's own ``float8_e4m3fn`` conversion and against the OCP E4M3 closed form
(largest finite 448, smallest subnormal 2^-9, round trip of every finite code);
the dequantisation against a per-element loop; the linear layer against a float64
sum and against the reference test's case (``tests/unit/test_fp8_cuda.py:10-24``:
seed 0, 384 x 256 weights from ``randn * 0.05``, scale 0.25, batches 3 and 17).
"""

from __future__ import annotations

import math

import numpy as np
import torch

BLOCK = 128


def e4m3_value(code: int) -> float:
    """Value of one E4M3 (fn) code (``src/csrc/fp8_linear_cuda.cu:66-77``; NaN codes as torch)."""
    sign = -1.0 if (code >> 7) & 1 else 1.0
    exp = (code >> 3) & 0xF
    mant = code & 0x7
    if exp == 0xF and mant == 0x7:
        return math.nan
    if exp == 0:
        return sign * math.ldexp(mant / 8.0, -6)
    return sign * math.ldexp(1.0 + mant / 8.0, exp - 7)


def e4m3_table() -> np.ndarray:
    return np.array([e4m3_value(c) for c in range(256)], dtype=np.float32)


def dequantize(weight_codes: np.ndarray, scale: torch.Tensor) -> torch.Tensor:
    """fp32 ``(N, K)`` weight from uint8 codes and a bf16 ``(ceil(N/128), ceil(K/128))`` scale
    (``src/reference_ops.py:500-506``)."""
    rows, cols = weight_codes.shape
    values = torch.from_numpy(e4m3_table()[weight_codes.astype(np.int64)])
    expanded = scale.float().repeat_interleave(BLOCK, dim=0).repeat_interleave(BLOCK, dim=1)
    return values * expanded[:rows, :cols]


def linear(x: torch.Tensor, weight_codes: np.ndarray, scale: torch.Tensor) -> torch.Tensor:
    """``F.linear(x.float(), dequantize(w, scale))`` -- fp32 output (``src/reference_ops.py:497``)."""
    return torch.nn.functional.linear(x.float(), dequantize(weight_codes, scale))


def linear_fp64(x: torch.Tensor, weight_codes: np.ndarray, scale: torch.Tensor) -> torch.Tensor:
    return x.double() @ dequantize(weight_codes, scale).double().t()
