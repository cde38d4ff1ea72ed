"""The fp8 linear oracle against torch's E4M3 decoding, the format's closed form and fp64."""

from __future__ import annotations

import math

import numpy as np
import torch

from oracle import fp8_linear


def test_e4m3_decode_matches_torch_for_all_codes() -> None:
    codes = torch.arange(256, dtype=torch.uint8)
    want = codes.view(torch.float8_e4m3fn).float().numpy()
    got = fp8_linear.e4m3_table()
    nan = np.isnan(want)
    assert nan.sum() == 2 and np.isnan(got[nan]).all()
    np.testing.assert_array_equal(got[~nan], want[~nan])


def test_e4m3_closed_form_landmarks() -> None:
    table = fp8_linear.e4m3_table()
    assert table[0x7E] == 448.0 and table[0xFE] == -448.0          # largest finite
    assert table[0x01] == 2.0**-9 and table[0x08] == 2.0**-6       # smallest subnormal, smallest normal
    assert table[0x38] == 1.0 and table[0x80] == 0.0 and math.copysign(1.0, table[0x80]) < 0
    finite = [c for c in range(256) if not math.isnan(table[c])]
    back = torch.from_numpy(table[finite]).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(back, np.array(finite, dtype=np.uint8))


def test_dequantize_matches_elementwise_loop() -> None:
    rng = np.random.default_rng(3)
    codes = rng.integers(0, 256, (200, 300)).astype(np.uint8)
    codes[codes & 0x7F == 0x7F] = 0x10
    scale = torch.from_numpy(rng.uniform(0.1, 2.0, (2, 3)).astype(np.float32)).to(torch.bfloat16)
    got = fp8_linear.dequantize(codes, scale).numpy()
    s = scale.float().numpy()
    for n, k in [(0, 0), (127, 127), (128, 0), (199, 299), (50, 256), (150, 130)]:
        assert got[n, k] == np.float32(fp8_linear.e4m3_value(int(codes[n, k])) * s[n // 128, k // 128])


def test_linear_matches_fp64_on_the_reference_test_case() -> None:
    # tests/unit/test_fp8_cuda.py:10-24 of the reference: seed 0, (384, 256) weights
    # randn * 0.05 cast to E4M3, scale 0.25 everywhere, batches 3 and 17.
    torch.manual_seed(0)
    weight = (torch.randn((384, 256), dtype=torch.float32) * 0.05).to(torch.float8_e4m3fn)
    codes = weight.view(torch.uint8).numpy()
    scale = torch.full((3, 2), 0.25, dtype=torch.bfloat16)
    np.testing.assert_array_equal(fp8_linear.dequantize(codes, scale).numpy(), (weight.float() * 0.25).numpy())
    for batch in (3, 17):
        x = torch.randn((batch, 256), dtype=torch.float32)
        out = fp8_linear.linear(x, codes, scale)
        assert out.dtype == torch.float32 and out.shape == (batch, 384)
        torch.testing.assert_close(out.double(), fp8_linear.linear_fp64(x, codes, scale), atol=1e-5, rtol=1e-5)
