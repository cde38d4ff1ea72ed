"""fp8 E4M3 block-scaled linear (``hip_ops.fp8_e4m3_bf16_linear``) against the oracle.

Tolerances: weight decoding bit-exact; fp32 output within 1e-5 x max|y| absolute
and 1e-3 relative of the float64 sum for bf16 inputs and for fp32 inputs of
fewer than 16 rows (fp32 summation of up to 4096 terms); fp32 inputs of 16 rows or more are
rounded to fp16 as the reference's own GEMM path does
(``src/csrc/fp8_linear_cuda.cu:1411-1460``): within 1e-3 x max|y| and 1e-3
relative; everything within the reference's own 2e-3 of its fp32 restatement
(``tests/unit/test_fp8_cuda.py:24``); bf16 output within 2e-2.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import fp8_linear as oracle

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _ops():
    import hip_ops

    return hip_ops


def _weights(gen: torch.Generator, n: int, k: int, *, scale_range=(0.05, 2.0)) -> tuple[torch.Tensor, torch.Tensor]:
    w = (torch.randn((n, k), generator=gen) * 0.5).to(torch.float8_e4m3fn)
    lo, hi = scale_range
    s = (torch.rand((n // 128, k // 128), generator=gen) * (hi - lo) + lo).to(torch.bfloat16)
    return w, s


def _close_to_fp64(out: torch.Tensor, ref: torch.Tensor, *, fp16_input: bool = False) -> None:
    atol = (1e-3 if fp16_input else 1e-5) * ref.abs().max().item()
    torch.testing.assert_close(out.cpu().double(), ref, atol=atol, rtol=1e-3)


def test_every_finite_e4m3_code_decodes_exactly() -> None:
    ops = _ops()
    n, k = 256, 128
    nn, kk = np.meshgrid(np.arange(n), np.arange(k), indexing="ij")
    codes = ((nn + 7 * kk) % 256).astype(np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0  # NaN codes: checked separately
    x = torch.eye(k, dtype=torch.float32)  # y[m][n] = W[n][m]
    scale = torch.ones((n // 128, 1), dtype=torch.bfloat16)
    out = ops.fp8_e4m3_bf16_linear(x.to(DEV), torch.from_numpy(codes).to(DEV).view(torch.float8_e4m3fn), scale.to(DEV))
    want = torch.from_numpy(oracle.e4m3_table()[codes.astype(np.int64)]).t()
    assert torch.equal(out.cpu(), want)
    assert sorted(set(codes.ravel().tolist())) == [c for c in range(256) if (c & 0x7F) != 0x7F]


@pytest.mark.parametrize("rows", [2, 32])
def test_nan_code_gives_nan_like_the_reference_cpu_path(rows) -> None:
    ops = _ops()
    codes = torch.zeros((128, 128), dtype=torch.uint8)
    codes[5, 3] = 0x7F
    out = ops.fp8_e4m3_bf16_linear(torch.ones((rows, 128), device=DEV), codes.to(DEV), torch.ones((1, 1), dtype=torch.bfloat16, device=DEV))
    ref = oracle.linear(torch.ones((rows, 128)), codes.numpy(), torch.ones((1, 1), dtype=torch.bfloat16))
    assert torch.isnan(out[:, 5]).all().item() and torch.isnan(ref[:, 5]).all().item()
    assert (out.cpu()[:, torch.arange(128) != 5] == 0).all().item()


def test_matches_reference_test_case() -> None:
    # tests/unit/test_fp8_cuda.py:10-24 of the reference
    ops = _ops()
    torch.manual_seed(0)
    weight = (torch.randn((384, 256), dtype=torch.float32) * 0.05).to(torch.float8_e4m3fn)
    scale = torch.full((3, 2), 0.25, dtype=torch.bfloat16)
    codes = weight.view(torch.uint8).numpy()
    for batch in (3, 17):
        x = torch.randn((batch, 256), dtype=torch.float32)
        out = ops.fp8_e4m3_bf16_linear(x.to(DEV), weight.to(DEV), scale.to(DEV))
        assert out.dtype == torch.float32 and out.shape == (batch, 384)
        torch.testing.assert_close(out.cpu(), oracle.linear(x, codes, scale), atol=2e-3, rtol=2e-3)
        _close_to_fp64(out, oracle.linear_fp64(x, codes, scale), fp16_input=batch >= 16)


@pytest.mark.parametrize("rows,n,k", [(1, 256, 512), (37, 384, 1024), (48, 256, 640), (128, 1024, 2048), (128, 1024, 4096), (200, 512, 768), (256, 256, 2048), (4096, 256, 256)])
def test_fp32_input_matches_fp64(rows, n, k) -> None:
    ops = _ops()
    gen = torch.Generator().manual_seed(rows + n + k)
    w, s = _weights(gen, n, k)
    x = torch.randn((rows, k), generator=gen)
    print(f"fp8 linear fp32: rows {rows}, out {n}, in {k}, workspace {ops.L.load_library().qa_fp8_linear_workspace(rows, n, k)}", flush=True)
    out = ops.fp8_e4m3_bf16_linear(x.to(DEV), w.to(DEV), s.to(DEV))
    ref = oracle.linear_fp64(x, w.view(torch.uint8).numpy(), s)
    _close_to_fp64(out, ref, fp16_input=rows >= 16)


@pytest.mark.parametrize("rows", [15, 16])
def test_regime_boundary_at_16_rows(rows) -> None:
    """Below 16 rows fp32 x enters exactly; from 16 rows on it is rounded to fp16 first, as the
    reference's ``batch < kDefaultCublasBatchThreshold`` (16) split does
    (``src/csrc/fp8_linear_cuda.cu:1411-1460``).  Each side matches its own fp64 form at 1e-5 and
    not the other one's."""
    ops = _ops()
    gen = torch.Generator().manual_seed(160 + rows)
    w, s = _weights(gen, 256, 1024)
    x = torch.randn((rows, 1024), generator=gen) * 3.0
    codes = w.view(torch.uint8).numpy()
    out = ops.fp8_e4m3_bf16_linear(x.to(DEV), w.to(DEV), s.to(DEV)).cpu().double()
    exact = oracle.linear_fp64(x, codes, s)
    rounded = oracle.linear_fp64(x.half().float(), codes, s)
    want, other = (rounded, exact) if rows >= 16 else (exact, rounded)
    scale = want.abs().max().item()
    torch.testing.assert_close(out, want, atol=1e-5 * scale, rtol=1e-4)
    assert (out - other).abs().max().item() > 1e-4 * scale


def test_bf16_input_and_output_and_leading_dims() -> None:
    ops = _ops()
    gen = torch.Generator().manual_seed(9)
    w, s = _weights(gen, 640, 1536)
    x = torch.randn((2, 33, 1536), generator=gen).to(torch.bfloat16)
    codes = w.view(torch.uint8).numpy()
    out = ops.fp8_e4m3_bf16_linear(x.to(DEV), w.to(DEV), s.to(DEV))
    assert out.shape == (2, 33, 640) and out.dtype == torch.float32
    ref = oracle.linear_fp64(x.float().view(-1, 1536), codes, s).view(2, 33, 640)
    _close_to_fp64(out, ref)
    out16 = ops.fp8_e4m3_bf16_linear(x.to(DEV), w.to(DEV), s.to(DEV), out_dtype=torch.bfloat16)
    assert out16.dtype == torch.bfloat16
    torch.testing.assert_close(out16.cpu().float(), ref.float(), atol=2e-2, rtol=2e-2)


def test_split_k_is_deterministic() -> None:
    ops = _ops()
    gen = torch.Generator().manual_seed(11)
    w, s = _weights(gen, 512, 4096)
    x = torch.randn((16, 4096), generator=gen).to(DEV)
    assert ops.L.load_library().qa_fp8_linear_workspace(16, 512, 4096) > 0
    a = ops.fp8_e4m3_bf16_linear(x, w.to(DEV), s.to(DEV))
    b = ops.fp8_e4m3_bf16_linear(x, w.to(DEV), s.to(DEV))
    assert torch.equal(a, b)


def test_rejects_shapes_the_reference_rejects() -> None:
    ops = _ops()
    x = torch.zeros((2, 256), device=DEV)
    with pytest.raises(RuntimeError, match="weight rows must be divisible by 128"):
        ops.fp8_e4m3_bf16_linear(x, torch.zeros((200, 256), dtype=torch.uint8, device=DEV), torch.ones((2, 2), dtype=torch.bfloat16, device=DEV))
    with pytest.raises(RuntimeError, match="input last dim must match weight cols"):
        ops.fp8_e4m3_bf16_linear(x, torch.zeros((128, 384), dtype=torch.uint8, device=DEV), torch.ones((1, 3), dtype=torch.bfloat16, device=DEV))
    with pytest.raises(RuntimeError, match="scale must be bfloat16"):
        ops.fp8_e4m3_bf16_linear(x, torch.zeros((128, 256), dtype=torch.uint8, device=DEV), torch.ones((1, 2), device=DEV))


@pytest.mark.parametrize("rows,n,k,xdt", [(1, 256, 512, torch.float32), (37, 384, 1024, torch.float32), (128, 1024, 2048, torch.bfloat16), (128, 1024, 4096, torch.bfloat16)])
def test_packed_weight_layout_and_identical_results(rows, n, k, xdt) -> None:
    ops = _ops()
    gen = torch.Generator().manual_seed(rows * 7 + k)
    w, s = _weights(gen, n, k)
    x = torch.randn((rows, k), generator=gen).to(xdt).to(DEV)
    packed = ops.fp8_pack_weight(w.to(DEV))
    # byte (t, kb, h, l, e) of the packed form is w[16 t + l % 16][128 kb + 32 (l // 16) + 16 h + e]
    codes = w.view(torch.uint8).numpy()
    want = codes.reshape(n // 16, 16, k // 128, 4, 2, 16).transpose(0, 2, 4, 3, 1, 5).reshape(-1)
    np.testing.assert_array_equal(packed.data.cpu().numpy(), want)
    a = ops.fp8_e4m3_bf16_linear(x, packed, s.to(DEV))
    b = ops.fp8_e4m3_bf16_linear(x, w.to(DEV), s.to(DEV))
    assert torch.equal(a, b)


def test_runtime_linear_native_hits_the_kernel() -> None:
    from attention_runtime import LinearDispatchStats, linear_native

    ops = _ops()
    gen = torch.Generator().manual_seed(17)
    w, s = _weights(gen, 256, 384)
    x = torch.randn((2, 5, 384), generator=gen).to(torch.bfloat16)
    stats = LinearDispatchStats()
    out = linear_native(x.to(DEV), w.to(DEV), s.to(DEV), stats=stats)
    out_packed = linear_native(x.to(DEV), ops.fp8_pack_weight(w.to(DEV)), s.to(DEV), stats=stats)
    assert stats.cuda_kernel_hits == 2 and stats.fallback_calls == 0
    assert out.shape == (2, 5, 256) and out.dtype == torch.float32 and torch.equal(out, out_packed)
    ref = oracle.linear(x.float().view(-1, 384), w.view(torch.uint8).numpy(), s).view(2, 5, 256)
    torch.testing.assert_close(out.cpu(), ref, atol=2e-3, rtol=2e-3)
