"""The decode-shaped MFMA linear layer against a plain fp32 torch product.

Tolerance: the fp32 sum rounded once to the storage type, so the result
sits within one unit in the last place of the fp32 reference plus the
reordering of a K-term fp32 sum (the reference's elementwise bars,
tests/test_triton_kernels.py:21-26: fp16 3e-3, bf16 3e-2 relative).
"""

from __future__ import annotations

import pytest
import torch

from tensorforge_amd.kernels import linear_rows, linear_rows_supported

pytestmark = pytest.mark.gpu

TOLERANCE = {torch.float16: 3e-3, torch.bfloat16: 3e-2}


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows", [1, 3, 16, 17, 40, 64])
@pytest.mark.parametrize(("n", "k"), [(3072, 2048), (2048, 5632), (11264, 2048), (1000, 96),
                                      (40, 32), (32000, 2048)])
def test_linear_rows_matches_fp32(device, dtype, rows, n, k):
    generator = torch.Generator().manual_seed(rows * 131 + n + k)
    x = torch.randn(rows, k, generator=generator).to(dtype)
    w = (torch.randn(n, k, generator=generator) * 0.02).to(dtype)
    expected = x.float() @ w.float().T
    actual = linear_rows(x.to(device), w.to(device))
    scale = float(expected.abs().max())
    tol = TOLERANCE[dtype]
    torch.testing.assert_close(actual.float().cpu(), expected, rtol=tol, atol=tol * scale)


@pytest.mark.parametrize("waves", [1, 3, 16])
def test_linear_rows_any_k_split_and_strided_operands(device, waves):
    """Every K split gives the same sums (within fp32 reordering); x and the
    output may be column slices of wider buffers."""

    generator = torch.Generator().manual_seed(waves)
    wide_x = torch.randn(24, 2048 + 64, generator=generator).to(torch.bfloat16).to(device)
    x = wide_x[:, 64:]
    w = (torch.randn(512, 2048, generator=generator) * 0.02).to(torch.bfloat16).to(device)
    out = torch.zeros(24, 600, dtype=torch.bfloat16, device=device)
    assert linear_rows_supported(x, w)
    linear_rows(x, w, output=out[:, 40:552], waves_per_tile=waves)
    expected = x.float() @ w.float().T
    torch.testing.assert_close(out[:, 40:552].float(), expected, rtol=3e-2,
                               atol=3e-2 * float(expected.abs().max()))
    assert not out[:, :40].any() and not out[:, 552:].any()


def test_linear_rows_rejects_unsupported_shapes(device):
    x = torch.randn(65, 64, dtype=torch.bfloat16, device=device)
    w = torch.randn(32, 64, dtype=torch.bfloat16, device=device)
    assert not linear_rows_supported(x, w)
    with pytest.raises(ValueError):
        linear_rows(x, w)
    assert not linear_rows_supported(x[:4, :48], w[:, :48])  # K % 32
