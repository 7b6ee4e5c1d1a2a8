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


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows", [1, 17, 33, 64])
@pytest.mark.parametrize(("n", "k", "splits"), [(2048, 2048, 8), (2048, 5632, 8), (2560, 2048, 7),
                                                (100, 96, 3), (64, 32, 1), (11264, 2048, 2)])
def test_linear_partials_sum_matches_fp32(device, dtype, rows, n, k, splits):
    """Split-K partials summed and rounded once equal the fp32 product within
    the storage type's bar; each partial is the product over its own K slice
    (slices of ceil(K / 32 / splits) k-steps)."""

    from tensorforge_amd.kernels import linear_partials, linear_partials_sum

    generator = torch.Generator().manual_seed(rows * 7 + n + k + splits)
    x = torch.randn(rows, k, generator=generator).to(dtype)
    w = (torch.randn(n, k, generator=generator) * 0.02).to(dtype)
    partials = linear_partials(x.to(device), w.to(device), splits)
    steps = k // 32
    per = -(-steps // splits) * 32
    expected_partials = torch.stack([x[:, s * per:(s + 1) * per].float()
                                     @ w[:, s * per:(s + 1) * per].float().T
                                     for s in range(splits)])
    scale = float(expected_partials.abs().max())
    torch.testing.assert_close(partials.cpu(), expected_partials, rtol=1e-4, atol=1e-4 * scale)
    out = linear_partials_sum(partials, dtype=dtype)
    expected = x.float() @ w.float().T
    tol = TOLERANCE[dtype]
    torch.testing.assert_close(out.float().cpu(), expected, rtol=tol,
                               atol=tol * float(expected.abs().max()))
    # The row sum rounds the fp32 sum of the partials (summed in slice order).
    running = partials[0].clone()
    for s in range(1, splits):
        running += partials[s]
    assert torch.equal(out.cpu(), running.to(dtype).cpu())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows", [1, 17, 33, 64])
@pytest.mark.parametrize(("n", "k", "splits"), [(2048, 2048, 8), (2048, 5632, 8), (2560, 2048, 1),
                                                (11264, 2048, 1), (100, 96, 3), (64, 32, 1),
                                                (300, 800, 5), (96, 2080, 1)])
def test_linear_stream_matches_fp32(device, dtype, rows, n, k, splits):
    """The LDS-staged weight stream: slice sums within fp32 accumulation
    error of the fp32 slice products, and the direct (one-slice) output
    within the storage type's bar of the fp32 product -- on partial 256-wide
    chunks (K = 800 in slices of 160, K = 2080), tail column tiles and
    every row count the decode step uses."""

    from tensorforge_amd.kernels import linear_stream

    generator = torch.Generator().manual_seed(rows * 11 + n + k + splits)
    x = torch.randn(rows, k, generator=generator).to(dtype)
    w = (torch.randn(n, k, generator=generator) * 0.02).to(dtype)
    steps = k // 32
    per = -(-steps // splits) * 32
    expected_partials = torch.stack([x[:, s * per:(s + 1) * per].float()
                                     @ w[:, s * per:(s + 1) * per].float().T
                                     for s in range(splits)])
    partials = torch.full((splits, rows, n), float("nan"), device=device)
    linear_stream(x.to(device), w.to(device), splits=splits, partials=partials)
    scale = float(expected_partials.abs().max())
    torch.testing.assert_close(partials.cpu(), expected_partials, rtol=1e-4, atol=1e-4 * scale)
    if splits == 1:
        out = torch.full((rows, n), float("nan"), device=device, dtype=dtype)
        linear_stream(x.to(device), w.to(device), output=out)
        expected = x.float() @ w.float().T
        tol = TOLERANCE[dtype]
        torch.testing.assert_close(out.float().cpu(), expected, rtol=tol,
                                   atol=tol * float(expected.abs().max()))
        # The direct output is the one-slice partial rounded once.
        assert torch.equal(out.cpu(), partials[0].to(dtype).cpu())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows", [1, 9, 33, 64])
@pytest.mark.parametrize(("inter", "k"), [(5632, 2048), (768, 256), (100, 800), (48, 96)])
def test_linear_swiglu_equals_projection_then_activation(device, dtype, rows, inter, k):
    """The gate|up projection with SwiGLU in its epilogue is bit-identical
    to linear_stream of the stacked weight followed by swiglu_gate_up, and
    within the storage bar of the fp32 reference; tail column groups
    (intermediate not a multiple of 32) included."""

    from tensorforge_amd.kernels import linear_stream, linear_swiglu, swiglu_gate_up

    generator = torch.Generator().manual_seed(rows * 17 + inter + k)
    x = torch.randn(rows, k, generator=generator).to(dtype).to(device)
    w = (torch.randn(2 * inter, k, generator=generator) * 0.05).to(dtype).to(device)
    want = swiglu_gate_up(linear_stream(x, w))
    got = torch.full((rows, inter), float("nan"), dtype=dtype, device=device)
    linear_swiglu(x, w, output=got)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    gu = (x.float() @ w.float().T).to(dtype).float().cpu()
    g, u = gu[:, :inter], gu[:, inter:]
    expected = g * torch.sigmoid(g) * u
    tol = TOLERANCE[dtype]
    torch.testing.assert_close(got.float().cpu(), expected, rtol=tol,
                               atol=tol * float(expected.abs().max()))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows", [1, 17, 33, 64])
@pytest.mark.parametrize(("n", "k"), [(2560, 2048), (2048, 2048), (100, 96), (48, 800),
                                    (256, 4128)])
def test_linear_kstream_matches_fp32(device, dtype, rows, n, k):
    """K split over a workgroup's wavefronts: within the storage bar of the
    fp32 product, on tail column tiles, K that ends inside a chunk or leaves
    a wavefront without work (K = 96: 3 k-steps for 4 wavefronts) and
    strided output rows, under each tiling the launcher picks (2560 columns:
    1 row tile x 2 column tiles in 3 row blocks at 33 rows, 2 x 2 in 2
    blocks at 64; 2048 columns: 2 x 1 in 2 blocks at 33-64 rows; 100
    columns: 1 x 1 in up to 4 blocks)."""

    from tensorforge_amd.kernels import linear_kstream

    generator = torch.Generator().manual_seed(rows * 19 + n + k)
    x = torch.randn(rows, k, generator=generator).to(dtype)
    w = (torch.randn(n, k, generator=generator) * 0.02).to(dtype)
    out_wide = torch.full((rows, n + 8), float("nan"), dtype=dtype, device=device)
    linear_kstream(x.to(device), w.to(device), output=out_wide[:, :n])
    expected = x.float() @ w.float().T
    tol = TOLERANCE[dtype]
    torch.testing.assert_close(out_wide[:, :n].float().cpu(), expected, rtol=tol,
                               atol=tol * float(expected.abs().max()))
    assert bool(out_wide[:, n:].isnan().all())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows", [1, 33, 64])
@pytest.mark.parametrize(("inter", "k"), [(5632, 2048), (4100, 256), (100, 800), (48, 96)])
def test_linear_kswiglu_equals_kstream_then_activation(device, dtype, rows, inter, k):
    """The K-split gate|up + SwiGLU launch is bit-identical to linear_kstream
    of the stacked weight followed by swiglu_gate_up, and within the storage
    bar of the fp32 reference.  From 4096 activation columns a workgroup
    takes two 16-column tiles (4100: the last workgroup holds 4 columns of
    its first tile and none of its second)."""

    from tensorforge_amd.kernels import linear_kstream, linear_swiglu, swiglu_gate_up

    generator = torch.Generator().manual_seed(rows * 23 + inter + k)
    x = torch.randn(rows, k, generator=generator).to(dtype).to(device)
    w = (torch.randn(2 * inter, k, generator=generator) * 0.05).to(dtype).to(device)
    want = swiglu_gate_up(linear_kstream(x, w))
    got = torch.full((rows, inter), float("nan"), dtype=dtype, device=device)
    linear_swiglu(x, w, output=got, k_split=True)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    gu = (x.float() @ w.float().T).to(dtype).float().cpu()
    g, u = gu[:, :inter], gu[:, inter:]
    expected = g * torch.sigmoid(g) * u
    tol = TOLERANCE[dtype]
    torch.testing.assert_close(got.float().cpu(), expected, rtol=tol,
                               atol=tol * float(expected.abs().max()))


def test_linear_stream_strided_rows_and_rejections(device):
    from tensorforge_amd.kernels import linear_stream

    generator = torch.Generator().manual_seed(9)
    wide = torch.randn(40, 2048 + 64, generator=generator).to(torch.bfloat16).to(device)
    x = wide[:, 64:]
    w = (torch.randn(300, 2048, generator=generator) * 0.02).to(torch.bfloat16).to(device)
    out_wide = torch.zeros(40, 320, dtype=torch.bfloat16, device=device)
    linear_stream(x, w, output=out_wide[:, :300])
    expected = x.float() @ w.float().T
    torch.testing.assert_close(out_wide[:, :300].float(), expected, rtol=2e-2,
                               atol=2e-2 * float(expected.abs().max()))
    assert bool((out_wide[:, 300:] == 0).all())
    with pytest.raises(ValueError, match="partials buffer"):
        linear_stream(x, w, splits=2)
    with pytest.raises(ValueError):
        linear_stream(torch.zeros(65, 2048, dtype=torch.bfloat16, device=device), w)
    partials = torch.empty(4, 40, 300, device=device)
    linear_stream(x[:, :96], w[:, :96], splits=3, partials=partials[:3])  # one k-step each
    torch.testing.assert_close(partials[:3].sum(0), x[:, :96].float() @ w[:, :96].float().T,
                               rtol=1e-4, atol=1e-3)
    with pytest.raises(RuntimeError, match="non-empty"):
        # 5 k-steps in slices of 2 fill only 3 slices
        linear_stream(x[:, :160], w[:, :160], splits=4, partials=partials)


def test_linear_partials_strided_x_and_rejections(device):
    from tensorforge_amd.kernels import linear_partials

    generator = torch.Generator().manual_seed(5)
    wide = torch.randn(40, 2048 + 64, generator=generator).to(torch.bfloat16).to(device)
    x = wide[:, 64:]
    w = (torch.randn(300, 2048, generator=generator) * 0.02).to(torch.bfloat16).to(device)
    partials = linear_partials(x, w, 4)
    expected = x.float() @ w.float().T
    torch.testing.assert_close(partials.sum(0), expected, rtol=1e-3,
                               atol=1e-3 * float(expected.abs().max()))
    with pytest.raises(RuntimeError, match="splits"):
        linear_partials(x, w, 65)  # more slices than k-steps
    with pytest.raises(RuntimeError, match="non-empty"):
        linear_partials(x[:, :160], w[:, :160], 4)  # 5 k-steps in slices of 2 fill only 3
    with pytest.raises(ValueError):
        linear_partials(torch.randn(65, 64, dtype=torch.bfloat16, device=device),
                        w[:, :64], 1)


def _rms_scale(x: torch.Tensor, eps: float) -> torch.Tensor:
    return torch.rsqrt(x.float().pow(2).mean(dim=-1, keepdim=True) + eps)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows", [1, 17, 33, 64])
@pytest.mark.parametrize(("n", "k"), [(2560, 2048), (2048, 2048), (100, 96), (48, 800)])
def test_linear_kstream_norm_is_the_norm_then_the_projection(device, dtype, rows, n, k):
    """The RMSNorm of x's rows fused into the K-split projection, with the
    norm gain folded into the weight: within the storage bar of
    rsqrt(mean(x^2) + eps) * (x . w') in fp32, and of the reference's
    unfused order (RMSNorm rounded to the storage type, then the
    projection of the unfolded weight)."""

    from tensorforge_amd.kernels import fold_norm_gain, linear_kstream, rms_norm

    eps = 1e-5
    generator = torch.Generator().manual_seed(rows * 7 + n + k)
    x = (torch.randn(rows, k, generator=generator) * 3.0).to(dtype)
    w = (torch.randn(n, k, generator=generator) * 0.02).to(dtype)
    gain = (1.0 + 0.1 * torch.randn(k, generator=generator)).to(dtype)
    folded = fold_norm_gain(w.to(device), gain.to(device))
    assert torch.equal(folded.cpu(), (w.float() * gain.float()).to(dtype))
    out = torch.full((rows, n + 8), float("nan"), dtype=dtype, device=device)
    linear_kstream(x.to(device), folded, output=out[:, :n], norm_eps=eps)
    got = out[:, :n].float().cpu()
    assert bool(out[:, n:].isnan().all())
    expected = _rms_scale(x, eps) * (x.float() @ folded.float().cpu().T)
    tol = TOLERANCE[dtype]
    torch.testing.assert_close(got, expected, rtol=tol, atol=tol * float(expected.abs().max()))
    normed = rms_norm(x.to(device), gain.to(device), eps)
    unfused = linear_kstream(normed, w.to(device)).float().cpu()
    torch.testing.assert_close(got, unfused, rtol=2 * tol,
                               atol=2 * tol * float(expected.abs().max()))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows", [1, 33, 64])
@pytest.mark.parametrize(("inter", "k"), [(5632, 2048), (4100, 256), (100, 800)])
def test_linear_kswiglu_norm_is_the_norm_then_the_mlp_input(device, dtype, rows, inter, k):
    from tensorforge_amd.kernels import fold_norm_gain, linear_swiglu

    eps = 1e-5
    generator = torch.Generator().manual_seed(rows * 11 + inter + k)
    x = (torch.randn(rows, k, generator=generator) * 2.0).to(dtype)
    w = (torch.randn(2 * inter, k, generator=generator) * 0.05).to(dtype)
    gain = (1.0 + 0.1 * torch.randn(k, generator=generator)).to(dtype)
    folded = fold_norm_gain(w.to(device), gain.to(device))
    got = linear_swiglu(x.to(device), folded, k_split=True, norm_eps=eps).float().cpu()
    gu = (_rms_scale(x, eps) * (x.float() @ folded.float().cpu().T)).to(dtype).float()
    g, u = gu[:, :inter], gu[:, inter:]
    expected = g * torch.sigmoid(g) * u
    tol = TOLERANCE[dtype]
    torch.testing.assert_close(got, expected, rtol=tol, atol=tol * float(expected.abs().max()))
    with pytest.raises(ValueError, match="K-split"):
        linear_swiglu(x.to(device), folded, norm_eps=eps)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows", [49, 57, 64])
@pytest.mark.parametrize("inter", [2048, 5632, 8192])
def test_activation_resident_swiglu_norm_equals_the_k_split_form(device, dtype, rows, inter):
    """At 49-64 rows and K = 2048 the SwiGLU + RMSNorm launch keeps each
    workgroup's rows of x in LDS and streams only the weight; per row it is
    bit-identical to the K-split form, which the same call takes in chunks of
    at most 32 rows (strided x and output rows)."""

    from tensorforge_amd.kernels import fold_norm_gain, linear_swiglu

    eps, k = 1e-5, 2048
    generator = torch.Generator().manual_seed(rows * 31 + inter)
    x_wide = (torch.randn(rows, k + 64, generator=generator) * 2.0).to(dtype).to(device)
    x = x_wide[:, 32:32 + k]
    w = (torch.randn(2 * inter, k, generator=generator) * 0.05).to(dtype)
    gain = (1.0 + 0.1 * torch.randn(k, generator=generator)).to(dtype)
    folded = fold_norm_gain(w.to(device), gain.to(device))
    wide = torch.full((rows, inter + 8), float("nan"), dtype=dtype, device=device)
    linear_swiglu(x, folded, output=wide[:, :inter], k_split=True, norm_eps=eps)
    chunks = torch.full_like(wide, float("nan"))
    for r0 in range(0, rows, 32):
        r1 = min(r0 + 32, rows)
        linear_swiglu(x[r0:r1], folded, output=chunks[r0:r1, :inter], k_split=True, norm_eps=eps)
    torch.cuda.synchronize()
    assert torch.equal(wide[:, :inter].view(torch.int16), chunks[:, :inter].view(torch.int16))
    assert bool(wide[:, inter:].isnan().all())
    gu = (_rms_scale(x.cpu(), eps) * (x.float().cpu() @ folded.float().cpu().T)).to(dtype).float()
    g, u = gu[:, :inter], gu[:, inter:]
    expected = g * torch.sigmoid(g) * u
    tol = TOLERANCE[dtype]
    torch.testing.assert_close(wide[:, :inter].float().cpu(), expected, rtol=tol,
                               atol=tol * float(expected.abs().max()))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows", [1, 33, 64])
@pytest.mark.parametrize(("n", "k"), [(2048, 2048), (2048, 5632), (100, 96)])
def test_linear_kstream_residual_is_the_rounded_residual_sum(device, dtype, rows, n, k):
    """round(round(x . w) + residual): the residual output of the
    reference's residual_rms_norm over the projection, bit for bit."""

    from tensorforge_amd.kernels import linear_kstream

    generator = torch.Generator().manual_seed(rows * 13 + n + k)
    x = torch.randn(rows, k, generator=generator).to(dtype).to(device)
    w = (torch.randn(n, k, generator=generator) * 0.02).to(dtype).to(device)
    residual = torch.randn(rows, n, generator=generator).to(dtype).to(device)
    got = linear_kstream(x, w, residual=residual)
    want = (linear_kstream(x, w).float() + residual.float()).to(dtype)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    with pytest.raises(ValueError, match="not both"):
        linear_kstream(x, w, residual=residual, norm_eps=1e-5)
    with pytest.raises(ValueError, match="residual must be"):
        linear_kstream(x, w, residual=residual[:, : n // 2])
