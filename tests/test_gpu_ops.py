"""Parity of the gfx950 RMSNorm, residual RMSNorm and SwiGLU with the oracle.

Mirrors tests/test_triton_kernels.py of the reference (grids :29-76,
adversarial fills :79-91, observability :94-110, cancellation/saturation
:113-127, rejections :130-150, caller-owned outputs :153-213) and adds the
BASELINE config 4 sizes with the build's bf16 bar (2e-2 abs + 1e-2 rel).
"""

from __future__ import annotations

import pytest
import torch

from helpers import NORTH_STAR_ATOL, NORTH_STAR_RTOL, REFERENCE_TOLERANCE, assert_bit_exact, assert_close
from oracle.reference import (
    residual_rms_norm_fused_reference,
    residual_rms_norm_reference,
    rms_norm_reference,
    swiglu_fused_reference,
    swiglu_reference,
)
from tensorforge_amd.kernels import (
    autotune_cache_size,
    residual_rms_norm,
    rms_norm,
    selected_autotune_config,
    swiglu,
    swiglu_gate_up,
)

pytestmark = pytest.mark.gpu
DTYPES = [torch.float32, torch.float16, torch.bfloat16]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(1, 1), (3, 7), (7, 513), (16, 1376), (4, 4096), (2, 8192),
                                   (2, 16384), (3, 16383)])
def test_rms_norm_shape_dtype_grid(device, shape, dtype):
    inputs = torch.randn(shape).to(dtype)
    weight = torch.randn(shape[-1]).to(dtype)
    actual = rms_norm(inputs.to(device), weight.to(device))
    expected = rms_norm_reference(inputs, weight, 1e-6)
    tol = REFERENCE_TOLERANCE[dtype]
    assert_close(actual, expected, tol, tol, f"rms_norm {shape} {dtype}")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(1, 7), (7, 513), (16, 1376), (4, 4096)])
def test_residual_rms_norm_shape_dtype_grid(device, shape, dtype):
    inputs = torch.randn(shape).to(dtype)
    residual = torch.randn(shape).to(dtype)
    weight = torch.randn(shape[-1]).to(dtype)
    actual_residual, actual_norm = residual_rms_norm(inputs.to(device), residual.to(device),
                                                     weight.to(device))
    expected_residual, expected_norm = residual_rms_norm_reference(inputs, residual, weight, 1e-6)
    tol = REFERENCE_TOLERANCE[dtype]
    assert_bit_exact(actual_residual, expected_residual, "residual sum")
    assert_close(actual_norm, expected_norm, tol, tol, f"residual norm {shape} {dtype}")
    _, fused_norm = residual_rms_norm_fused_reference(inputs, residual, weight, 1e-6)
    assert_close(actual_norm, fused_norm, tol, tol, "fused semantics")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(1, 1), (3, 7), (7, 513), (16, 1376), (2, 11008)])
def test_swiglu_shape_dtype_grid(device, shape, dtype):
    gate = torch.randn(shape).to(dtype)
    up = torch.randn(shape).to(dtype)
    actual = swiglu(gate.to(device), up.to(device))
    tol = REFERENCE_TOLERANCE[dtype]
    assert_close(actual, swiglu_reference(gate, up), tol, tol, f"swiglu {shape} {dtype}")
    assert_close(actual, swiglu_fused_reference(gate, up), tol, tol, "fused semantics")


@pytest.mark.parametrize("tokens", [1, 8, 64, 256])
@pytest.mark.parametrize("hidden", [2048, 4096])
def test_config4_residual_rms_norm_bf16(device, tokens, hidden):
    generator = torch.Generator().manual_seed(tokens * hidden)
    inputs = torch.randn(tokens, hidden, generator=generator).to(torch.bfloat16)
    residual = torch.randn(tokens, hidden, generator=generator).to(torch.bfloat16)
    weight = (1.0 + 0.1 * torch.randn(hidden, generator=generator)).to(torch.bfloat16)
    res, norm = residual_rms_norm(inputs.to(device), residual.to(device), weight.to(device), 1e-5)
    exp_res, exp_norm = residual_rms_norm_fused_reference(inputs, residual, weight, 1e-5)
    assert_bit_exact(res, exp_res, "residual sum")
    assert_close(norm, exp_norm, NORTH_STAR_ATOL, NORTH_STAR_RTOL, "norm")
    plain = rms_norm(inputs.to(device), weight.to(device), 1e-5)
    assert_close(plain, rms_norm_reference(inputs, weight, 1e-5), NORTH_STAR_ATOL,
                 NORTH_STAR_RTOL, "rms_norm")


@pytest.mark.parametrize("tokens", [1, 8, 64, 256])
@pytest.mark.parametrize("ffn", [5632, 14336])
def test_config4_swiglu_bf16(device, tokens, ffn):
    generator = torch.Generator().manual_seed(tokens + ffn)
    gate = torch.randn(tokens, ffn, generator=generator).to(torch.bfloat16)
    up = torch.randn(tokens, ffn, generator=generator).to(torch.bfloat16)
    actual = swiglu(gate.to(device), up.to(device))
    assert_close(actual, swiglu_fused_reference(gate, up), NORTH_STAR_ATOL, NORTH_STAR_RTOL,
                 "swiglu")


@pytest.mark.parametrize("fill", [0.0, 1e-5, 100.0, -100.0])
def test_rms_norm_adversarial_values(device, fill):
    inputs = torch.full((3, 513), fill, dtype=torch.float32)
    weight = torch.linspace(-2, 2, 513)
    actual = rms_norm(inputs.to(device), weight.to(device))
    assert_close(actual, rms_norm_reference(inputs, weight, 1e-6), 1e-5, 1e-5, f"fill {fill}")
    assert bool(torch.isfinite(actual).all())


def test_autotune_selection_is_observable(device):
    """The reference's test body (tests/test_triton_kernels.py:94-110),
    assertion unchanged: the norm launches 1, 2, 4 or 8 wavefronts."""

    inputs = torch.randn(4, 513, device=device, dtype=torch.float16)
    weight = torch.ones(513, device=device, dtype=torch.float16)
    rms_norm(inputs, weight)
    rms_norm(torch.randn(16, 513, device=device, dtype=torch.float16), weight)

    config = selected_autotune_config("rms_norm")
    assert config is not None
    assert config["num_warps"] in {1, 2, 4, 8}
    assert autotune_cache_size("rms_norm") >= 2
    with pytest.raises(ValueError, match="unknown operation"):
        selected_autotune_config("layer_norm")


@pytest.mark.parametrize("columns", [1, 63, 513, 2048, 4096, 16383, 16384])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_norm_hooks_report_reference_warp_counts_at_every_width(device, columns, dtype):
    """Every width up to the 16384-column limit runs in 1..8 wavefronts,
    residual variant included, and stays within the bar."""

    generator = torch.Generator().manual_seed(columns)
    inputs = torch.randn(3, columns, generator=generator).to(dtype)
    residual = torch.randn(3, columns, generator=generator).to(dtype)
    weight = (1 + 0.1 * torch.randn(columns, generator=generator)).to(dtype)
    actual = rms_norm(inputs.to(device), weight.to(device), 1e-5)
    assert selected_autotune_config("rms_norm")["num_warps"] in {1, 2, 4, 8}
    assert_close(actual, rms_norm_reference(inputs, weight, 1e-5), NORTH_STAR_ATOL,
                 NORTH_STAR_RTOL, f"rms_norm {columns}")
    summed, normed = residual_rms_norm(inputs.to(device), residual.to(device), weight.to(device),
                                       1e-5)
    assert selected_autotune_config("residual_rms_norm")["num_warps"] in {1, 2, 4, 8}
    assert_bit_exact(summed, (inputs.float() + residual.float()).to(dtype), "residual sum")
    assert_close(normed, rms_norm_reference(summed.cpu(), weight, 1e-5), NORTH_STAR_ATOL,
                 NORTH_STAR_RTOL, f"residual_rms_norm {columns}")


def test_residual_cancellation_and_swiglu_extremes(device):
    inputs = torch.linspace(-10, 10, 513).repeat(3, 1)
    residual = -inputs + 1e-5
    weight = torch.linspace(0.5, 1.5, 513)
    actual_residual, actual_norm = residual_rms_norm(inputs.to(device), residual.to(device),
                                                     weight.to(device))
    expected_residual, expected_norm = residual_rms_norm_reference(inputs, residual, weight, 1e-6)
    assert_close(actual_residual, expected_residual, 1e-5, 1e-5, "cancellation sum")
    assert_close(actual_norm, expected_norm, 1e-4, 1e-4, "cancellation norm")
    gate = torch.linspace(-20, 20, 513).repeat(3, 1)
    up = torch.linspace(2, -2, 513).repeat(3, 1)
    assert_close(swiglu(gate.to(device), up.to(device)), swiglu_reference(gate, up), 1e-5, 1e-5,
                 "swiglu saturation")


def test_kernels_reject_cpu_and_noncontiguous_inputs(device):
    with pytest.raises(ValueError, match="CUDA"):
        rms_norm(torch.randn(2, 8), torch.ones(8))
    inputs = torch.randn(8, 8, device=device).transpose(0, 1)
    with pytest.raises(ValueError, match="contiguous"):
        rms_norm(inputs, torch.ones(8, device=device))
    gate = torch.randn(2, 8, device=device, requires_grad=True)
    with pytest.raises(RuntimeError, match="inference-only"):
        swiglu(gate, torch.randn_like(gate))


def test_caller_owned_outputs_are_reused_and_numerically_correct(device):
    inputs = torch.randn(3, 64, device=device, dtype=torch.float16)
    residual = torch.randn_like(inputs)
    weight = torch.randn(64, device=device, dtype=torch.float16)
    gate = torch.randn(3, 160, device=device, dtype=torch.float16)
    up = torch.randn_like(gate)
    norm_output = torch.empty_like(inputs)
    residual_output = torch.empty_like(inputs)
    post_norm_output = torch.empty_like(inputs)
    swiglu_output = torch.empty_like(gate)
    buffers = (norm_output, residual_output, post_norm_output, swiglu_output)
    addresses = tuple(tensor.data_ptr() for tensor in buffers)
    assert rms_norm(inputs, weight, output=norm_output) is norm_output
    actual_residual, actual_post = residual_rms_norm(
        inputs, residual, weight, residual_output=residual_output, norm_output=post_norm_output,
    )
    assert actual_residual is residual_output and actual_post is post_norm_output
    assert swiglu(gate, up, output=swiglu_output) is swiglu_output
    assert addresses == tuple(tensor.data_ptr() for tensor in buffers)
    expected_residual, expected_post = residual_rms_norm_reference(inputs, residual, weight, 1e-6)
    assert_close(norm_output, rms_norm_reference(inputs, weight, 1e-6), 3e-3, 3e-3, "norm")
    assert_close(residual_output, expected_residual, 3e-3, 3e-3, "residual")
    assert_close(post_norm_output, expected_post, 3e-3, 3e-3, "post norm")
    assert_close(swiglu_output, swiglu_reference(gate, up), 3e-3, 3e-3, "swiglu")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize(("rows", "ffn", "pad"), [(1, 5632, 0), (64, 5632, 0), (8, 14336, 0),
                                                  (3, 77, 0), (5, 256, 8), (7, 96, 3)])
def test_swiglu_gate_up_equals_separate_swiglu(device, dtype, rows, ffn, pad):
    """The fused gate|up form is bit-identical to swiglu on the two halves
    (same arithmetic), for vector and scalar paths and padded row strides."""

    generator = torch.Generator().manual_seed(rows * 31 + ffn)
    gate_up = torch.randn(rows, 2 * ffn + pad, generator=generator).to(dtype).to(device)
    actual = swiglu_gate_up(gate_up[:, :2 * ffn] if pad else gate_up, output=None)
    gate = gate_up[:, :ffn].contiguous()
    up = gate_up[:, ffn:2 * ffn].contiguous()
    assert_bit_exact(actual, swiglu(gate, up), f"gate_up {rows}x{ffn}+{pad} {dtype}")
    tol = REFERENCE_TOLERANCE[dtype]
    assert_close(actual, swiglu_reference(gate.cpu(), up.cpu()), tol, tol, "oracle")
    wide = torch.zeros(rows, ffn + 5, dtype=dtype, device=device)
    swiglu_gate_up(gate_up[:, :2 * ffn + pad], output=wide[:, :ffn])
    assert_bit_exact(wide[:, :ffn], actual, "strided output")
    assert not wide[:, ffn:].any()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize(("rows", "columns", "splits"), [(64, 2048, 8), (17, 2048, 1), (5, 513, 3),
                                                         (32, 4096, 11)])
def test_residual_rms_norm_partials_equals_the_unfused_pair(device, dtype, rows, columns, splits):
    """The fused form equals rounding the slice sum (summed in slice order)
    and then running residual_rms_norm on it: the residual output bit for
    bit; the norm within one rounding of the storage type, since the fused
    form reduces the sum of squares over a different lane layout (one
    vector per lane instead of two), which can move inv_rms by an fp32 ulp."""

    from tensorforge_amd.kernels.ops import residual_rms_norm_partials

    generator = torch.Generator().manual_seed(rows + columns + splits)
    partials = torch.randn(splits, rows, columns, generator=generator).to(device)
    residual = torch.randn(rows, columns, generator=generator).to(dtype).to(device)
    weight = (1 + 0.1 * torch.randn(columns, generator=generator)).to(dtype).to(device)
    running = partials[0].clone()
    for s in range(1, splits):
        running += partials[s]
    inputs = running.to(dtype)
    want_residual, want_norm = residual_rms_norm(inputs, residual, weight, 1e-5)
    got_residual, got_norm = residual_rms_norm_partials(partials, residual, weight, 1e-5)
    assert torch.equal(got_residual, want_residual)
    ulp = {torch.float16: 2.0**-10, torch.bfloat16: 2.0**-7, torch.float32: 2.0**-22}[dtype]
    torch.testing.assert_close(got_norm.float(), want_norm.float(), rtol=ulp, atol=1e-6)
    with pytest.raises(ValueError, match="partials"):
        residual_rms_norm_partials(partials[:, :, 1:], residual, weight, 1e-5)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize(("hidden", "vocab"), [(2048, 32000), (256, 1024), (200, 50)])
def test_embedding_rms_norm_equals_gather_then_norm(device, dtype, hidden, vocab):
    """Token feedback + embedding + RMSNorm in one launch, bit-identical to
    index_select / where / F.embedding followed by rms_norm; lanes fed back
    (source >= 0) and host-given, out-of-range ids clamped."""

    import torch.nn.functional as F

    from tensorforge_amd.kernels import embedding_rms_norm, rms_norm

    generator = torch.Generator().manual_seed(hidden + vocab)
    rows = 12
    table = torch.randn(vocab, hidden, generator=generator).to(dtype).to(device)
    weight = (1 + 0.1 * torch.randn(hidden, generator=generator)).to(dtype).to(device)
    state = torch.randint(0, vocab, (16,), generator=generator).to(device)
    source = torch.tensor([3, -1, 0, 15, -1, 7, -1, 2, 2, -1, 9, -1], device=device)
    host = torch.randint(0, vocab, (rows,), generator=generator).to(device)
    host[5] = vocab + 7  # unused (fed lane)
    x = torch.full((rows, hidden), float("nan"), dtype=dtype, device=device)
    h = torch.full_like(x, float("nan"))
    embedding_rms_norm(state, source, host, table, weight, 1e-5, x_output=x, norm_output=h)
    ids = torch.where(source >= 0, state.index_select(0, source.clamp(min=0)), host)
    want_x = F.embedding(ids, table)
    want_h = rms_norm(want_x, weight, 1e-5)
    assert torch.equal(x.view(torch.int16), want_x.view(torch.int16))
    assert torch.equal(h.view(torch.int16), want_h.view(torch.int16))
    # A host id past the table reads its last row.
    host[1] = vocab + 3
    embedding_rms_norm(state, source, host, table, weight, 1e-5, x_output=x, norm_output=h)
    assert torch.equal(x[1].view(torch.int16), table[vocab - 1].view(torch.int16))
