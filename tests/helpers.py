"""Comparison helpers shared by the parity tests."""

from __future__ import annotations

import torch
from torch import Tensor

# Tolerances of the reference's own kernel tests
# (tests/test_decode_attention.py:103, tests/test_triton_kernels.py:21-26).
REFERENCE_TOLERANCE = {torch.float32: 1e-5, torch.float16: 3e-3, torch.bfloat16: 3e-2}
# Bar of this build for bf16/fp16 outputs with fp32 accumulation:
# |actual - expected| <= 2e-2 + 1e-2 * |expected|.
NORTH_STAR_ATOL = 2e-2
NORTH_STAR_RTOL = 1e-2


def assert_close(actual: Tensor, expected: Tensor, atol: float, rtol: float, what: str = "") -> None:
    actual = actual.detach().cpu().float()
    expected = expected.detach().cpu().float()
    assert actual.shape == expected.shape, f"{what}: shape {actual.shape} != {expected.shape}"
    diff = (actual - expected).abs()
    bound = atol + rtol * expected.abs()
    bad = diff > bound
    if bool(bad.any()) or not bool(torch.isfinite(actual).all()):
        index = int(torch.argmax((diff - bound).flatten()))
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {bad.numel()} elements out of tolerance "
            f"(atol {atol}, rtol {rtol}); max abs diff {float(diff.max()):.3e}; "
            f"worst flat index {index}: actual {float(actual.flatten()[index]):.6f} "
            f"expected {float(expected.flatten()[index]):.6f}"
        )


def assert_bit_exact(actual: Tensor, expected: Tensor, what: str = "") -> None:
    actual = actual.detach().cpu().contiguous()
    expected = expected.detach().cpu().contiguous()
    assert actual.shape == expected.shape and actual.dtype == expected.dtype, what
    width = {1: torch.int8, 2: torch.int16, 4: torch.int32, 8: torch.int64}[actual.element_size()]
    mismatch = actual.view(width) != expected.view(width)
    assert not bool(mismatch.any()), f"{what}: {int(mismatch.sum())} elements differ bitwise"
