"""Greedy sampling on the device (tf_argmax_rows) against torch.argmax of
the same values on the CPU, the reference's sampling rule
(scheduler/continuous.py:265-275): bit-exact indices, including ties (the
first index), NaN (the first NaN), rows of -inf, zeros of either sign, odd widths (the scalar
tail), several passes per row and strided rows."""

from __future__ import annotations

import pytest
import torch

from tensorforge_amd.kernels import argmax_rows

pytestmark = pytest.mark.gpu


def _expect(values: torch.Tensor) -> torch.Tensor:
    return torch.argmax(values.float().cpu(), dim=-1)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize(("rows", "columns"), [(1, 32000), (64, 32000), (3, 7), (5, 40000),
                                               (2, 1), (7, 1031)])
def test_argmax_rows_matches_torch(device, dtype, rows, columns):
    generator = torch.Generator().manual_seed(rows * 131 + columns)
    values = torch.randn(rows, columns, generator=generator).to(dtype)
    got = argmax_rows(values.to(device))
    assert got.dtype == torch.int64
    assert torch.equal(got.cpu(), _expect(values))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_argmax_rows_ties_nan_and_infinities(device, dtype):
    columns = 32000
    values = torch.zeros(8, columns).to(dtype)
    values[0, [5, 17, 31999]] = 3.0                 # ties: the first index
    values[1, [9000, 100]] = 7.0                    # ties across threads and passes
    values[2, [40, 20000]] = float("nan")           # the first NaN
    values[2, 10] = float("inf")
    values[3] = float("-inf")                       # all -inf: index 0
    values[4, 12345] = float("inf")
    values[5, -1] = 1e-3                            # the last column
    values[6] = float("-inf")                       # +0 then -0: the first zero
    values[6, 5], values[6, 10] = 0.0, -0.0
    values[7] = float("-inf")                       # -0 then +0: the first zero
    values[7, 5], values[7, 10] = -0.0, 0.0
    got = argmax_rows(values.to(device)).cpu()
    assert got.tolist() == [5, 100, 40, 0, 12345, columns - 1, 5, 5]
    assert torch.equal(got, torch.argmax(values.float(), dim=-1))


def test_argmax_rows_strided_rows_and_output(device):
    generator = torch.Generator().manual_seed(5)
    wide = torch.randn(9, 1000 + 3, generator=generator).to(torch.bfloat16).to(device)
    view = wide[:, 3:]                              # row stride 1003: the scalar path
    out = torch.full((9,), -1, dtype=torch.int64, device=device)
    argmax_rows(view, output=out)
    assert torch.equal(out.cpu(), _expect(view))
    assert argmax_rows(torch.empty(0, 5, device=device)).numel() == 0
    with pytest.raises(ValueError, match="empty row"):
        argmax_rows(torch.empty(2, 0, device=device))
    with pytest.raises(ValueError, match="int64"):
        argmax_rows(view, output=torch.empty(9, dtype=torch.int32, device=device))
