"""Decode-shaped linear layer on gfx950 MFMA (``csrc/tf_linear_rows.hip``).

``linear_rows(x, weight)`` computes ``x @ weight.T`` like
``torch.nn.functional.linear`` without bias, for at most 64 rows -- the
shape of every projection in a decode step (the reference's nn.Linear
layers, tensorforge/model/layers.py:88-95, 144-146).  At that shape the
product streams the weight matrix once and is HBM-bound; the kernel splits
K across wavefronts so a launch has thousands of wavefronts streaming
short weight slabs instead of a hundred walking all of K.
"""

from __future__ import annotations

import torch
from torch import Tensor

from tensorforge_amd import _native

MAX_ROWS = 64


def linear_rows_supported(x: Tensor, weight: Tensor) -> bool:
    """Whether :func:`linear_rows` takes these operands (else use F.linear)."""

    return (x.ndim == 2 and weight.ndim == 2 and x.shape[0] <= MAX_ROWS
            and x.dtype in (torch.float16, torch.bfloat16) and weight.dtype == x.dtype
            and x.shape[1] == weight.shape[1] and x.shape[1] % 32 == 0 and x.stride(1) == 1
            and weight.stride(1) == 1 and x.stride(0) % 8 == 0 and weight.stride(0) % 8 == 0
            and x.data_ptr() % 16 == 0 and weight.data_ptr() % 16 == 0 and x.is_cuda
            and weight.is_cuda)


def linear_rows(x: Tensor, weight: Tensor, *, output: Tensor | None = None,
                waves_per_tile: int = 0) -> Tensor:
    """``x [m, k] @ weight[n, k].T`` for m <= 64, fp16/bf16, fp32 accumulation."""

    if not _native.is_available():
        raise RuntimeError(
            "the gfx950 kernel library is unavailable; build it with "
            "`python -m tensorforge_amd.build`"
        )
    if not linear_rows_supported(x, weight):
        raise ValueError("linear_rows needs fp16/bf16 CUDA operands [m <= 64, k] and [n, k] "
                         "with k % 32 == 0 and 16-byte aligned contiguous rows")
    m, k = x.shape
    n = weight.shape[0]
    if output is None:
        output = torch.empty((m, n), dtype=x.dtype, device=x.device)
    if (output.shape != (m, n) or output.dtype != x.dtype or output.device != x.device
            or output.stride(1) != 1):
        raise ValueError("output must be [m, n] with contiguous rows, x's dtype and device")
    _native.check(
        _native.library().tf_linear_rows(
            x.data_ptr(), x.stride(0), weight.data_ptr(), weight.stride(0), output.data_ptr(),
            output.stride(0), m, n, k, waves_per_tile, _native.dtype_code(x.dtype),
            _native.current_stream(x.device),
        ),
        "linear_rows",
    )
    return output
