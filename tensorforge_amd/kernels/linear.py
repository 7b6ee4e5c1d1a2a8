"""Decode-shaped linear layers on gfx950 MFMA (``csrc/tf_linear_rows.hip``,
``csrc/tf_linear_splitk.hip``).

``linear_rows(x, weight)`` computes ``x @ weight.T`` like
``torch.nn.functional.linear`` without bias, for at most 64 rows -- the
shape of every projection in a decode step (the reference's nn.Linear
layers, tensorforge/model/layers.py:88-95, 144-146).  At that shape the
product streams the weight matrix once and is HBM-bound; the kernel splits
K across wavefronts so a launch has thousands of wavefronts streaming
short weight slabs instead of a hundred walking all of K.

``linear_partials(x, weight, splits)`` is the split-K form for 17..64 rows:
each workgroup owns 64 output columns and one of ``splits`` slices of K, and
writes the slice's fp32 partial product; ``linear_partials_sum`` (or a
fused consumer) adds the slices and rounds once, which is the result of a
GEMM with fp32 accumulation.

``linear_stream`` computes the same products (direct, or as split-K slice
sums) with both operands staged through LDS by whole-row loads, which a
compute unit issues about 2.5x faster than loads in the MFMA operand layout.
``linear_swiglu`` is its form for the MLP's stacked gate|up weight with the
SwiGLU applied in the epilogue.
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


def linear_partials_supported(x: Tensor, weight: Tensor) -> bool:
    """Whether :func:`linear_partials` takes these operands."""

    return linear_rows_supported(x, weight) and x.shape[1] > 0


def default_splits(n: int, k: int) -> int:
    """K slices for an [n, k] weight: enough 64-column x slice workgroups
    (>= 256) to stream from every compute unit, slices of >= 256 k, and a
    count that divides K / 32 into non-empty slices."""

    steps = k // 32
    tiles = (n + 63) // 64
    want = max(1, min(-(-256 // tiles), max(1, k // 256)))
    want = min(want, steps)
    while want > 1 and -(-steps // -(-steps // want)) != want:
        want -= 1
    return want


def linear_partials(x: Tensor, weight: Tensor, splits: int, *,
                    partials: Tensor | None = None) -> Tensor:
    """fp32 ``[splits, m, n]`` partial products of ``x [m, k] @ weight[n, k].T``
    over ``splits`` contiguous slices of K (m <= 64, fp16/bf16)."""

    if not _native.is_available():
        raise RuntimeError(
            "the gfx950 kernel library is unavailable; build it with "
            "`python -m tensorforge_amd.build`"
        )
    if not linear_partials_supported(x, weight):
        raise ValueError("linear_partials needs fp16/bf16 CUDA operands [m <= 64, k] and [n, k] "
                         "with k % 32 == 0 and 16-byte aligned contiguous rows")
    m, k = x.shape
    n = weight.shape[0]
    if partials is None:
        partials = torch.empty((splits, m, n), dtype=torch.float32, device=x.device)
    if (partials.shape != (splits, m, n) or partials.dtype != torch.float32
            or partials.device != x.device or not partials.is_contiguous()):
        raise ValueError("partials must be a contiguous fp32 [splits, m, n] tensor on x's device")
    _native.check(
        _native.library().tf_linear_partials(
            x.data_ptr(), x.stride(0), weight.data_ptr(), weight.stride(0), partials.data_ptr(),
            m, n, k, splits, _native.dtype_code(x.dtype), _native.current_stream(x.device),
        ),
        "linear_partials",
    )
    return partials


def linear_stream(x: Tensor, weight: Tensor, *, splits: int = 1, output: Tensor | None = None,
                  partials: Tensor | None = None) -> Tensor:
    """``x [m, k] @ weight[n, k].T`` for m <= 64 with both operands staged
    through LDS by whole-row loads.  With ``partials`` (fp32 ``[splits, m,
    n]``) it writes the split-K slice sums of :func:`linear_partials` and
    returns them; otherwise ``splits`` must be 1 and it returns the rounded
    product in ``output`` (allocated when None)."""

    if not _native.is_available():
        raise RuntimeError(
            "the gfx950 kernel library is unavailable; build it with "
            "`python -m tensorforge_amd.build`"
        )
    if not linear_rows_supported(x, weight):
        raise ValueError("linear_stream needs fp16/bf16 CUDA operands [m <= 64, k] and [n, k] "
                         "with k % 32 == 0 and 16-byte aligned contiguous rows")
    m, k = x.shape
    n = weight.shape[0]
    y_ptr, y_stride, p_ptr = None, 0, None
    if partials is not None:
        if (partials.shape != (splits, m, n) or partials.dtype != torch.float32
                or partials.device != x.device or not partials.is_contiguous()):
            raise ValueError("partials must be a contiguous fp32 [splits, m, n] tensor on x's device")
        p_ptr = partials.data_ptr()
        result = partials
    else:
        if splits != 1:
            raise ValueError("several K slices need a partials buffer")
        if output is None:
            output = torch.empty((m, n), dtype=x.dtype, device=x.device)
        if (output.shape != (m, n) or output.dtype != x.dtype or output.device != x.device
                or output.stride(1) != 1):
            raise ValueError("output must be [m, n] with contiguous rows, x's dtype and device")
        y_ptr, y_stride = output.data_ptr(), output.stride(0)
        result = output
    _native.check(
        _native.library().tf_linear_stream(
            x.data_ptr(), x.stride(0), weight.data_ptr(), weight.stride(0), y_ptr, y_stride,
            p_ptr, m, n, k, splits, _native.dtype_code(x.dtype), _native.current_stream(x.device),
        ),
        "linear_stream",
    )
    return result


def linear_kstream(x: Tensor, weight: Tensor, *, output: Tensor | None = None,
                   norm_eps: float | None = None, residual: Tensor | None = None) -> Tensor:
    """``x [m, k] @ weight[n, k].T`` for m <= 64 with K split over the four
    wavefronts of workgroups of one or two 16-column tiles, each staging its
    chunks through LDS with whole-row loads (the form for weights with few
    64-column tiles).

    ``norm_eps``: the RMSNorm of x's rows applied to the product,
    ``round(rsqrt(mean(x[r]^2) + eps) * (x[r] . weight[n]))``, for a weight
    whose columns carry the norm's gain (:func:`fold_norm_gain`) -- the
    reference's RMSNorm followed by the projection
    (kernels/triton_ops.py:179-205; model/layers.py:88-95), with the gain
    rounded into the weight instead of into the normalised input.

    ``residual`` (``[m, n]``): the projection added to it,
    ``round(round(x . weight) + residual)`` -- the residual sum of the
    reference's residual_rms_norm (triton_ops.py:208-243), bit for bit."""

    if not _native.is_available():
        raise RuntimeError(
            "the gfx950 kernel library is unavailable; build it with "
            "`python -m tensorforge_amd.build`"
        )
    if not linear_rows_supported(x, weight):
        raise ValueError("linear_kstream needs fp16/bf16 CUDA operands [m <= 64, k] and [n, k] "
                         "with k % 32 == 0 and 16-byte aligned contiguous rows")
    if norm_eps is not None and residual is not None:
        raise ValueError("linear_kstream takes norm_eps or residual, not both")
    m, k = x.shape
    n = weight.shape[0]
    if output is None:
        output = torch.empty((m, n), dtype=x.dtype, device=x.device)
    if (output.shape != (m, n) or output.dtype != x.dtype or output.device != x.device
            or output.stride(1) != 1):
        raise ValueError("output must be [m, n] with contiguous rows, x's dtype and device")
    library = _native.library()
    stream = _native.current_stream(x.device)
    if residual is not None:
        if (residual.shape != (m, n) or residual.dtype != x.dtype
                or residual.device != x.device or residual.stride(1) != 1):
            raise ValueError("residual must be [m, n] with contiguous rows, x's dtype and device")
        _native.check(
            library.tf_linear_kstream_residual(
                x.data_ptr(), x.stride(0), weight.data_ptr(), weight.stride(0),
                residual.data_ptr(), residual.stride(0), output.data_ptr(), output.stride(0),
                m, n, k, _native.dtype_code(x.dtype), stream,
            ),
            "linear_kstream_residual",
        )
    elif norm_eps is not None:
        _native.check(
            library.tf_linear_kstream_norm(
                x.data_ptr(), x.stride(0), weight.data_ptr(), weight.stride(0),
                output.data_ptr(), output.stride(0), m, n, k, float(norm_eps),
                _native.dtype_code(x.dtype), stream,
            ),
            "linear_kstream_norm",
        )
    else:
        _native.check(
            library.tf_linear_kstream(
                x.data_ptr(), x.stride(0), weight.data_ptr(), weight.stride(0),
                output.data_ptr(), output.stride(0), m, n, k, _native.dtype_code(x.dtype),
                stream,
            ),
            "linear_kstream",
        )
    return output


def fold_norm_gain(weight: Tensor, gain: Tensor) -> Tensor:
    """``round(weight[n][k] * gain[k])`` in the weight's dtype: a projection
    weight carrying the gain of the RMSNorm before it, for the ``norm_eps``
    forms of :func:`linear_kstream` and :func:`linear_swiglu`."""

    if gain.ndim != 1 or gain.shape[0] != weight.shape[1]:
        raise ValueError("gain must have one element per weight column")
    return (weight.float() * gain.float()).to(weight.dtype).contiguous()


def linear_swiglu(x: Tensor, gate_up_weight: Tensor, *, output: Tensor | None = None,
                  k_split: bool = False, norm_eps: float | None = None) -> Tensor:
    """``swiglu(x @ gate.T, x @ up.T)`` for m <= 64 rows, with
    ``gate_up_weight`` stacking the gate rows over the up rows (``[2I, k]``)
    -- the stacked projection and its activation in one launch.  The default
    form is bit-identical to :func:`linear_stream` of the stacked weight
    followed by ``swiglu_gate_up``; ``k_split=True`` splits K over the
    wavefronts of workgroups of one or two 16-column tiles (bit-identical to
    :func:`linear_kstream` followed by ``swiglu_gate_up``).  ``norm_eps``
    (with ``k_split``): the RMSNorm of x's rows applied to both products
    before the activation, for a weight carrying the norm's gain
    (:func:`fold_norm_gain`).  Returns ``[m, I]`` in ``output`` (allocated
    when None)."""

    if not _native.is_available():
        raise RuntimeError(
            "the gfx950 kernel library is unavailable; build it with "
            "`python -m tensorforge_amd.build`"
        )
    if not linear_rows_supported(x, gate_up_weight) or gate_up_weight.shape[0] % 2:
        raise ValueError("linear_swiglu needs fp16/bf16 CUDA operands [m <= 64, k] and a "
                         "stacked [2I, k] weight with k % 32 == 0 and 16-byte aligned rows")
    if norm_eps is not None and not k_split:
        raise ValueError("the norm_eps form of linear_swiglu is the K-split one")
    m, k = x.shape
    inter = gate_up_weight.shape[0] // 2
    if output is None:
        output = torch.empty((m, inter), dtype=x.dtype, device=x.device)
    if (output.shape != (m, inter) or output.dtype != x.dtype or output.device != x.device
            or output.stride(1) != 1):
        raise ValueError("output must be [m, I] with contiguous rows, x's dtype and device")
    library = _native.library()
    args = (x.data_ptr(), x.stride(0), gate_up_weight.data_ptr(), gate_up_weight.stride(0),
            output.data_ptr(), output.stride(0), m, inter, k)
    if norm_eps is not None:
        _native.check(
            library.tf_linear_kswiglu_norm(*args, float(norm_eps), _native.dtype_code(x.dtype),
                                           _native.current_stream(x.device)),
            "linear_kswiglu_norm",
        )
        return output
    entry = "tf_linear_kswiglu" if k_split else "tf_linear_swiglu"
    _native.check(
        getattr(library, entry)(*args, _native.dtype_code(x.dtype),
                                _native.current_stream(x.device)),
        entry,
    )
    return output


def linear_partials_sum(partials: Tensor, *, dtype: torch.dtype | None = None,
                        output: Tensor | None = None) -> Tensor:
    """``round(partials.sum(0))`` into fp16/bf16 rows (one rounding)."""

    if partials.ndim != 3 or partials.dtype != torch.float32 or not partials.is_contiguous():
        raise ValueError("partials must be a contiguous fp32 [splits, m, n] tensor")
    splits, m, n = partials.shape
    if output is None:
        output = torch.empty((m, n), dtype=dtype or torch.bfloat16, device=partials.device)
    if (output.shape != (m, n) or output.stride(1) != 1 or output.device != partials.device
            or output.dtype not in (torch.float16, torch.bfloat16)):
        raise ValueError("output must be fp16/bf16 [m, n] with contiguous rows on the same device")
    _native.check(
        _native.library().tf_linear_partials_sum(
            partials.data_ptr(), splits, m, n, output.data_ptr(), output.stride(0),
            _native.dtype_code(output.dtype), _native.current_stream(partials.device),
        ),
        "linear_partials_sum",
    )
    return output
