"""RMSNorm, fused residual RMSNorm and SwiGLU on gfx950 HIP kernels.

Drop-in counterpart of ``tensorforge/kernels/triton_ops.py``: same names,
signatures, validation order, exception types and messages
(``:129-176``), caller-owned outputs returned by identity, and the
``selected_autotune_config`` / ``autotune_cache_size`` observability hooks
(``:263-295``).  The kernels are in ``csrc/tf_fused_ops.hip``.
"""

from __future__ import annotations

from typing import Any

import torch
from torch import Tensor

from tensorforge_amd import _native

_OPERATIONS = ("rms_norm", "residual_rms_norm", "swiglu")
# Launch shapes chosen per (operation, rows, columns, dtype), kept as the
# observable equivalent of the reference's autotune cache.
_LAUNCH_CACHE: dict[str, dict[tuple[Any, ...], dict[str, Any]]] = {
    name: {} for name in _OPERATIONS
}
_LAST_CONFIG: dict[str, dict[str, Any] | None] = {name: None for name in _OPERATIONS}


def is_hip_available() -> bool:
    return _native.is_available()


def _require_library() -> None:
    if not _native.is_available():
        raise RuntimeError(
            "the gfx950 kernel library is unavailable; build it with "
            "`python -m tensorforge_amd.build`"
        )


def _validate_common(inputs: Tensor, weight: Tensor | None = None) -> None:
    if not inputs.is_cuda:
        raise ValueError("HIP kernels require CUDA tensors")
    if inputs.dtype not in _native.DTYPE_CODES:
        raise TypeError(f"unsupported dtype: {inputs.dtype}")
    if inputs.numel() == 0 or inputs.ndim == 0:
        raise ValueError("inputs must be a non-empty tensor with a hidden dimension")
    if not inputs.is_contiguous():
        raise ValueError("inputs must be contiguous")
    if inputs.requires_grad and torch.is_grad_enabled():
        raise RuntimeError("TensorForge HIP kernels are inference-only")
    if weight is not None:
        if weight.shape != (inputs.shape[-1],):
            raise ValueError("weight must match the final input dimension")
        if weight.device != inputs.device or weight.dtype != inputs.dtype:
            raise ValueError("weight must share input device and dtype")
        if not weight.is_contiguous():
            raise ValueError("weight must be contiguous")


def _norm_launch_shape(inputs: Tensor) -> tuple[int, int]:
    columns = inputs.shape[-1]
    if columns > 16_384:
        raise ValueError("single-program RMSNorm supports at most 16,384 columns")
    return inputs.numel() // columns, columns


def _output_or_empty(output: Tensor | None, reference: Tensor, name: str) -> Tensor:
    if output is None:
        return torch.empty_like(reference)
    if (
        output.shape != reference.shape
        or output.dtype != reference.dtype
        or output.device != reference.device
        or not output.is_contiguous()
    ):
        raise ValueError(f"{name} must be contiguous and share input shape, dtype, and device")
    return output


def _norm_config(columns: int, dtype: torch.dtype, aligned: bool,
                 per_lane: int = 2) -> dict[str, Any]:
    """The norm kernels' launch shape, as ``launch_norm`` in
    csrc/tf_fused_ops.hip picks it: 16-byte vectors where the row and every
    pointer allow, and the fewest of 1, 2, 4 or 8 wavefronts (the
    reference's autotune set, triton_ops.py:28-33) that leave each lane at
    most ``per_lane`` vectors (1 when summing split-K partials)."""

    vector = 16 // torch.empty((), dtype=dtype).element_size()
    vectorised = aligned and columns % vector == 0
    width = vector if vectorised else 1
    units = columns // width
    warps = 1
    while warps < 8 and warps * 64 * per_lane < units:
        warps *= 2
    return {"kwargs": {"VECTOR": width}, "num_warps": warps, "wave_size": 64}


def _record(operation: str, key: tuple[Any, ...], config: dict[str, Any]) -> None:
    _LAUNCH_CACHE[operation].setdefault(key, config)
    _LAST_CONFIG[operation] = config


def _aligned(*tensors: Tensor) -> bool:
    return all(tensor.data_ptr() % 16 == 0 for tensor in tensors)


def embedding_rms_norm(
    token_state: Tensor,
    source_lanes: Tensor,
    host_tokens: Tensor,
    embedding: Tensor,
    weight: Tensor,
    eps: float,
    *,
    x_output: Tensor,
    norm_output: Tensor,
) -> tuple[Tensor, Tensor]:
    """A decode step's input rows and first RMSNorm in one launch: row b
    embeds ``token_state[source_lanes[b]]`` when ``source_lanes[b] >= 0``
    and ``host_tokens[b]`` otherwise (int64; indices clamped to the arrays),
    writing the embedding row to ``x_output`` and its RMSNorm to
    ``norm_output`` -- bit-identical to ``F.embedding`` of those ids followed
    by :func:`rms_norm` (reference: runtime/decode_bucket.py:427-440,
    triton_ops.py:179-205)."""

    _require_library()
    rows = source_lanes.shape[0]
    vocab, columns = embedding.shape
    for name, t in (("token_state", token_state), ("source_lanes", source_lanes),
                    ("host_tokens", host_tokens)):
        if t.dtype != torch.int64 or not t.is_cuda or not t.is_contiguous() or t.ndim != 1:
            raise ValueError(f"{name} must be a contiguous 1-D int64 CUDA tensor")
    if host_tokens.shape[0] != rows or token_state.shape[0] < 1:
        raise ValueError("host_tokens must have one entry per row and token_state at least one")
    if eps <= 0:
        raise ValueError("eps must be positive")
    _validate_common(embedding, weight)
    for name, t in (("x_output", x_output), ("norm_output", norm_output)):
        if (t.shape != (rows, columns) or t.dtype != embedding.dtype or not t.is_contiguous()
                or t.device != embedding.device):
            raise ValueError(f"{name} must be a contiguous [rows, hidden] tensor like the table")
    _native.check(
        _native.library().tf_embedding_rms_norm(
            token_state.data_ptr(), token_state.shape[0], source_lanes.data_ptr(),
            host_tokens.data_ptr(), embedding.data_ptr(), vocab, weight.data_ptr(),
            x_output.data_ptr(), norm_output.data_ptr(), rows, columns, eps,
            _native.dtype_code(embedding.dtype), _native.current_stream(embedding.device),
        ),
        "embedding_rms_norm",
    )
    return x_output, norm_output


def rms_norm(
    inputs: Tensor,
    weight: Tensor,
    eps: float = 1e-6,
    *,
    output: Tensor | None = None,
) -> Tensor:
    """RMSNorm over the last dimension (reference: triton_ops.py:179-205)."""

    _require_library()
    _validate_common(inputs, weight)
    if eps <= 0:
        raise ValueError("eps must be positive")
    rows, columns = _norm_launch_shape(inputs)
    output = _output_or_empty(output, inputs, "output")
    _native.check(
        _native.library().tf_rms_norm(
            inputs.data_ptr(),
            weight.data_ptr(),
            output.data_ptr(),
            rows,
            columns,
            eps,
            _native.dtype_code(inputs.dtype),
            _native.current_stream(inputs.device),
        ),
        "rms_norm",
    )
    _record(
        "rms_norm",
        (rows, columns, inputs.dtype),
        _norm_config(columns, inputs.dtype, _aligned(inputs, weight, output)),
    )
    return output


def residual_rms_norm(
    inputs: Tensor,
    residual: Tensor,
    weight: Tensor,
    eps: float = 1e-6,
    *,
    residual_output: Tensor | None = None,
    norm_output: Tensor | None = None,
) -> tuple[Tensor, Tensor]:
    """Fuse residual addition and RMSNorm (reference: triton_ops.py:208-243).

    ``residual_output`` is the rounded sum; the norm is taken of the fp32 sum
    (the reference kernel's semantics, triton_ops.py:89-97).
    """

    _require_library()
    _validate_common(inputs, weight)
    _validate_common(residual)
    if residual.shape != inputs.shape or residual.dtype != inputs.dtype:
        raise ValueError("residual must share input shape and dtype")
    if residual.device != inputs.device:
        raise ValueError("residual must share input device")
    if eps <= 0:
        raise ValueError("eps must be positive")
    rows, columns = _norm_launch_shape(inputs)
    residual_output = _output_or_empty(residual_output, inputs, "residual_output")
    norm_output = _output_or_empty(norm_output, inputs, "norm_output")
    _native.check(
        _native.library().tf_residual_rms_norm(
            inputs.data_ptr(),
            residual.data_ptr(),
            weight.data_ptr(),
            residual_output.data_ptr(),
            norm_output.data_ptr(),
            rows,
            columns,
            eps,
            _native.dtype_code(inputs.dtype),
            _native.current_stream(inputs.device),
        ),
        "residual_rms_norm",
    )
    _record(
        "residual_rms_norm",
        (rows, columns, inputs.dtype),
        _norm_config(
            columns,
            inputs.dtype,
            _aligned(inputs, residual, weight, residual_output, norm_output),
        ),
    )
    return residual_output, norm_output


def residual_rms_norm_partials(
    partials: Tensor,
    residual: Tensor,
    weight: Tensor,
    eps: float = 1e-6,
    *,
    residual_output: Tensor | None = None,
    norm_output: Tensor | None = None,
) -> tuple[Tensor, Tensor]:
    """:func:`residual_rms_norm` whose inputs are the rounded sum of fp32
    split-K partials ``[splits, rows, columns]`` (``linear_partials``): the
    projection's K-slice sum is fused into the norm's row read, so the
    projection output is never written in the storage type."""

    _require_library()
    _validate_common(residual, weight)
    if partials.dtype != torch.float32 or partials.ndim != 3 or not partials.is_contiguous():
        raise ValueError("partials must be a contiguous fp32 [splits, rows, columns] tensor")
    if partials.device != residual.device:
        raise ValueError("partials must share the residual's device")
    rows, columns = _norm_launch_shape(residual)
    if partials.shape[1:] != (rows, columns):
        raise ValueError("partials must be [splits, rows, columns] of the residual's rows")
    if eps <= 0:
        raise ValueError("eps must be positive")
    residual_output = _output_or_empty(residual_output, residual, "residual_output")
    norm_output = _output_or_empty(norm_output, residual, "norm_output")
    _native.check(
        _native.library().tf_residual_rms_norm_partials(
            partials.data_ptr(),
            partials.shape[0],
            residual.data_ptr(),
            weight.data_ptr(),
            residual_output.data_ptr(),
            norm_output.data_ptr(),
            rows,
            columns,
            eps,
            _native.dtype_code(residual.dtype),
            _native.current_stream(residual.device),
        ),
        "residual_rms_norm_partials",
    )
    return residual_output, norm_output


def swiglu(gate: Tensor, up: Tensor, *, output: Tensor | None = None) -> Tensor:
    """Fuse SiLU and gating after the two projections (reference: triton_ops.py:246-260)."""

    _require_library()
    _validate_common(gate)
    _validate_common(up)
    if up.shape != gate.shape or up.dtype != gate.dtype or up.device != gate.device:
        raise ValueError("gate and up tensors must share shape, dtype, and device")
    output = _output_or_empty(output, gate, "output")
    numel = gate.numel()
    _native.check(
        _native.library().tf_swiglu(
            gate.data_ptr(),
            up.data_ptr(),
            output.data_ptr(),
            numel,
            _native.dtype_code(gate.dtype),
            _native.current_stream(gate.device),
        ),
        "swiglu",
    )
    vector = 16 // gate.element_size()
    width = vector if numel % vector == 0 and _aligned(gate, up, output) else 1
    blocks = min((numel // width + 255) // 256, 8192)
    _record(
        "swiglu",
        (numel, gate.dtype),
        {"kwargs": {"BLOCK_SIZE": 256 * width, "VECTOR": width, "BLOCKS": blocks},
         "num_warps": 4, "wave_size": 64},
    )
    return output


def swiglu_gate_up(gate_up: Tensor, *, output: Tensor | None = None) -> Tensor:
    """SwiGLU over a fused gate|up projection ``[rows, >= 2F]`` (rows may be
    strided): ``output[r] = silu(gate_up[r, :F]) * gate_up[r, F:2F]`` with
    ``F = output.shape[-1]`` (or half the row length).  The arithmetic of
    :func:`swiglu`; no reference counterpart (the reference projects gate and
    up separately, model/layers.py:146-158)."""

    _require_library()
    if gate_up.ndim != 2 or gate_up.stride(1) != 1:
        raise ValueError("gate_up must be [rows, features] with contiguous rows")
    if not gate_up.is_cuda:
        raise ValueError("swiglu_gate_up requires CUDA tensors")
    if gate_up.dtype not in _native.DTYPE_CODES:
        raise TypeError(f"unsupported dtype: {gate_up.dtype}")
    rows = gate_up.shape[0]
    columns = output.shape[-1] if output is not None else gate_up.shape[1] // 2
    if 2 * columns > gate_up.shape[1]:
        raise ValueError("gate_up rows are shorter than twice the output width")
    if output is None:
        output = torch.empty((rows, columns), dtype=gate_up.dtype, device=gate_up.device)
    if (output.shape != (rows, columns) or output.dtype != gate_up.dtype
            or output.device != gate_up.device or output.stride(1) != 1):
        raise ValueError("output must be [rows, F] with contiguous rows, gate_up's dtype and device")
    _native.check(
        _native.library().tf_swiglu_rows(
            gate_up.data_ptr(), gate_up.stride(0), output.data_ptr(), output.stride(0), rows,
            columns, _native.dtype_code(gate_up.dtype), _native.current_stream(gate_up.device),
        ),
        "swiglu_gate_up",
    )
    return output


def argmax_rows(logits: Tensor, *, output: Tensor | None = None) -> Tensor:
    """``torch.argmax(logits, dim=-1)`` of a ``[rows, columns]`` matrix with
    contiguous rows (rows may be strided) into int64 ``output`` -- greedy
    sampling as the reference's scheduler applies it
    (scheduler/continuous.py:265-275): the first index of the largest value,
    a NaN counting as larger than every number."""

    _require_library()
    if logits.ndim != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be [rows, columns] with contiguous rows")
    if not logits.is_cuda:
        raise ValueError("argmax_rows requires CUDA tensors")
    if logits.dtype not in _native.DTYPE_CODES:
        raise TypeError(f"unsupported dtype: {logits.dtype}")
    rows, columns = logits.shape
    if columns < 1:
        raise ValueError("argmax of an empty row")
    if output is None:
        output = torch.empty(rows, dtype=torch.int64, device=logits.device)
    if (output.shape != (rows,) or output.dtype != torch.int64 or output.device != logits.device
            or (rows > 1 and output.stride(0) != 1)):
        raise ValueError("output must be a contiguous int64 [rows] tensor on the logits' device")
    _native.check(
        _native.library().tf_argmax_rows(
            logits.data_ptr(), logits.stride(0) if rows > 1 else columns, rows, columns,
            _native.dtype_code(logits.dtype), output.data_ptr(),
            _native.current_stream(logits.device),
        ),
        "argmax_rows",
    )
    return output


def selected_autotune_config(operation: str) -> dict[str, Any] | None:
    """Most recent launch configuration of ``operation`` (reference: triton_ops.py:263-283)."""

    if operation not in _LAST_CONFIG:
        raise ValueError(f"unknown operation: {operation}")
    return _LAST_CONFIG[operation]


def autotune_cache_size(operation: str) -> int:
    """Number of distinct launch shapes seen (reference: triton_ops.py:286-295)."""

    if operation not in _LAUNCH_CACHE:
        raise ValueError(f"unknown operation: {operation}")
    return len(_LAUNCH_CACHE[operation])
