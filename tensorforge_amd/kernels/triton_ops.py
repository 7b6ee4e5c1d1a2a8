"""RMSNorm, residual RMSNorm and SwiGLU under the reference's module path.

``tensorforge/kernels/triton_ops.py`` is where the reference's runtime and
benchmarks import these from (``runtime/decode_bucket.py:22``,
``runtime/triton_model.py:11``, ``benchmark/kernel_benchmark.py:27-32``).
This module exposes the gfx950 implementation (``tensorforge_amd.kernels.ops``)
under the same names, so a caller changes only the package prefix.
``is_triton_available`` keeps the reference's hook name (``:129-130``); it
reports whether the gfx950 library is loadable.
"""

from __future__ import annotations

from tensorforge_amd.kernels.ops import (
    autotune_cache_size,
    is_hip_available,
    residual_rms_norm,
    rms_norm,
    selected_autotune_config,
    swiglu,
)


def is_triton_available() -> bool:
    """The reference's availability hook (triton_ops.py:129-130): True when
    the gfx950 kernel library is built and loadable."""

    return is_hip_available()


__all__ = [
    "autotune_cache_size",
    "is_triton_available",
    "residual_rms_norm",
    "rms_norm",
    "selected_autotune_config",
    "swiglu",
]
