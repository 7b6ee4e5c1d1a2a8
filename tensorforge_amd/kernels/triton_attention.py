"""The attention entry points under the reference's module path and names.

``tensorforge/kernels/triton_attention.py`` is where the reference's
runtime imports decode attention from (``runtime/decode_bucket.py:17-20``,
``runtime/batched_decode.py:13``, ``runtime/paged_decode.py:12``,
``benchmark/attention_benchmark.py:23-27``).  This module exposes the
gfx950 implementation (``tensorforge_amd.kernels.attention``) under the same
module and function names, so a caller changes only the package prefix.
``is_triton_attention_available`` keeps the reference's hook name
(``:322-323``); it reports whether the gfx950 library is loadable.
"""

from __future__ import annotations

from tensorforge_amd.kernels.attention import (
    PagedAttentionWorkspace,
    is_hip_attention_available,
    paged_gqa_decode_attention,
    selected_attention_autotune_config,
)


def is_triton_attention_available() -> bool:
    """The reference's availability hook (triton_attention.py:322-323):
    True when the gfx950 attention library is built and loadable."""

    return is_hip_attention_available()


__all__ = [
    "PagedAttentionWorkspace",
    "is_triton_attention_available",
    "paged_gqa_decode_attention",
    "selected_attention_autotune_config",
]
