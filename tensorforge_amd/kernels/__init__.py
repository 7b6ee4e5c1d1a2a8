"""gfx950 HIP kernels of the batched decode hot path.

Public surface of ``tensorforge/kernels/__init__.py:3-19`` (minus the
PyTorch oracles, which stay test infrastructure) plus the attention entry
points the reference exposes from ``triton_attention.py``.
"""

from tensorforge_amd.kernels.attention import (
    PagedAttentionWorkspace,
    is_hip_attention_available,
    paged_gqa_decode_attention,
    selected_attention_autotune_config,
    selected_attention_launch,
    set_attention_split_size,
)
from tensorforge_amd.kernels.cache_write import paged_kv_write_slots, paged_kv_write_token
from tensorforge_amd.kernels.linear import (
    fold_norm_gain,
    linear_partials,
    linear_partials_sum,
    linear_kstream,
    linear_stream,
    linear_swiglu,
    linear_rows,
    linear_rows_supported,
)
from tensorforge_amd.kernels.ops import (
    argmax_rows,
    autotune_cache_size,
    is_hip_available,
    embedding_rms_norm,
    residual_rms_norm,
    rms_norm,
    selected_autotune_config,
    swiglu,
    swiglu_gate_up,
)
from tensorforge_amd.kernels.rope import rope_paged_kv_append

__all__ = [
    "PagedAttentionWorkspace",
    "argmax_rows",
    "autotune_cache_size",
    "is_hip_attention_available",
    "is_hip_available",
    "linear_partials",
    "linear_partials_sum",
    "linear_kstream",
    "linear_stream",
    "linear_swiglu",
    "linear_rows",
    "linear_rows_supported",
    "paged_gqa_decode_attention",
    "paged_kv_write_slots",
    "paged_kv_write_token",
    "embedding_rms_norm",
    "fold_norm_gain",
    "residual_rms_norm",
    "rms_norm",
    "rope_paged_kv_append",
    "selected_attention_autotune_config",
    "selected_attention_launch",
    "selected_autotune_config",
    "set_attention_split_size",
    "swiglu",
    "swiglu_gate_up",
]
