"""Capture-safe masked writes into paged KV storage (gfx950 HIP).

Drop-in counterpart of ``tensorforge/kernels/triton_cache.py``: same name,
signature, validation order and messages (``:68-113``).  The copy is a
byte-exact row scatter (``csrc/tf_cache_write.hip``) on torch's current
stream.
"""

from __future__ import annotations

import torch
from torch import Tensor

from tensorforge_amd import _native


def paged_kv_write_token(
    keys: Tensor,
    values: Tensor,
    key_cache: Tensor,
    value_cache: Tensor,
    physical_blocks: Tensor,
    block_offsets: Tensor,
    active_mask: Tensor,
) -> None:
    """Write at most one KV token per batch lane using device-side destinations.

    Lane ``b`` with ``active_mask[b] != 0`` stores ``keys[b]``/``values[b]`` at
    ``cache[physical_blocks[b], block_offsets[b]]``; masked lanes store
    nothing (``triton_cache.py:41-63``).  Destinations outside the cache are
    skipped rather than written out of bounds.
    """

    if not _native.is_available():
        raise RuntimeError(
            "the gfx950 kernel library is unavailable; build it with "
            "`python -m tensorforge_amd.build`"
        )
    if keys.ndim != 3 or values.shape != keys.shape:
        raise ValueError("keys and values must share [batch, kv_heads, head_dim]")
    if key_cache.ndim != 4 or value_cache.shape != key_cache.shape:
        raise ValueError("cache tensors must share [blocks, block_size, kv_heads, head_dim]")
    if keys.shape[1:] != key_cache.shape[2:]:
        raise ValueError("source and cache KV head dimensions must match")
    tensors = (
        keys,
        values,
        key_cache,
        value_cache,
        physical_blocks,
        block_offsets,
        active_mask,
    )
    if any(not tensor.is_cuda for tensor in tensors):
        raise ValueError("paged KV writes require CUDA tensors")
    if any(not tensor.is_contiguous() for tensor in tensors):
        raise ValueError("paged KV writes require contiguous tensors")
    if (
        values.dtype != keys.dtype
        or key_cache.dtype != keys.dtype
        or value_cache.dtype != keys.dtype
    ):
        raise ValueError("source and cache tensors must share dtype")
    if keys.dtype not in _native.DTYPE_CODES:
        raise TypeError(f"unsupported dtype: {keys.dtype}")
    batch = keys.shape[0]
    for name, tensor in (
        ("physical_blocks", physical_blocks),
        ("block_offsets", block_offsets),
        ("active_mask", active_mask),
    ):
        if tensor.shape != (batch,) or tensor.dtype != torch.int32:
            raise ValueError(f"{name} must be int32 with shape [batch]")
    num_blocks, block_size, kv_heads, head_dim = key_cache.shape
    _native.check(
        _native.library().tf_paged_kv_write_token(
            keys.data_ptr(),
            values.data_ptr(),
            key_cache.data_ptr(),
            value_cache.data_ptr(),
            physical_blocks.data_ptr(),
            block_offsets.data_ptr(),
            active_mask.data_ptr(),
            batch,
            kv_heads,
            head_dim,
            num_blocks,
            block_size,
            _native.dtype_code(keys.dtype),
            _native.current_stream(keys.device),
        ),
        "paged_kv_write_token",
    )


def paged_kv_write_slots(
    keys: Tensor,
    values: Tensor,
    key_cache: Tensor,
    value_cache: Tensor,
    slot_mapping: Tensor,
) -> None:
    """Scatter T token rows into pages through an int64 slot mapping.

    ``slot_mapping[t] = physical_block * block_size + offset``; negative
    slots (padded lanes) are skipped.  This is the multi-token append of
    ``PagedKVCache.write_layer`` (``cache/paged.py:221-235``) as one launch.
    """

    if not _native.is_available():
        raise RuntimeError(
            "the gfx950 kernel library is unavailable; build it with "
            "`python -m tensorforge_amd.build`"
        )
    if keys.ndim != 3 or values.shape != keys.shape:
        raise ValueError("keys and values must share [tokens, kv_heads, head_dim]")
    if key_cache.ndim != 4 or value_cache.shape != key_cache.shape:
        raise ValueError("cache tensors must share [blocks, block_size, kv_heads, head_dim]")
    if keys.shape[1:] != key_cache.shape[2:]:
        raise ValueError("source and cache KV head dimensions must match")
    tensors = (keys, values, key_cache, value_cache, slot_mapping)
    if any(not tensor.is_cuda for tensor in tensors):
        raise ValueError("paged KV writes require CUDA tensors")
    if any(not tensor.is_contiguous() for tensor in tensors):
        raise ValueError("paged KV writes require contiguous tensors")
    if (
        values.dtype != keys.dtype
        or key_cache.dtype != keys.dtype
        or value_cache.dtype != keys.dtype
    ):
        raise ValueError("source and cache tensors must share dtype")
    if keys.dtype not in _native.DTYPE_CODES:
        raise TypeError(f"unsupported dtype: {keys.dtype}")
    tokens = keys.shape[0]
    if slot_mapping.shape != (tokens,) or slot_mapping.dtype != torch.int64:
        raise ValueError("slot_mapping must be int64 with shape [tokens]")
    num_blocks, block_size, kv_heads, head_dim = key_cache.shape
    _native.check(
        _native.library().tf_paged_kv_write_slots(
            keys.data_ptr(),
            values.data_ptr(),
            key_cache.data_ptr(),
            value_cache.data_ptr(),
            slot_mapping.data_ptr(),
            tokens,
            kv_heads,
            head_dim,
            num_blocks,
            block_size,
            _native.dtype_code(keys.dtype),
            _native.current_stream(keys.device),
        ),
        "paged_kv_write_slots",
    )
