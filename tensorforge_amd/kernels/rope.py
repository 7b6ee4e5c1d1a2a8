"""RoPE fused with the paged KV append (gfx950 HIP).

Replaces, in one launch per layer (``csrc/tf_rope_append.hip``), the
reference decode step's ``apply_batched_rotary_embedding``
(tensorforge/model/layers.py:57-69), the ``.contiguous()`` copies of the
rotated q/k and of v, and the masked one-token cache write
(tensorforge/runtime/decode_bucket.py:448-458); for prefill, the RoPE and
per-request ``write_layer`` loop of runtime/prefill.py:99-115 over all
prompts' tokens at once.
"""

from __future__ import annotations

import torch
from torch import Tensor

from tensorforge_amd import _native


def rope_paged_kv_append(
    qkv: Tensor,
    positions: Tensor,
    cos_table: Tensor,
    sin_table: Tensor,
    key_cache: Tensor,
    value_cache: Tensor,
    physical_blocks: Tensor,
    block_offsets: Tensor,
    active_mask: Tensor,
    *,
    query_heads: int,
    query_output: Tensor | None = None,
    key_output: Tensor | None = None,
) -> Tensor:
    """Rotate q and k of a fused projection and append k, v to the cache.

    ``qkv`` [batch, >= (Hq + 2 Hkv) * D] (rows may be strided; elements
    contiguous) holds the q, k and v heads of one token per lane;
    ``positions`` int64 [batch] index ``cos_table``/``sin_table``
    [max_position, D].  Returns the rotated query [batch, Hq, D] (written
    into ``query_output`` when given) and, when ``key_output`` [batch, Hkv, D]
    is given, the rotated keys of every lane.  Lanes with ``active_mask[b] != 0``
    store their rotated key and value at cache row
    ``(physical_blocks[b], block_offsets[b])``; other lanes store nothing.
    """

    if not _native.is_available():
        raise RuntimeError(
            "the gfx950 kernel library is unavailable; build it with "
            "`python -m tensorforge_amd.build`"
        )
    if key_cache.ndim != 4 or value_cache.shape != key_cache.shape:
        raise ValueError("cache tensors must share [blocks, block_size, kv_heads, head_dim]")
    num_blocks, block_size, kv_heads, head_dim = key_cache.shape
    if qkv.ndim != 2 or qkv.stride(1) != 1:
        raise ValueError("qkv must be [batch, features] with contiguous rows")
    if qkv.shape[1] < (query_heads + 2 * kv_heads) * head_dim:
        raise ValueError("qkv rows are shorter than the q, k and v heads")
    batch = qkv.shape[0]
    if cos_table.ndim != 2 or cos_table.shape[1] != head_dim or sin_table.shape != cos_table.shape:
        raise ValueError("cos/sin tables must share [max_position, head_dim]")
    if query_output is None:
        query_output = torch.empty((batch, query_heads, head_dim), dtype=qkv.dtype,
                                   device=qkv.device)
    if query_output.shape != (batch, query_heads, head_dim) or not query_output.is_contiguous():
        raise ValueError("query_output must be a contiguous [batch, query_heads, head_dim]")
    if key_output is not None and (key_output.shape != (batch, kv_heads, head_dim)
                                   or not key_output.is_contiguous()):
        raise ValueError("key_output must be a contiguous [batch, kv_heads, head_dim]")
    tensors = (qkv, positions, cos_table, sin_table, key_cache, value_cache, physical_blocks,
               block_offsets, active_mask, query_output) + (
                   () if key_output is None else (key_output,))
    if any(not tensor.is_cuda for tensor in tensors):
        raise ValueError("rope_paged_kv_append requires CUDA tensors")
    if any(not t.is_contiguous() for t in tensors[1:]):
        raise ValueError("rope_paged_kv_append requires contiguous control and cache tensors")
    if any(t.dtype != qkv.dtype for t in (cos_table, sin_table, key_cache, value_cache,
                                          query_output, *tensors[10:])):
        raise ValueError("qkv, tables, caches and output must share dtype")
    if qkv.dtype not in _native.DTYPE_CODES:
        raise TypeError(f"unsupported dtype: {qkv.dtype}")
    if positions.shape != (batch,) or positions.dtype != torch.int64:
        raise ValueError("positions must be int64 with shape [batch]")
    for name, tensor in (("physical_blocks", physical_blocks), ("block_offsets", block_offsets),
                         ("active_mask", active_mask)):
        if tensor.shape != (batch,) or tensor.dtype != torch.int32:
            raise ValueError(f"{name} must be int32 with shape [batch]")
    _native.check(
        _native.library().tf_rope_kv_append(
            qkv.data_ptr(), qkv.stride(0), positions.data_ptr(), cos_table.data_ptr(),
            sin_table.data_ptr(), cos_table.shape[0], query_output.data_ptr(),
            None if key_output is None else key_output.data_ptr(), key_cache.data_ptr(),
            value_cache.data_ptr(), physical_blocks.data_ptr(), block_offsets.data_ptr(),
            active_mask.data_ptr(), batch, query_heads, kv_heads, head_dim, num_blocks,
            block_size, _native.dtype_code(qkv.dtype),
            _native.current_stream(qkv.device),
        ),
        "rope_paged_kv_append",
    )
    return query_output
