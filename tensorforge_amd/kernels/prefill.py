"""Causal GQA attention over packed prompts (``csrc/tf_prefill_attention.hip``).

Prefill packs the tokens of all admitted prompts into one stream with no
padding.  ``prefill_attention`` attends every token causally within its own
prompt in one launch, where the reference pads the prompts into one batch
and runs a masked SDPA (tensorforge/runtime/prefill.py:84-88, 109-118).
The work list -- 64-token query blocks, heaviest first -- is built on the
host from the prompt lengths once per prefill and reused by every layer.
"""

from __future__ import annotations

import numpy as np
import torch
from torch import Tensor

from tensorforge_amd import _native

TILE = 64  # query tokens per work item (four wavefronts of 16)


def prefill_attention_supported(dtype: torch.dtype, query_heads: int, kv_heads: int,
                                head_dim: int) -> bool:
    """Whether the kernel serves this geometry (else use a library SDPA)."""

    group = query_heads // kv_heads if kv_heads > 0 else 0
    return (dtype in (torch.float16, torch.bfloat16) and head_dim in (32, 64, 128)
            and kv_heads > 0 and query_heads % kv_heads == 0 and 1 <= group <= 16
            and group & (group - 1) == 0)


def prefill_tiles(lengths: list[int]) -> np.ndarray:
    """[blocks, 3] int32 rows (first query token, prompt start, prompt end) of
    the packed prompts' TILE-token query blocks, most key tokens first."""

    rows = []
    start = 0
    for length in lengths:
        if length <= 0:
            raise ValueError("prompt lengths must be positive")
        for i0 in range(start, start + length, TILE):
            rows.append((i0, start, start + length))
        start += length
    tiles = np.asarray(rows, dtype=np.int32).reshape(-1, 3)
    work = np.minimum(tiles[:, 0] + TILE, tiles[:, 2]) - tiles[:, 1]
    return np.ascontiguousarray(tiles[np.argsort(-work, kind="stable")])


def prefill_attention(q: Tensor, k: Tensor, v: Tensor, tiles: Tensor, *, query_heads: int,
                      kv_heads: int, scale: float, output: Tensor,
                      heads_per_wave: int = 0) -> Tensor:
    """``output[t] = softmax(scale q[t] K^T) V`` over the keys of ``t``'s own
    prompt up to ``t`` (GQA: query head h reads kv head h // (Hq / Hkv)).

    ``q`` / ``output`` are ``[T, query_heads * head_dim]`` row-major token
    rows, ``k`` / ``v`` ``[T, kv_heads * head_dim]`` (rows may be strided,
    e.g. a column slice of the fused QKV projection); ``tiles`` comes from
    :func:`prefill_tiles` (int32, on the device).
    """

    if not _native.is_available():
        raise RuntimeError(
            "the gfx950 kernel library is unavailable; build it with "
            "`python -m tensorforge_amd.build`"
        )
    tokens = q.shape[0]
    head_dim = q.shape[1] // query_heads
    if not prefill_attention_supported(q.dtype, query_heads, kv_heads, head_dim):
        raise ValueError("prefill attention needs fp16/bf16, head_dim 32/64/128 and a "
                         "power-of-two group of at most 16 query heads per kv head")
    for name, tensor, width in (("q", q, query_heads * head_dim),
                                ("k", k, kv_heads * head_dim),
                                ("v", v, kv_heads * head_dim),
                                ("output", output, query_heads * head_dim)):
        if (not tensor.is_cuda or tensor.ndim != 2 or tensor.shape != (tokens, width)
                or tensor.stride(1) != 1 or tensor.dtype != q.dtype):
            raise ValueError(f"{name} must be a CUDA [{tokens}, {width}] tensor with "
                             "contiguous rows and q's dtype")
    if tiles.dtype != torch.int32 or tiles.ndim != 2 or tiles.shape[1] != 3 or not tiles.is_cuda:
        raise ValueError("tiles must be a CUDA int32 [n, 3] tensor from prefill_tiles")
    _native.check(
        _native.library().tf_prefill_attention(
            q.data_ptr(), q.stride(0), k.data_ptr(), k.stride(0), v.data_ptr(), v.stride(0),
            output.data_ptr(), output.stride(0), tiles.data_ptr(), tiles.shape[0], query_heads,
            kv_heads, head_dim, scale, heads_per_wave, _native.dtype_code(q.dtype),
            _native.current_stream(q.device),
        ),
        "prefill_attention",
    )
    return output
