"""Seeded synthetic workloads of the benchmark configurations and their byte models.

Inputs are generated on the CPU with ``torch.Generator().manual_seed(seed)``
and copied to the device afterwards, so a CPU checker and the GPU path see
bit-identical tensors.  Block tables are carved from a seeded random
permutation of the page pool, so logical neighbours are never physical
neighbours (the reference allocator hands out the lowest free page,
cache/paged.py:134-137,168; the permutation makes the workloads harder).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import Tensor


@dataclass
class DecodeAttentionCase:
    """Inputs of one paged decode-attention call (all tensors on one device)."""

    query: Tensor  # [batch, query_heads, head_dim]
    key_cache: Tensor  # [num_blocks, block_size, kv_heads, head_dim]
    value_cache: Tensor
    block_tables: Tensor  # [batch, table_width] int32, -1 padded
    context_lengths: Tensor  # [batch] int32
    scale: float

    @property
    def lengths(self) -> list[int]:
        return [int(v) for v in self.context_lengths.cpu().tolist()]

    def to(self, device: torch.device | str) -> DecodeAttentionCase:
        return DecodeAttentionCase(
            query=self.query.to(device),
            key_cache=self.key_cache.to(device),
            value_cache=self.value_cache.to(device),
            block_tables=self.block_tables.to(device),
            context_lengths=self.context_lengths.to(device),
            scale=self.scale,
        )


def make_decode_attention_case(
    lengths: list[int],
    *,
    query_heads: int,
    kv_heads: int,
    head_dim: int,
    block_size: int,
    dtype: torch.dtype,
    seed: int = 0,
    table_width: int | None = None,
    extra_pages: int = 0,
) -> DecodeAttentionCase:
    """Random N(0,1) q/K/V over a page pool of exactly sum(ceil(ctx/page)) pages
    (plus ``extra_pages``), tables carved from a seeded permutation of it."""

    generator = torch.Generator().manual_seed(seed)
    pages = [(max(ctx, 0) + block_size - 1) // block_size for ctx in lengths]
    pool = max(sum(pages) + extra_pages, 1)
    width = table_width if table_width is not None else max(max(pages, default=1), 1)
    permutation = torch.randperm(pool, generator=generator)
    tables = torch.full((len(lengths), width), -1, dtype=torch.int32)
    cursor = 0
    for row, count in enumerate(pages):
        tables[row, :count] = permutation[cursor:cursor + count].to(torch.int32)
        cursor += count
    query = torch.randn(len(lengths), query_heads, head_dim, generator=generator).to(dtype)
    key_cache = torch.randn(pool, block_size, kv_heads, head_dim, generator=generator).to(dtype)
    value_cache = torch.randn(pool, block_size, kv_heads, head_dim, generator=generator).to(dtype)
    return DecodeAttentionCase(
        query=query,
        key_cache=key_cache,
        value_cache=value_cache,
        block_tables=tables,
        context_lengths=torch.tensor(lengths, dtype=torch.int32),
        scale=head_dim**-0.5,
    )


def tinyllama_decode_lengths(seed: int = 0, batch: int = 64, padded: int = 8,
                             min_context: int = 128, max_context: int = 2048) -> list[int]:
    """Config 2 lengths: ``batch`` rows uniform in [min, max] plus ``padded``
    zero-length rows (64 + 8 = 72 rows)."""

    generator = torch.Generator().manual_seed(seed)
    active = torch.randint(min_context, max_context + 1, (batch,), generator=generator)
    return [int(v) for v in active.tolist()] + [0] * padded


def tinyllama_decode_case(seed: int = 0, dtype: torch.dtype = torch.bfloat16) -> DecodeAttentionCase:
    """Config 2: TinyLlama geometry (32 q heads, 4 kv heads, head_dim 64),
    page 16, bf16, table width 128 (2048 tokens)."""

    lengths = tinyllama_decode_lengths(seed)
    return make_decode_attention_case(
        lengths,
        query_heads=32,
        kv_heads=4,
        head_dim=64,
        block_size=16,
        dtype=dtype,
        seed=seed + 1,
        table_width=2048 // 16,
    )


def llama3_long_context_case(seed: int = 0, dtype: torch.dtype = torch.bfloat16) -> DecodeAttentionCase:
    """Config 3: Llama-3-8B geometry (32/8 heads, head_dim 128), contexts
    8k/16k/24k/32k, page 16."""

    lengths = [8192, 16384, 24576, 32768]
    return make_decode_attention_case(
        lengths,
        query_heads=32,
        kv_heads=8,
        head_dim=128,
        block_size=16,
        dtype=dtype,
        seed=seed + 1,
        table_width=32768 // 16,
    )


def decode_attention_bytes(lengths: list[int], query_heads: int, kv_heads: int, head_dim: int,
                           block_size: int, element_size: int) -> int:
    """Algorithmic HBM bytes of one decode-attention call over the active rows.

    q in + out: 2 * Hq * D * e per row; K + V: ctx * Hkv * D * 2 * e; block
    table entries plus the length: (ceil(ctx / page) + 1) * 4.  This is the
    logical byte model of benchmark/attention_benchmark.py:148-161; split
    partials are implementation overhead and are not counted.
    """

    total = 0
    for ctx in lengths:
        if ctx <= 0:
            continue
        total += 2 * query_heads * head_dim * element_size
        total += ctx * kv_heads * head_dim * 2 * element_size
        total += ((ctx + block_size - 1) // block_size + 1) * 4
    return total


def decode_attention_flops(lengths: list[int], query_heads: int, head_dim: int) -> int:
    """2 * Hq * D flops for q.K plus the same for P.V per token
    (benchmark/attention_benchmark.py:154-161)."""

    return sum(4 * query_heads * head_dim * ctx for ctx in lengths if ctx > 0)


def rms_norm_bytes(rows: int, columns: int, element_size: int, residual: bool) -> int:
    """(2T + 1) H e for RMSNorm, (4T + 1) H e with the residual
    (benchmark/kernel_benchmark.py:144-158)."""

    per_row = 4 if residual else 2
    return (per_row * rows + 1) * columns * element_size


def swiglu_bytes(numel: int, element_size: int) -> int:
    """3 N e: gate and up read, output written."""

    return 3 * numel * element_size


def kv_append_bytes(tokens: int, kv_heads: int, head_dim: int, element_size: int) -> int:
    """K and V rows read and written plus 12 bytes of control per token."""

    return 2 * (2 * tokens * kv_heads * head_dim * element_size) + 12 * tokens


def decode_step_bytes(config, sum_context: int, batch: int, element_size: int) -> dict:
    """Algorithmic HBM bytes of one decode step of a Llama-style decoder
    (``tensorforge_amd.decode.DecoderConfig``) over ``batch`` rows whose
    contexts sum to ``sum_context`` tokens (the new token included): every
    layer's weights once (qkv, o, gate|up, down and the two norm gains), the
    rows' cached K and V read and the new token's K and V written, the LM
    head and final norm once, the embedding rows read and the logits
    written.  Activations passed between kernels are not counted (a fused
    step need not write them)."""

    e = element_size
    h, f, d = config.hidden_size, config.intermediate_size, config.head_dim
    hq, hkv = config.num_attention_heads, config.num_key_value_heads
    layers = config.num_hidden_layers
    weights = ((hq + 2 * hkv) * d * h + h * hq * d + 2 * f * h + h * f + 2 * h) * e
    kv_read = sum_context * hkv * d * 2 * e
    kv_write = batch * hkv * d * 2 * e
    head = (config.vocab_size * h + h) * e
    io = batch * h * e + batch * config.vocab_size * e
    return {"layer_weights": layers * weights, "kv_read": layers * kv_read,
            "kv_write": layers * kv_write, "lm_head": head, "embedding_and_logits": io,
            "total": layers * (weights + kv_read + kv_write) + head + io}
