"""Seeded sweep of the fused ops and the paged KV writes over drawn shapes.

Norms and SwiGLU: fp32 / fp16 / bf16, 1-300 rows, 1-16384 columns (odd
widths, widths that are no multiple of a wavefront's vector, and widths
that take every wavefront count of the launch), eps drawn, weights or
inputs with a constant row.  Checked against the oracle with the
reference's per-dtype tolerance (tests/test_triton_kernels.py:21-26 of the
reference), the residual sum bit for bit.

KV writes: fp32 / fp16 / bf16, 1-8 kv heads, head_dim 1-160, pages of
1-64 tokens, 1-300 tokens, the one-token-per-lane writer with random
inactive lanes and the slot-mapping writer with random padded (-1) slots
and slots in any order.  Checked bit for bit against the oracle scatter.
"""

from __future__ import annotations

import random

import pytest
import torch

from helpers import REFERENCE_TOLERANCE, assert_bit_exact, assert_close
from oracle.reference import (
    paged_kv_write_slots_reference,
    paged_kv_write_token_reference,
    residual_rms_norm_reference,
    rms_norm_reference,
    swiglu_reference,
)
from tensorforge_amd.kernels import (
    paged_kv_write_slots,
    paged_kv_write_token,
    residual_rms_norm,
    rms_norm,
    swiglu,
)

CASES = 24
DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def draw_op(seed: int) -> dict:
    rng = random.Random(7907 * seed + 11)
    return {
        "dtype": rng.choice(DTYPES),
        "rows": rng.choice([1, 2, 3, 17, 64, 256, rng.randint(1, 300)]),
        "cols": rng.choice([1, 5, 63, 64, 65, 511, 2048, 4095, 5632, 8192, 16384,
                            rng.randint(1, 16384)]),
        "eps": rng.choice([1e-6, 1e-5, 1e-3]),
        "constant_row": rng.random() < 0.3,
    }


def draw_kv(seed: int) -> dict:
    rng = random.Random(6007 * seed + 29)
    block = rng.choice([1, 5, 8, 16, 16, 32, 48, 64])
    tokens = rng.choice([1, 7, 64, 256, rng.randint(1, 300)])
    return {
        "dtype": rng.choice(DTYPES),
        "kv_heads": rng.choice([1, 2, 4, 8]),
        "head_dim": rng.choice([1, 3, 32, 64, 80, 128, 160]),
        "block_size": block,
        "tokens": tokens,
        "blocks": max(1, -(-tokens // block)) + rng.randint(0, 6),
    }


def test_the_sweeps_reach_the_shapes_they_are_for():
    """The drawn shapes cover what the sweeps are for (host only)."""

    ops = [draw_op(s) for s in range(CASES)]
    assert {c["dtype"] for c in ops} == set(DTYPES)
    assert any(c["cols"] % 64 for c in ops) and any(c["cols"] >= 8192 for c in ops)
    assert any(c["constant_row"] for c in ops)
    kvs = [draw_kv(s) for s in range(CASES)]
    assert {c["dtype"] for c in kvs} == set(DTYPES)
    assert any(c["head_dim"] % 8 for c in kvs) and any(c["block_size"] % 16 for c in kvs)
    assert any(c["tokens"] > c["block_size"] for c in kvs)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(CASES))
def test_drawn_norms_and_swiglu_match_the_oracle(device, seed):
    spec = draw_op(seed)
    dtype, rows, cols, eps = spec["dtype"], spec["rows"], spec["cols"], spec["eps"]
    what = f"seed {seed}: {dtype} [{rows}x{cols}] eps {eps}"
    generator = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, cols, generator=generator).to(dtype)
    r = torch.randn(rows, cols, generator=generator).to(dtype)
    weight = (1 + 0.1 * torch.randn(cols, generator=generator)).to(dtype)
    if spec["constant_row"]:
        x[0] = 0.75
    tol = REFERENCE_TOLERANCE[dtype]

    actual = rms_norm(x.to(device), weight.to(device), eps)
    assert_close(actual, rms_norm_reference(x, weight, eps), tol, tol, f"{what} rms_norm")

    res, norm = residual_rms_norm(x.to(device), r.to(device), weight.to(device), eps)
    want_res, want_norm = residual_rms_norm_reference(x, r, weight, eps)
    assert_bit_exact(res, want_res, f"{what} residual sum")
    assert_close(norm, want_norm, tol, tol, f"{what} residual_rms_norm")

    act = swiglu(x.to(device), r.to(device))
    assert_close(act, swiglu_reference(x, r), tol, tol, f"{what} swiglu")


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(CASES))
def test_drawn_kv_writes_are_bit_exact(device, seed):
    spec = draw_kv(seed)
    dtype, hkv, d = spec["dtype"], spec["kv_heads"], spec["head_dim"]
    block, tokens, blocks = spec["block_size"], spec["tokens"], spec["blocks"]
    what = f"seed {seed}: {dtype} {hkv}x{d}, pages of {block} x {blocks}, {tokens} tokens"
    generator = torch.Generator().manual_seed(seed)
    rng = random.Random(seed)
    keys = torch.randn(tokens, hkv, d, generator=generator).to(dtype)
    values = torch.randn(tokens, hkv, d, generator=generator).to(dtype)
    key_cache = torch.randn(blocks, block, hkv, d, generator=generator).to(dtype)
    value_cache = torch.randn(blocks, block, hkv, d, generator=generator).to(dtype)

    # One token per lane: distinct slots, some lanes inactive.
    lanes = min(tokens, blocks * block)
    slots = torch.randperm(blocks * block, generator=generator)[:lanes]
    physical = (slots // block).to(torch.int32)
    offsets = (slots % block).to(torch.int32)
    active = torch.tensor([int(rng.random() < 0.8) for _ in range(lanes)], dtype=torch.int32)
    want_k, want_v = paged_kv_write_token_reference(
        keys[:lanes], values[:lanes], key_cache, value_cache, physical, offsets, active)
    k_dev, v_dev = key_cache.to(device), value_cache.to(device)
    paged_kv_write_token(keys[:lanes].to(device), values[:lanes].to(device), k_dev, v_dev,
                         physical.to(device), offsets.to(device), active.to(device))
    assert_bit_exact(k_dev, want_k, f"{what} token writer, keys")
    assert_bit_exact(v_dev, want_v, f"{what} token writer, values")

    # Slot mapping: distinct slots in any order, some padded (-1).
    order = torch.randperm(blocks * block, generator=generator)[:lanes].to(torch.int64)
    mapping = torch.where(torch.rand(lanes, generator=generator) < 0.15,
                          torch.full_like(order, -1), order)
    want_k, want_v = paged_kv_write_slots_reference(
        keys[:lanes], values[:lanes], key_cache, value_cache, mapping)
    k_dev, v_dev = key_cache.to(device), value_cache.to(device)
    paged_kv_write_slots(keys[:lanes].to(device), values[:lanes].to(device), k_dev, v_dev,
                         mapping.to(device))
    assert_bit_exact(k_dev, want_k, f"{what} slot writer, keys")
    assert_bit_exact(v_dev, want_v, f"{what} slot writer, values")
