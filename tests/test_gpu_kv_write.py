"""Bit-exact parity of the gfx950 paged KV append with the CPU oracle.

Single-token writer: reference tests/test_decode_bucket.py:233-287 (padded
lanes must not write) and kernels/triton_cache.py:23-63.  Multi-token slot
append: cache/paged.py:221-235 and BASELINE config 4 (T in {1, 8, 64, 256},
4 KV heads x 64, slots straddling pages, slot -1 for padded lanes).
"""

from __future__ import annotations

import pytest
import torch

from helpers import assert_bit_exact
from oracle.reference import (
    paged_kv_write_slots_reference,
    paged_kv_write_token_reference,
    write_layer_slots,
)
from tensorforge_amd.kernels import paged_kv_write_slots, paged_kv_write_token

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def _cache(num_blocks, block_size, kv_heads, head_dim, dtype, seed):
    generator = torch.Generator().manual_seed(seed)
    key_cache = torch.randn(num_blocks, block_size, kv_heads, head_dim, generator=generator).to(dtype)
    value_cache = torch.randn(num_blocks, block_size, kv_heads, head_dim, generator=generator).to(dtype)
    return key_cache, value_cache


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(("kv_heads", "head_dim"), [(4, 64), (2, 80), (1, 3), (8, 128)])
def test_token_write_masks_padded_lanes(device, dtype, kv_heads, head_dim):
    batch, num_blocks, block_size = 12, 9, 16
    generator = torch.Generator().manual_seed(kv_heads * 1000 + head_dim)
    keys = torch.randn(batch, kv_heads, head_dim, generator=generator).to(dtype)
    values = torch.randn(batch, kv_heads, head_dim, generator=generator).to(dtype)
    slots = torch.randperm(num_blocks * block_size, generator=generator)[:batch]
    physical = (slots // block_size).to(torch.int32)
    offsets = (slots % block_size).to(torch.int32)
    active = torch.tensor([1, 1, 0, 1, 0, 0, 1, 1, 1, 0, 1, 1], dtype=torch.int32)
    key_cache, value_cache = _cache(num_blocks, block_size, kv_heads, head_dim, dtype, 5)
    expected_k, expected_v = paged_kv_write_token_reference(
        keys, values, key_cache, value_cache, physical, offsets, active,
    )
    k_dev, v_dev = key_cache.to(device), value_cache.to(device)
    paged_kv_write_token(keys.to(device), values.to(device), k_dev, v_dev, physical.to(device),
                         offsets.to(device), active.to(device))
    assert_bit_exact(k_dev, expected_k, "key cache")
    assert_bit_exact(v_dev, expected_v, "value cache")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("tokens", [1, 8, 64, 256])
def test_slot_append_config4(device, dtype, tokens):
    """T tokens x 4 KV heads x 64, slots straddling pages, -1 padded lanes."""

    kv_heads, head_dim, block_size = 4, 64, 16
    num_blocks = (tokens + block_size - 1) // block_size * 2 + 3
    generator = torch.Generator().manual_seed(tokens)
    keys = torch.randn(tokens, kv_heads, head_dim, generator=generator).to(dtype)
    values = torch.randn(tokens, kv_heads, head_dim, generator=generator).to(dtype)
    # A sequence whose pages are a random permutation, starting mid-page.
    blocks = torch.randperm(num_blocks, generator=generator).tolist()
    start = 11
    slots = torch.from_numpy(write_layer_slots(blocks, start, tokens, block_size))
    if tokens > 1:
        slots[torch.arange(tokens) % 5 == 3] = -1  # padded lanes
    key_cache, value_cache = _cache(num_blocks, block_size, kv_heads, head_dim, dtype, tokens + 1)
    expected_k, expected_v = paged_kv_write_slots_reference(keys, values, key_cache,
                                                            value_cache, slots)
    k_dev, v_dev = key_cache.to(device), value_cache.to(device)
    paged_kv_write_slots(keys.to(device), values.to(device), k_dev, v_dev, slots.to(device))
    assert_bit_exact(k_dev, expected_k, "key cache")
    assert_bit_exact(v_dev, expected_v, "value cache")


def test_slot_append_known_answer_arange(device):
    """tests/test_paged_cache.py:11-37: three tokens across two 2-token pages."""

    keys = torch.arange(24, dtype=torch.float32).view(3, 2, 4)
    values = keys + 100
    key_cache = torch.zeros(4, 2, 2, 4)
    value_cache = torch.zeros(4, 2, 2, 4)
    slots = torch.from_numpy(write_layer_slots([0, 1], 0, 3, 2))
    k_dev, v_dev = key_cache.to(device), value_cache.to(device)
    paged_kv_write_slots(keys.to(device), values.to(device), k_dev, v_dev, slots.to(device))
    k_host = k_dev.cpu()
    dense = torch.cat((k_host[0], k_host[1, :1]))  # logical order: page 0, then page 1 row 0
    assert torch.equal(dense, keys)
    assert torch.equal(torch.cat((v_dev.cpu()[0], v_dev.cpu()[1, :1])), values)
    assert torch.equal(k_host[1, 1:], torch.zeros(1, 2, 4)) and torch.equal(k_host[2:], torch.zeros(2, 2, 2, 4))


def test_out_of_range_destinations_are_skipped(device):
    keys = torch.ones(3, 2, 8, dtype=torch.bfloat16, device=device)
    key_cache = torch.zeros(2, 4, 2, 8, dtype=torch.bfloat16, device=device)
    value_cache = torch.zeros_like(key_cache)
    slots = torch.tensor([-1, 8, 7], dtype=torch.int64, device=device)
    paged_kv_write_slots(keys, keys, key_cache, value_cache, slots)
    physical = torch.tensor([5, 0, 1], dtype=torch.int32, device=device)
    offsets = torch.tensor([0, 4, 3], dtype=torch.int32, device=device)
    active = torch.ones(3, dtype=torch.int32, device=device)
    paged_kv_write_token(keys, keys, key_cache, value_cache, physical, offsets, active)
    flat = key_cache.view(8, 2, 8).cpu().float()
    assert float(flat[7].sum()) == 16.0  # slot 7 written by both calls
    assert float(flat[:7].sum()) == 0.0


def test_write_rejects_cpu_and_bad_controls(device):
    keys = torch.ones(2, 2, 8, device=device)
    cache = torch.zeros(2, 4, 2, 8, device=device)
    control = torch.zeros(2, dtype=torch.int32, device=device)
    with pytest.raises(ValueError, match="CUDA"):
        paged_kv_write_token(keys.cpu(), keys, cache, cache, control, control, control)
    with pytest.raises(ValueError, match="int32"):
        paged_kv_write_token(keys, keys, cache, cache, control.long(), control, control)
    with pytest.raises(ValueError, match="int64"):
        paged_kv_write_slots(keys, keys, cache, cache, control)
