"""The decode step's fused RoPE + KV append + attention launch against the
two launches it replaces (rope_paged_kv_append, then
paged_gqa_decode_attention) and against the CPU oracle.

The fused kernel rotates with the same arithmetic as the RoPE kernel, so the
attention output and both caches must be bit-identical to the unfused pair,
in the wide and narrow one-pass plans and the narrow split-KV plan, with
padded lanes that write nothing.  The
oracle check (RoPE oracle, then the paged attention oracle over the updated
caches) uses the north-star bar (max-abs 2e-2 + rel 1e-2).
"""

from __future__ import annotations

import pytest
import torch

from helpers import NORTH_STAR_ATOL, NORTH_STAR_RTOL, assert_close
from oracle.model import rope_tables
from oracle.reference import paged_gqa_decode_reference, rope_kv_append_reference
from tensorforge_amd.kernels import (
    PagedAttentionWorkspace,
    paged_gqa_decode_attention,
    rope_paged_kv_append,
)
from tensorforge_amd.kernels.attention import paged_gqa_decode_attention_rope_append
from tensorforge_amd.workloads import make_decode_attention_case

pytestmark = pytest.mark.gpu


def _inputs(lengths, hq, hkv, d, dtype, seed, row_pad=0, block_size=16):
    case = make_decode_attention_case(lengths, query_heads=hq, kv_heads=hkv, head_dim=d,
                                      block_size=block_size, dtype=dtype, seed=seed, extra_pages=4)
    generator = torch.Generator().manual_seed(seed + 1)
    qkv = torch.randn(len(lengths), (hq + 2 * hkv) * d + row_pad, generator=generator).to(dtype)
    positions = torch.tensor([max(c - 1, 0) for c in lengths], dtype=torch.int64)
    pages = torch.tensor([int(case.block_tables[r, (c - 1) // block_size]) if c > 0 else -1
                          for r, c in enumerate(lengths)], dtype=torch.int32)
    offsets = torch.tensor([(c - 1) % block_size if c > 0 else 0 for c in lengths],
                           dtype=torch.int32)
    active = torch.tensor([1 if c > 0 else 0 for c in lengths], dtype=torch.int32)
    cos, sin = rope_tables(d, 10000.0, torch.arange(4096))
    return case, qkv, positions, cos.to(dtype), sin.to(dtype), pages, offsets, active


@pytest.mark.parametrize(("hq", "hkv", "d", "dtype"),
                         [(32, 4, 64, torch.bfloat16), (8, 2, 32, torch.float16),
                          (32, 8, 128, torch.bfloat16), (16, 1, 64, torch.float16)])
@pytest.mark.parametrize("rows", ["wide", "narrow", "long"])
def test_fused_rope_attention_equals_the_two_launches(device, hq, hkv, d, dtype, rows):
    generator = torch.Generator().manual_seed(hq + d)
    if rows == "wide":  # >= 192 (row, kv head) workgroups: the one-pass plan
        count = max(48, -(-192 // hkv))
        lengths = [int(x) for x in torch.randint(1, 700, (count,), generator=generator)]
        lengths[3] = 0
        lengths[7] = 1
    elif rows == "narrow":  # few rows, short: one pass, up to 8 wavefronts per kv head
        lengths = [700, 1, 0, 33, 512, 17]
    else:  # few rows, long: split-KV with several wavefronts per split, merge launch
        lengths = [3000, 1, 0, 1500, 2047, 17]
    case, qkv, positions, cos, sin, pages, offsets, active = _inputs(lengths, hq, hkv, d, dtype,
                                                                     seed=len(lengths) + d,
                                                                     row_pad=8)
    gpu = case.to(device)
    width = (hq + 2 * hkv) * d
    qkv_dev = qkv.to(device)[:, :width]  # strided rows
    args = [t.to(device) for t in (positions, cos, sin)]
    append = [t.to(device) for t in (pages, offsets, active)]
    capacity = max(lengths)
    workspace = PagedAttentionWorkspace.allocate(batch_capacity=len(lengths), query_heads=hq,
                                                 head_dim=d, max_context_length=4096,
                                                 device=device)

    k1, v1 = gpu.key_cache.clone(), gpu.value_cache.clone()
    q = rope_paged_kv_append(qkv_dev, *args, k1, v1, *append, query_heads=hq)
    out1 = paged_gqa_decode_attention(q, k1, v1, gpu.block_tables, gpu.context_lengths,
                                      max_context_length=capacity, workspace=workspace)
    k2, v2 = gpu.key_cache.clone(), gpu.value_cache.clone()
    out2 = torch.full_like(out1, float("nan"))
    paged_gqa_decode_attention_rope_append(
        qkv_dev, *args, k2, v2, *append, gpu.block_tables, gpu.context_lengths,
        query_heads=hq, max_context_length=capacity, output=out2, workspace=workspace)
    torch.cuda.synchronize()
    assert torch.equal(out2.view(torch.int16), out1.view(torch.int16))
    assert torch.equal(k2.view(torch.int16), k1.view(torch.int16))
    assert torch.equal(v2.view(torch.int16), v1.view(torch.int16))

    # Against the oracle: rotate and append on the CPU, then attend.
    q_ref, k_ref, v_ref = rope_kv_append_reference(
        qkv[:, :width], positions, cos, sin, case.key_cache, case.value_cache, pages, offsets,
        active, query_heads=hq)
    tol = {torch.float16: 3e-3, torch.bfloat16: 3e-2}[dtype]  # one rounding of an fp32 value
    assert_close(k2.cpu(), k_ref, tol, tol, "rotated keys in the cache")
    assert torch.equal(v2.cpu().view(torch.int16), v_ref.view(torch.int16))
    live = [r for r, c in enumerate(lengths) if c > 0]
    want = paged_gqa_decode_reference(q_ref.view(len(lengths), hq, d)[live], k_ref, v_ref,
                                      case.block_tables[live], case.context_lengths[live],
                                      scale=d ** -0.5)
    assert_close(out2.cpu()[live], want, NORTH_STAR_ATOL, NORTH_STAR_RTOL, "fused vs oracle")
    assert bool((out2.cpu()[[r for r, c in enumerate(lengths) if c == 0]] == 0).all())


@pytest.mark.parametrize("block_size", [32, 48, 64])
@pytest.mark.parametrize(("hq", "hkv", "d", "dtype"),
                         [(32, 4, 64, torch.bfloat16), (8, 2, 32, torch.float16)])
@pytest.mark.parametrize("rows", ["wide", "long"])
def test_fused_rope_attention_on_larger_pages(device, hq, hkv, d, dtype, rows, block_size):
    """Pages of 32, 48 (not a power of two: the division form of the page and
    in-page indices) and 64 tokens: the new token's append slot lands at any
    offset of a page, and the fused launch still equals the two launches."""

    generator = torch.Generator().manual_seed(block_size + d)
    if rows == "wide":
        count = max(48, -(-192 // hkv))
        lengths = [int(x) for x in torch.randint(1, 700, (count,), generator=generator)]
        lengths[3] = 0
        lengths[5] = block_size          # the new token is a page's last slot
        lengths[6] = block_size + 1      # ... or the first slot of a new page
    else:
        lengths = [3000, 1, 0, 1500, 2047, block_size]
    case, qkv, positions, cos, sin, pages, offsets, active = _inputs(
        lengths, hq, hkv, d, dtype, seed=len(lengths) + block_size, block_size=block_size)
    gpu = case.to(device)
    qkv_dev = qkv.to(device)
    args = [t.to(device) for t in (positions, cos, sin)]
    append = [t.to(device) for t in (pages, offsets, active)]
    capacity = gpu.block_tables.shape[1] * block_size
    workspace = PagedAttentionWorkspace.allocate(batch_capacity=len(lengths), query_heads=hq,
                                                 head_dim=d, max_context_length=4096,
                                                 device=device)
    k1, v1 = gpu.key_cache.clone(), gpu.value_cache.clone()
    q = rope_paged_kv_append(qkv_dev, *args, k1, v1, *append, query_heads=hq)
    out1 = paged_gqa_decode_attention(q, k1, v1, gpu.block_tables, gpu.context_lengths,
                                      max_context_length=capacity, workspace=workspace)
    k2, v2 = gpu.key_cache.clone(), gpu.value_cache.clone()
    out2 = torch.full_like(out1, float("nan"))
    paged_gqa_decode_attention_rope_append(
        qkv_dev, *args, k2, v2, *append, gpu.block_tables, gpu.context_lengths,
        query_heads=hq, max_context_length=capacity, output=out2, workspace=workspace)
    torch.cuda.synchronize()
    assert torch.equal(out2.view(torch.int16), out1.view(torch.int16))
    assert torch.equal(k2.view(torch.int16), k1.view(torch.int16))
    assert torch.equal(v2.view(torch.int16), v1.view(torch.int16))
    live = [r for r, c in enumerate(lengths) if c > 0]
    q_ref, k_ref, v_ref = rope_kv_append_reference(
        qkv, positions, cos, sin, case.key_cache, case.value_cache, pages, offsets, active,
        query_heads=hq)
    want = paged_gqa_decode_reference(q_ref.view(len(lengths), hq, d)[live], k_ref, v_ref,
                                      case.block_tables[live], case.context_lengths[live],
                                      scale=d ** -0.5)
    assert_close(out2.cpu()[live], want, NORTH_STAR_ATOL, NORTH_STAR_RTOL,
                 f"fused vs oracle, pages of {block_size}")


def test_fused_rope_attention_rejects_non_mfma_geometry(device):
    case, qkv, positions, cos, sin, pages, offsets, active = _inputs(
        [40, 3], 4, 2, 80, torch.bfloat16, seed=3)
    gpu = case.to(device)
    workspace = PagedAttentionWorkspace.allocate(batch_capacity=2, query_heads=4, head_dim=80,
                                                 max_context_length=64, device=device)
    with pytest.raises(RuntimeError, match="MFMA"):
        paged_gqa_decode_attention_rope_append(
            qkv.to(device), positions.to(device), cos.to(device), sin.to(device),
            gpu.key_cache, gpu.value_cache, pages.to(device), offsets.to(device),
            active.to(device), gpu.block_tables, gpu.context_lengths, query_heads=4,
            max_context_length=40, output=torch.empty(2, 4, 80, dtype=torch.bfloat16,
                                                      device=device),
            workspace=workspace)
