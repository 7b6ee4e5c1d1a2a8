"""Split-KV with balanced partitions (TF_ATTENTION_FLAG_BALANCED) against the
oracle and against fixed partitions of the same size, through the C ABI.

A balanced call sizes its partitions on the device from the rows' lengths
-- max(split_size, ceil32(ceil(total / (num_splits - batch)))) tokens, the
same for every row -- and launches one compact grid of (kv-head group x
slot) workgroups that take the rows' partitions in row order.  So its
partials and output must be bit-identical to a fixed-partition call with
that partition size, and within the north-star bar of the oracle: ragged
rows, zero-length rows, one long row among short ones, 64 rows, pages of 32
and 48 tokens, one and several wavefronts per partition, HIP-graph replay
with lengths that change between replays (the partition size changes with
them), the fused RoPE + append launch, and the rejected combinations.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from helpers import NORTH_STAR_ATOL, NORTH_STAR_RTOL, assert_close
from oracle.model import rope_tables
from oracle.reference import paged_gqa_decode_reference
from tensorforge_amd import _native
from tensorforge_amd.kernels import (
    PagedAttentionWorkspace,
    paged_gqa_decode_attention,
    rope_paged_kv_append,
    selected_attention_autotune_config,
    selected_attention_launch,
)
from tensorforge_amd.kernels.attention import paged_gqa_decode_attention_rope_append
from tensorforge_amd.workloads import llama3_long_context_case, make_decode_attention_case

pytestmark = pytest.mark.gpu

UNSUPPORTED = 2  # TF_ERROR_UNSUPPORTED


def _wave_flags(waves_per_head: int, tokens_per_wave: int = 64, heads_per_wg: int = 1) -> int:
    if waves_per_head <= 1 and heads_per_wg <= 1:
        return 0
    return ((heads_per_wg << _native.TF_ATTENTION_HEADS_PER_WG_SHIFT)
            | (waves_per_head << _native.TF_ATTENTION_WAVES_PER_CU_SHIFT)
            | ((tokens_per_wave // 64) << _native.TF_ATTENTION_TOKENS_PER_WAVE_SHIFT))


def _partition_size(lengths, split_size, num_splits, capacity):
    """The device's balanced partition size, restated on the host."""

    max_tokens = min(num_splits * split_size, capacity)
    total = sum(min(max(n, 0), max_tokens) for n in lengths)
    spare = num_splits - len(lengths)
    size = (-(-total // spare) + 31) // 32 * 32
    size = min(size, (max_tokens + 31) // 32 * 32)
    return max(size, split_size)


def _call(gpu, out, flags, split_size, num_splits, counters=None, partials=None):
    batch, query_heads, head_dim = gpu.query.shape
    num_blocks, block_size, kv_heads, _ = gpu.key_cache.shape
    rows = batch * query_heads * num_splits
    if partials is None:
        partials = (torch.empty(rows, device=out.device), torch.empty(rows, device=out.device),
                    torch.empty((rows, head_dim), device=out.device))
    status = _native.library().tf_paged_gqa_decode(
        gpu.query.data_ptr(), gpu.key_cache.data_ptr(), gpu.value_cache.data_ptr(),
        gpu.block_tables.data_ptr(), gpu.context_lengths.data_ptr(), out.data_ptr(),
        partials[0].data_ptr(), partials[1].data_ptr(), partials[2].data_ptr(), counters,
        partials[0].numel(), head_dim, batch, query_heads, kv_heads, head_dim, num_blocks,
        block_size, gpu.block_tables.shape[1], split_size, num_splits, ctypes.c_float(gpu.scale),
        _native.dtype_code(gpu.query.dtype), flags, _native.current_stream(out.device))
    return status, partials


def _oracle(case):
    rows = [r for r, n in enumerate(case.lengths) if n > 0]
    cpu = case.to("cpu")
    want = paged_gqa_decode_reference(cpu.query[rows], cpu.key_cache, cpu.value_cache,
                                      cpu.block_tables[rows], cpu.context_lengths[rows],
                                      scale=cpu.scale)
    return rows, want


def _check(case, actual, what):
    rows, want = _oracle(case)
    assert_close(actual.cpu()[rows], want, NORTH_STAR_ATOL, NORTH_STAR_RTOL, what)
    for r, n in enumerate(case.lengths):
        if n <= 0:
            assert bool((actual[r] == 0).all()), f"{what}: zero-length row {r} not zero"


# lengths, query heads, kv heads, head_dim, page, dtype, slots, smallest partition, waves.
# A call covers slots x smallest partition tokens of a row (longer rows are
# clamped, as with fixed partitions), so each case's longest row fits.
CASES = {
    "long among short, D128": ([8192, 16384, 0, 3000, 1], 32, 8, 128, 16, torch.bfloat16, 32,
                               512, 4),
    "ragged fp16, one wave": ([5000, 37, 0, 0, 1200, 64, 2049], 16, 4, 64, 16, torch.float16, 16,
                              320, 1),
    "one slot more than rows": ([300, 7000], 8, 2, 32, 16, torch.bfloat16, 3, 2336, 2),
    "pages of 32": ([900, 2500, 17, 4096], 16, 2, 64, 32, torch.bfloat16, 20, 224, 4),
    "pages of 48": ([1000, 47, 48, 49, 3001], 16, 4, 64, 48, torch.float16, 24, 128, 8),
    "smallest partition wins": ([100, 200, 50], 8, 2, 64, 16, torch.bfloat16, 8, 256, 4),
}


# Each case with 1, 2 and 4 kv heads per workgroup where they divide its kv
# heads and fit 8 wavefronts.
HEADS_CASES = [(name, heads) for name in sorted(CASES) for heads in (1, 2, 4)
               if CASES[name][2] % heads == 0 and heads * CASES[name][8] <= 8]


@pytest.mark.parametrize(("name", "heads_per_wg"), HEADS_CASES)
def test_balanced_partitions_match_oracle_and_fixed_partitions(device, name, heads_per_wg):
    """Also with 2 and 4 kv heads per workgroup (the slots then count
    groups of kv heads): bit-identical to one kv head per workgroup, since a
    kv head's partition is dealt over its own wavefronts the same way."""

    lengths, hq, hkv, d, page, dtype, slots, smallest, waves = CASES[name]
    assert max(lengths) <= slots * smallest
    width = max((max(lengths) + page - 1) // page, 1) + 2
    case = make_decode_attention_case(lengths, query_heads=hq, kv_heads=hkv, head_dim=d,
                                      block_size=page, dtype=dtype, seed=len(lengths) + d,
                                      table_width=width)
    gpu = case.to(device)
    flags = _wave_flags(waves, heads_per_wg=heads_per_wg)
    out = torch.full_like(gpu.query, float("nan"))
    status, _ = _call(gpu, out, flags | _native.TF_ATTENTION_FLAG_BALANCED, smallest, slots)
    assert status == 0, _native.library().tf_last_error()
    torch.cuda.synchronize()
    _check(case, out, f"balanced {name}")
    if heads_per_wg > 1:
        one = torch.full_like(gpu.query, float("nan"))
        status, _ = _call(gpu, one, _wave_flags(waves) | _native.TF_ATTENTION_FLAG_BALANCED,
                          smallest, slots)
        assert status == 0, _native.library().tf_last_error()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), one.view(torch.int16)), (
            f"{name}: {heads_per_wg} kv heads per workgroup differ from one")

    size = _partition_size(lengths, smallest, slots, width * page)
    fixed_splits = max(1, -(-min(slots * smallest, width * page) // size))
    fixed = torch.full_like(gpu.query, float("nan"))
    if fixed_splits > 1:
        status, _ = _call(gpu, fixed, flags, size, fixed_splits)
    else:  # one partition per row: the one-pass form
        status, _ = _call(gpu, fixed, flags, size, 1)
    assert status == 0, _native.library().tf_last_error()
    torch.cuda.synchronize()
    if fixed_splits > 1:
        assert torch.equal(out.view(torch.int16), fixed.view(torch.int16)), (
            f"{name}: balanced partitions of {size} tokens differ from fixed ones")
    else:
        _check(case, fixed, f"fixed one pass {name}")


def test_sixty_four_rows(device):
    generator = torch.Generator().manual_seed(64)
    lengths = [int(x) for x in torch.randint(0, 3000, (64,), generator=generator)]
    lengths[5] = 0
    lengths[9] = 12000
    case = make_decode_attention_case(lengths, query_heads=8, kv_heads=2, head_dim=64,
                                      block_size=16, dtype=torch.bfloat16, seed=3)
    gpu = case.to(device)
    out = torch.full_like(gpu.query, float("nan"))
    status, _ = _call(gpu, out, _wave_flags(4) | _native.TF_ATTENTION_FLAG_BALANCED, 256, 128)
    assert status == 0, _native.library().tf_last_error()
    torch.cuda.synchronize()
    _check(case, out, "balanced 64 rows")


def test_config3_entry_point_plan(device):
    """BASELINE config 3 through the entry point: 2..64 rows of >= 8k take
    balanced partitions (four kv heads per workgroup, 128 slots per group of
    four on 256 compute units)."""

    case = llama3_long_context_case(seed=2)
    gpu = case.to(device)
    output = paged_gqa_decode_attention(gpu.query, gpu.key_cache, gpu.value_cache,
                                        gpu.block_tables, gpu.context_lengths,
                                        max_context_length=32768)
    assert selected_attention_autotune_config() == {
        "path": "split_kv", "split_size": 256, "num_splits": 128,
    }
    launch = selected_attention_launch()
    assert launch["balanced_partitions"] and launch["waves_per_head"] == 2
    assert launch["heads_per_workgroup"] == 4
    assert launch["grid"] == (2 * 128, 1)
    _check(case, output, "cfg3 balanced")


def test_many_long_rows_take_the_slots_their_workspace_holds(device):
    """16 rows of 8k-9k: with the entry point's own workspace the plan takes
    four kv heads per workgroup and 128 slots; a workspace sized as the
    reference sizes it (one partial per 256 tokens of a row) holds only 36
    slots per row, so the plan drops to 32 slots of one kv head.  Both
    match the oracle."""

    lengths = [8192 + 64 * i for i in range(16)]
    case = make_decode_attention_case(lengths, query_heads=32, kv_heads=8, head_dim=128,
                                      block_size=16, dtype=torch.bfloat16, seed=16)
    gpu = case.to(device)
    output = paged_gqa_decode_attention(gpu.query, gpu.key_cache, gpu.value_cache,
                                        gpu.block_tables, gpu.context_lengths)
    launch = selected_attention_launch()
    assert launch["balanced_partitions"] and launch["heads_per_workgroup"] == 4
    assert launch["grid"] == (2 * 128, 1)
    _check(case, output, "16 long rows, own workspace")
    workspace = PagedAttentionWorkspace.allocate(batch_capacity=16, query_heads=32,
                                                 head_dim=128, max_context_length=max(lengths),
                                                 device=device)
    output = paged_gqa_decode_attention(gpu.query, gpu.key_cache, gpu.value_cache,
                                        gpu.block_tables, gpu.context_lengths,
                                        workspace=workspace)
    launch = selected_attention_launch()
    assert launch["balanced_partitions"] and launch["heads_per_workgroup"] == 1
    assert launch["grid"] == (8 * 32, 1)
    _check(case, output, "16 long rows, reference-sized workspace")


def test_graph_replay_follows_device_lengths(device):
    """The partition size is recomputed from the device lengths on every
    replay: shrink and grow the rows between replays of one graph."""

    # Every row's table holds 6000 tokens; the lengths then vary below that.
    case = make_decode_attention_case([6000] * 4, query_heads=16, kv_heads=4, head_dim=64,
                                      block_size=16, dtype=torch.bfloat16, seed=11)
    case.context_lengths = torch.tensor([6000, 300, 4000, 0], dtype=torch.int32)
    gpu = case.to(device)
    out = torch.full_like(gpu.query, float("nan"))
    rows = 4 * 16 * 16
    partials = (torch.empty(rows, device=device), torch.empty(rows, device=device),
                torch.empty((rows, 64), device=device))
    flags = _wave_flags(4) | _native.TF_ATTENTION_FLAG_BALANCED
    stream = torch.cuda.Stream(device)
    with torch.cuda.stream(stream):
        status, _ = _call(gpu, out, flags, 384, 16, partials=partials)
        assert status == 0
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        status, _ = _call(gpu, out, flags, 384, 16, partials=partials)
        assert status == 0
    for new_lengths in ([6000, 300, 4000, 0], [17, 5999, 0, 4000], [0, 0, 1, 0],
                        [3000, 3000, 3000, 3000]):
        gpu.context_lengths.copy_(torch.tensor(new_lengths, dtype=torch.int32))
        torch.cuda.synchronize()
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        case.context_lengths = gpu.context_lengths.cpu()
        _check(case, out, f"graph replay {new_lengths}")


def test_fused_rope_append_with_balanced_partitions(device):
    """The fused RoPE + append + attention launch under the balanced plan is
    bit-identical to the RoPE kernel followed by the attention entry point
    (both planned alike), output and caches."""

    lengths = [9000, 1, 0, 8192, 300]
    hq, hkv, d, dtype = 32, 8, 128, torch.bfloat16
    case = make_decode_attention_case(lengths, query_heads=hq, kv_heads=hkv, head_dim=d,
                                      block_size=16, dtype=dtype, seed=5, extra_pages=4)
    generator = torch.Generator().manual_seed(6)
    qkv = torch.randn(len(lengths), (hq + 2 * hkv) * d, generator=generator).to(dtype)
    positions = torch.tensor([max(c - 1, 0) for c in lengths], dtype=torch.int64)
    pages = torch.tensor([int(case.block_tables[r, (c - 1) // 16]) if c > 0 else -1
                          for r, c in enumerate(lengths)], dtype=torch.int32)
    offsets = torch.tensor([(c - 1) % 16 if c > 0 else 0 for c in lengths], dtype=torch.int32)
    active = torch.tensor([1 if c > 0 else 0 for c in lengths], dtype=torch.int32)
    cos, sin = rope_tables(d, 10000.0, torch.arange(16384))
    gpu = case.to(device)
    args = [t.to(device) for t in (positions, cos.to(dtype), sin.to(dtype))]
    append = [t.to(device) for t in (pages, offsets, active)]
    qkv_dev = qkv.to(device)
    capacity = max(lengths)
    workspace = PagedAttentionWorkspace.allocate(batch_capacity=len(lengths), query_heads=hq,
                                                 head_dim=d, max_context_length=capacity,
                                                 device=device)
    k1, v1 = gpu.key_cache.clone(), gpu.value_cache.clone()
    q = rope_paged_kv_append(qkv_dev, *args, k1, v1, *append, query_heads=hq)
    out1 = paged_gqa_decode_attention(q, k1, v1, gpu.block_tables, gpu.context_lengths,
                                      max_context_length=capacity, workspace=workspace)
    assert selected_attention_launch()["balanced_partitions"]
    k2, v2 = gpu.key_cache.clone(), gpu.value_cache.clone()
    out2 = torch.full_like(out1, float("nan"))
    paged_gqa_decode_attention_rope_append(
        qkv_dev, args[0], args[1], args[2], k2, v2, append[0], append[1], append[2],
        gpu.block_tables, gpu.context_lengths, query_heads=hq, max_context_length=capacity,
        workspace=workspace, output=out2)
    torch.cuda.synchronize()
    assert torch.equal(out1.view(torch.int16), out2.view(torch.int16))
    assert torch.equal(k1.view(torch.int16), k2.view(torch.int16))
    assert torch.equal(v1.view(torch.int16), v2.view(torch.int16))


def test_unsupported_combinations_are_rejected(device):
    case = make_decode_attention_case([3000, 200], query_heads=8, kv_heads=2, head_dim=64,
                                      block_size=16, dtype=torch.bfloat16, seed=1)
    gpu = case.to(device)
    out = torch.empty_like(gpu.query)
    bal = _native.TF_ATTENTION_FLAG_BALANCED
    counters = torch.zeros(16, dtype=torch.int32, device=device)
    for flags, splits, ctr, what in ((bal, 2, None, "num_splits <= batch"),
                                     (bal, 8, counters.data_ptr(), "arrival counters"),
                                     (bal | _native.TF_ATTENTION_FLAG_VALU, 8, None, "VALU"),
                                     (bal | _native.TF_ATTENTION_FLAG_FORCE_GENERIC, 8, None,
                                      "generic kernel")):
        status, _ = _call(gpu, out, flags, 256, splits, counters=ctr)
        assert status == UNSUPPORTED, what
        assert b"balanced partitions need" in _native.library().tf_last_error(), what
    status, _ = _call(gpu, out, 4, 256, 8)  # bit 2: no meaning in this ABI
    assert status == UNSUPPORTED
    assert b"unknown attention flag bits" in _native.library().tf_last_error()
    many = make_decode_attention_case([40] * 65, query_heads=8, kv_heads=2, head_dim=64,
                                      block_size=16, dtype=torch.bfloat16, seed=2)
    gpu65 = many.to(device)
    status, _ = _call(gpu65, torch.empty_like(gpu65.query), bal, 32, 80)
    assert status == UNSUPPORTED
    rows = 2 * 8 * 8
    status = _native.library().tf_paged_gqa_decode_partials(
        gpu.query.data_ptr(), gpu.key_cache.data_ptr(), gpu.value_cache.data_ptr(),
        gpu.block_tables.data_ptr(), gpu.context_lengths.data_ptr(),
        torch.empty(rows, device=device).data_ptr(), torch.empty(rows, device=device).data_ptr(),
        torch.empty((rows, 64), device=device).data_ptr(), rows, 64, 2, 8, 2, 64,
        gpu.key_cache.shape[0], 16, gpu.block_tables.shape[1], 256, 8, ctypes.c_float(0.125),
        _native.dtype_code(torch.bfloat16), bal, _native.current_stream(device))
    assert status == UNSUPPORTED
