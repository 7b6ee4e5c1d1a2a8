"""The page-stream attention kernel (TF_ATTENTION_FLAG_PAGES) against the
oracle, through the C ABI.

The kernel gives every workgroup an equal contiguous range of the batch's
pages, so rows are cut into pieces at arbitrary page boundaries and merged
in the same launch by the last piece of each (row, kv head).  The cases pin
what that decomposition could get wrong: rows of 0, 1, 15, 16, 17 tokens,
rows split over many workgroups (one long row over 256 ranges), ranges that
hold several whole rows, empty ranges (fewer pages than workgroups), page
entries outside the cache, every supported geometry, and repeated graph
replays with changing lengths (the arrival counters must return to zero).
"""

from __future__ import annotations

import pytest
import torch

from oracle.reference import paged_gqa_decode_reference
from tensorforge_amd import _native
from tensorforge_amd.workloads import make_decode_attention_case, tinyllama_decode_case
from tests.helpers import NORTH_STAR_ATOL, NORTH_STAR_RTOL, REFERENCE_TOLERANCE, assert_close

pytestmark = pytest.mark.gpu


class PageCall:
    """tf_paged_gqa_decode with the PAGES flag on a workspace sized for it."""

    def __init__(self, case, device, per_cu: int = 1, depth: int = 0):
        self.case = case
        batch, query_heads, head_dim = case.query.shape
        units = torch.cuda.get_device_properties(device).multi_processor_count
        rows = 2 * units * per_cu * query_heads
        stride = 1 << (head_dim - 1).bit_length()
        self.partial_max = torch.empty(rows, dtype=torch.float32, device=device)
        self.partial_sum = torch.empty(rows, dtype=torch.float32, device=device)
        self.partial_acc = torch.empty((rows, stride), dtype=torch.float32, device=device)
        self.counters = torch.zeros(max(batch, 1) * case.key_cache.shape[2], dtype=torch.int32,
                                    device=device)
        self.rows, self.stride = rows, stride
        self.flags = (_native.TF_ATTENTION_FLAG_PAGES
                      | (per_cu << _native.TF_ATTENTION_WAVES_PER_CU_SHIFT)
                      | (depth << _native.TF_ATTENTION_DEPTH_SHIFT))

    def __call__(self, output, lengths=None, stream=None, max_context=None):
        case = self.case
        batch, query_heads, head_dim = case.query.shape
        num_blocks, block_size, kv_heads, _ = case.key_cache.shape
        width = case.block_tables.shape[1]
        lengths = case.context_lengths if lengths is None else lengths
        if stream is None:
            stream = torch.cuda.current_stream().cuda_stream
        _native.check(_native.library().tf_paged_gqa_decode(
            case.query.data_ptr(), case.key_cache.data_ptr(), case.value_cache.data_ptr(),
            case.block_tables.data_ptr(), lengths.data_ptr(), output.data_ptr(),
            self.partial_max.data_ptr(), self.partial_sum.data_ptr(), self.partial_acc.data_ptr(),
            self.counters.data_ptr(), self.rows, self.stride, batch, query_heads, kv_heads,
            head_dim, num_blocks, block_size, width, max_context or width * block_size, 1,
            case.scale, _native.dtype_code(case.query.dtype), self.flags, stream), "pages call")
        return output


def _expected(cpu_case, lengths):
    rows = [r for r, n in enumerate(lengths) if n > 0]
    want = paged_gqa_decode_reference(
        cpu_case.query[rows], cpu_case.key_cache, cpu_case.value_cache,
        cpu_case.block_tables[rows], cpu_case.context_lengths[rows], scale=cpu_case.scale)
    return rows, want


def _check(cpu_case, actual, what, tol=None):
    lengths = cpu_case.lengths
    rows, want = _expected(cpu_case, lengths)
    atol, rtol = (NORTH_STAR_ATOL, NORTH_STAR_RTOL) if tol is None else (tol, tol)
    assert_close(actual.cpu()[rows], want, atol, rtol, what)
    empty = [r for r, n in enumerate(lengths) if n <= 0]
    if empty:
        assert bool((actual.cpu()[empty] == 0).all()), f"{what}: empty rows not zero"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize(("per_cu", "depth"), [(1, 0), (2, 2), (1, 4)])
def test_config2_batch(device, dtype, per_cu, depth):
    cpu = tinyllama_decode_case(seed=0, dtype=dtype)
    call = PageCall(cpu.to(device), device, per_cu, depth)
    out = torch.full_like(call.case.query, float("nan"))
    call(out)
    torch.cuda.synchronize()
    _check(cpu, out, f"cfg2 {dtype} per_cu {per_cu} depth {depth}")
    assert int(call.counters.abs().sum()) == 0  # every counter back at zero


@pytest.mark.parametrize(("lengths", "heads", "head_dim"), [
    ([0, 1, 15, 16, 17, 31, 33, 2048, 700, 5, 0, 64], (32, 4), 64),
    ([2048], (32, 4), 64),                          # one row over every range
    ([3] * 40 + [1000, 0, 1], (32, 4), 64),         # ranges of many whole rows
    ([17, 900, 250, 1], (32, 8), 64),               # group 4, 8 kv heads (1 KB rows)
    ([129, 1024, 7, 600], (32, 4), 128),            # head_dim 128 (1 KB rows)
    ([100, 33, 480, 255], (8, 2), 32),              # the config-1 model's geometry
    ([64, 500, 1], (16, 1), 128),                   # group 16, one kv head
])
def test_ragged_rows_and_geometries(device, lengths, heads, head_dim):
    query_heads, kv_heads = heads
    cpu = make_decode_attention_case(lengths, query_heads=query_heads, kv_heads=kv_heads,
                                     head_dim=head_dim, block_size=16, dtype=torch.bfloat16,
                                     seed=len(lengths) + head_dim, table_width=128)
    call = PageCall(cpu.to(device), device)
    out = torch.full_like(call.case.query, float("nan"))
    call(out)
    torch.cuda.synchronize()
    _check(cpu, out, f"pages {lengths[:6]} {heads} D{head_dim}")
    assert int(call.counters.abs().sum()) == 0


def test_pages_outside_the_cache_are_skipped(device):
    """Table entries outside [0, num_blocks) contribute no tokens (the grid
    kernel's rule): equal to the same rows with those pages' tokens masked."""

    cpu = make_decode_attention_case([300, 80, 47], query_heads=32, kv_heads=4, head_dim=64,
                                     block_size=16, dtype=torch.float16, seed=5, table_width=32)
    bad = cpu.block_tables.clone()
    bad[0, 3] = -1
    bad[0, 10] = cpu.key_cache.shape[0] + 7
    bad[2, 0] = -5
    gpu = cpu.to(device)
    gpu.block_tables = bad.to(device)
    call = PageCall(gpu, device)
    out = call(torch.empty_like(gpu.query))
    # Reference form: drop the bad pages' tokens by pointing them at a page
    # of -inf keys is not expressible; compare with the grid kernel instead,
    # whose skip rule the oracle-checked tests pin.
    expected = torch.empty_like(gpu.query)
    _native.check(_native.library().tf_paged_gqa_decode(
        gpu.query.data_ptr(), gpu.key_cache.data_ptr(), gpu.value_cache.data_ptr(),
        gpu.block_tables.data_ptr(), gpu.context_lengths.data_ptr(), expected.data_ptr(),
        None, None, None, None, 0, 64, 3, 32, 4, 64, gpu.key_cache.shape[0], 16, 32, 512, 1,
        gpu.scale, _native.dtype_code(torch.float16), 0,
        torch.cuda.current_stream().cuda_stream), "grid call")
    torch.cuda.synchronize()
    tol = REFERENCE_TOLERANCE[torch.float16]
    assert_close(out, expected, tol, tol, "pages vs grid with bad table entries")


def test_graph_replays_with_changing_lengths(device):
    """One captured call replayed with different device-side lengths: every
    replay matches the oracle for its lengths, so the arrival counters are
    back at zero after each call."""

    cpu = tinyllama_decode_case(seed=3, dtype=torch.bfloat16)
    gpu = cpu.to(device)
    call = PageCall(gpu, device)
    lengths = gpu.context_lengths.clone()
    out = torch.empty_like(gpu.query)
    stream = torch.cuda.Stream(device)
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        call(out, lengths=lengths, stream=stream.cuda_stream, max_context=2048)
    torch.cuda.current_stream().wait_stream(stream)
    generator = torch.Generator().manual_seed(9)
    original = cpu.context_lengths.clone()
    for replay in range(4):
        # Within each row's table: a random fraction of its length, some zeroed.
        fraction = torch.rand(original.numel(), generator=generator)
        new = (original.float() * fraction).round().to(torch.int32)
        new[replay::7] = 0
        lengths.copy_(new.to(device))
        graph.replay()
        torch.cuda.synchronize()
        cpu.context_lengths = new
        _check(cpu, out, f"replay {replay}")
        assert int(call.counters.abs().sum()) == 0
