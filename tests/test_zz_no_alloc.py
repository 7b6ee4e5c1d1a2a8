"""tf_paged_gqa_decode_noalloc against tf_paged_gqa_decode, through the C ABI.

The no-allocation call keeps its split partials in the library's fixed
device array instead of a caller workspace; it runs the same kernels, so
its output must equal the workspace call's bit for bit.  Two split-KV calls
in a row (the second smaller, so stale partials of the first sit in the
array), a call captured in a HIP graph and replayed, a one-pass call, and
the size limit are checked.  Collected last
(``test_zz_``): it must pass alone in a fresh process and after the rest.
"""

from __future__ import annotations

import pytest
import torch

from tensorforge_amd import _native
from tensorforge_amd.kernels import PagedAttentionWorkspace
from tensorforge_amd.workloads import make_decode_attention_case
from tests.helpers import assert_bit_exact

pytestmark = pytest.mark.gpu


def _workspace_call(lib, gpu, output, split_size, num_splits, stream):
    batch, query_heads, head_dim = gpu.query.shape
    num_blocks, block_size, kv_heads, _ = gpu.key_cache.shape
    workspace = PagedAttentionWorkspace.allocate(
        batch_capacity=batch, query_heads=query_heads, head_dim=head_dim,
        max_context_length=num_splits * 256, device=gpu.query.device)
    _native.check(lib.tf_paged_gqa_decode(
        gpu.query.data_ptr(), gpu.key_cache.data_ptr(), gpu.value_cache.data_ptr(),
        gpu.block_tables.data_ptr(), gpu.context_lengths.data_ptr(), output.data_ptr(),
        workspace.partial_max.data_ptr(), workspace.partial_sum.data_ptr(),
        workspace.partial_accumulator.data_ptr(), None, workspace.partial_max.numel(),
        workspace.partial_accumulator.shape[1], batch, query_heads, kv_heads, head_dim,
        num_blocks, block_size, gpu.block_tables.shape[1], split_size, num_splits, gpu.scale,
        _native.dtype_code(gpu.query.dtype), 0, stream), "workspace call")


def _noalloc_call(lib, gpu, output, split_size, num_splits, stream):
    batch, query_heads, head_dim = gpu.query.shape
    num_blocks, block_size, kv_heads, _ = gpu.key_cache.shape
    return lib.tf_paged_gqa_decode_noalloc(
        gpu.query.data_ptr(), gpu.key_cache.data_ptr(), gpu.value_cache.data_ptr(),
        gpu.block_tables.data_ptr(), gpu.context_lengths.data_ptr(), output.data_ptr(),
        batch, query_heads, kv_heads, head_dim, num_blocks, block_size,
        gpu.block_tables.shape[1], split_size, num_splits, gpu.scale,
        _native.dtype_code(gpu.query.dtype), 0, stream)


def test_noalloc_under_graph_capture_replays_like_the_workspace_call(device):
    """The callers the entry point is for: the call captured in a HIP graph
    (torch.cuda.graph).  Collected first in this file, so in a process that
    has made no no-allocation call yet (this file alone, or the whole suite,
    where nothing else calls it) the scratch address is taken inside the
    capture.  The graph is replayed three times, with the query changed in
    place and eager work and synchronisations between replays; every replay
    must equal an eager workspace call on the same inputs bit for bit."""

    lib = _native.library()
    case = make_decode_attention_case(
        [1500, 3, 0, 640, 2048, 96], query_heads=32, kv_heads=4, head_dim=64, block_size=16,
        dtype=torch.bfloat16, seed=21, table_width=128).to(device)
    stream = torch.cuda.Stream(device)
    expected = torch.empty_like(case.query)
    captured = torch.full_like(case.query, float("nan"))
    with torch.cuda.stream(stream):
        _workspace_call(lib, case, expected, 256, 8, stream.cuda_stream)  # module loaded
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        status = _noalloc_call(lib, case, captured, 256, 8,
                               torch.cuda.current_stream(device).cuda_stream)
    _native.check(status, "no-allocation call under capture")
    generator = torch.Generator().manual_seed(22)
    for replay in range(3):
        fresh = torch.randn(case.query.shape, generator=generator).to(torch.bfloat16)
        case.query.copy_(fresh.to(device))
        torch.cuda.synchronize(device)
        graph.replay()
        torch.cuda.synchronize(device)
        _workspace_call(lib, case, expected, 256, 8,
                        torch.cuda.current_stream(device).cuda_stream)
        torch.cuda.synchronize(device)
        assert_bit_exact(captured, expected, f"graph replay {replay}")
        assert bool(torch.isfinite(captured.float()).all())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_noalloc_matches_the_workspace_call_twice_in_a_row(device, dtype):
    lib = _native.library()
    stream = torch.cuda.current_stream(device).cuda_stream
    # First call: 24 rows (3 empty) up to 2k tokens, 256-token splits.
    big = make_decode_attention_case(
        [2048, 17, 0, 700, 1333, 256, 1, 0] * 2 + [2000, 640, 0, 1500, 96, 32, 1024, 511],
        query_heads=32, kv_heads=4, head_dim=64, block_size=16, dtype=dtype, seed=11,
        table_width=128).to(device)
    # Second call: fewer, shorter rows and another geometry.
    small = make_decode_attention_case(
        [300, 5, 129], query_heads=8, kv_heads=2, head_dim=128, block_size=16, dtype=dtype,
        seed=12, table_width=32).to(device)
    for case, split_size, num_splits in ((big, 256, 8), (small, 128, 4)):
        expected = torch.full_like(case.query, float("nan"))
        actual = torch.full_like(case.query, float("nan"))
        _workspace_call(lib, case, expected, split_size, num_splits, stream)
        _native.check(_noalloc_call(lib, case, actual, split_size, num_splits, stream),
                      "no-allocation call")
        torch.cuda.synchronize(device)
        assert_bit_exact(actual, expected, f"split {split_size} x {num_splits}")
        assert bool(torch.isfinite(actual.float()).all())


def test_noalloc_one_pass_and_size_limit(device):
    lib = _native.library()
    stream = torch.cuda.current_stream(device).cuda_stream
    case = make_decode_attention_case(
        [900, 3, 0, 64], query_heads=32, kv_heads=4, head_dim=64, block_size=16,
        dtype=torch.bfloat16, seed=13, table_width=64).to(device)
    expected = torch.empty_like(case.query)
    actual = torch.empty_like(case.query)
    _workspace_call(lib, case, expected, 1024, 1, stream)
    _native.check(_noalloc_call(lib, case, actual, 1024, 1, stream), "no-allocation one pass")
    torch.cuda.synchronize(device)
    assert_bit_exact(actual, expected, "one pass")
    # 4 rows x 32 heads x 2048 splits x (64 + 2) floats > 8 MiB: rejected, nothing launched.
    status = _noalloc_call(lib, case, actual, 32, 2048, stream)
    assert status == 1 and b"no-allocation scratch" in lib.tf_last_error()
