"""Parity of the gfx950 paged GQA decode attention with the CPU oracle.

Mirrors tests/test_decode_attention.py of the reference (known answer :38-57,
shape/dtype grid with flipped tables :60-104, split-KV selection and
caller-owned output :107-162) and adds the BASELINE configurations, ragged
and zero-length rows, page sizes that straddle the 16-token MFMA tile,
MFMA/generic agreement and HIP-graph replay.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from helpers import NORTH_STAR_ATOL, NORTH_STAR_RTOL, REFERENCE_TOLERANCE, assert_close
from oracle.reference import paged_gqa_decode_reference, paged_gqa_decode_split_reference
from tensorforge_amd import _native
from tensorforge_amd.kernels import (
    PagedAttentionWorkspace,
    paged_gqa_decode_attention,
    selected_attention_autotune_config,
    selected_attention_launch,
    set_attention_split_size,
)
from tensorforge_amd.workloads import (
    llama3_long_context_case,
    make_decode_attention_case,
    tinyllama_decode_case,
)

pytestmark = pytest.mark.gpu


def _active_rows(lengths: list[int]) -> list[int]:
    return [row for row, ctx in enumerate(lengths) if ctx > 0]


def _check_against_oracle(case, actual, atol, rtol, what):
    rows = _active_rows(case.lengths)
    cpu = case.to("cpu")
    expected = paged_gqa_decode_reference(
        cpu.query[rows],
        cpu.key_cache,
        cpu.value_cache,
        cpu.block_tables[rows],
        cpu.context_lengths[rows],
        scale=case.scale,
    )
    assert_close(actual[rows], expected, atol, rtol, what)
    for row, ctx in enumerate(case.lengths):
        if ctx <= 0:
            assert bool((actual[row] == 0).all()), f"{what}: zero-length row {row} not zero"


def test_reference_known_answer_noncontiguous_table(device):
    query = torch.randn(1, 4, 64, dtype=torch.float32)
    key_cache = torch.randn(3, 2, 2, 64, dtype=torch.float32)
    value_cache = torch.randn_like(key_cache)
    block_tables = torch.tensor([[2, 0]], dtype=torch.int32)
    context_lengths = torch.tensor([3], dtype=torch.int32)
    actual = paged_gqa_decode_attention(
        query.to(device), key_cache.to(device), value_cache.to(device),
        block_tables.to(device), context_lengths.to(device),
    )
    expected = paged_gqa_decode_reference(query, key_cache, value_cache, block_tables,
                                          context_lengths)
    assert_close(actual, expected, 1e-5, 1e-5, "known answer")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize(
    ("batch", "query_heads", "kv_heads", "head_dim", "block_size", "lengths"),
    [
        (2, 8, 2, 80, 4, [1, 7]),
        (2, 32, 8, 128, 16, [17, 31]),
        (1, 8, 1, 64, 16, [129]),
        (1, 32, 8, 128, 16, [2048]),
    ],
)
def test_shape_dtype_grid_with_flipped_tables(device, batch, query_heads, kv_heads, head_dim,
                                              block_size, lengths, dtype):
    logical_blocks = (max(lengths) + block_size - 1) // block_size
    physical_blocks = batch * logical_blocks
    query = torch.randn(batch, query_heads, head_dim).to(dtype)
    key_cache = torch.randn(physical_blocks, block_size, kv_heads, head_dim).to(dtype)
    value_cache = torch.randn_like(key_cache)
    block_tables = (
        torch.arange(physical_blocks, dtype=torch.int32).view(batch, logical_blocks).flip(1)
        .contiguous()
    )
    context_lengths = torch.tensor(lengths, dtype=torch.int32)
    actual = paged_gqa_decode_attention(
        query.to(device), key_cache.to(device), value_cache.to(device),
        block_tables.to(device), context_lengths.to(device),
    )
    expected = paged_gqa_decode_reference(query, key_cache, value_cache, block_tables,
                                          context_lengths)
    tol = REFERENCE_TOLERANCE[dtype]
    assert_close(actual, expected, tol, tol, f"grid {dtype} {lengths}")


def test_long_context_with_few_heads_selects_split_kv_path(device):
    query = torch.randn(1, 8, 64).to(torch.float16)
    key_cache = torch.randn(128, 16, 4, 64).to(torch.float16)
    value_cache = torch.randn_like(key_cache)
    block_tables = torch.arange(128, dtype=torch.int32).view(1, 128)
    context_lengths = torch.tensor([2048], dtype=torch.int32)
    q, k, v = query.to(device), key_cache.to(device), value_cache.to(device)
    t, c = block_tables.to(device), context_lengths.to(device)
    output = torch.empty_like(q)
    workspace = PagedAttentionWorkspace.allocate(
        batch_capacity=1, query_heads=8, head_dim=64, max_context_length=2048, device=device,
    )
    actual = paged_gqa_decode_attention(q, k, v, t, c, max_context_length=2048, output=output,
                                        workspace=workspace)
    selected = selected_attention_autotune_config()
    one_pass = paged_gqa_decode_attention(q, k, v, t, c, max_context_length=2048,
                                          attention_path="one_pass")
    expected = paged_gqa_decode_reference(query, key_cache, value_cache, block_tables,
                                          context_lengths)
    assert actual is output and actual.data_ptr() == output.data_ptr()
    assert_close(actual, expected, 3e-3, 3e-3, "split")
    assert_close(one_pass, expected, 3e-3, 3e-3, "one pass")
    # The reference's own assertion, unchanged (tests/test_decode_attention.py:158-162).
    assert selected == {"path": "split_kv", "split_size": 256, "num_splits": 8}


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_tinyllama_batch64_config(device, dtype):
    """64 rows ctx U[128, 2048] + 8 zero-length rows, one
    pass with four wavefronts per kv head (the plan for a wide batch), and
    the forced split-KV path."""

    case = tinyllama_decode_case(seed=0, dtype=dtype)
    gpu = case.to(device)
    output = paged_gqa_decode_attention(
        gpu.query, gpu.key_cache, gpu.value_cache, gpu.block_tables, gpu.context_lengths,
        scale=case.scale, max_context_length=2048,
    )
    assert selected_attention_launch()["kernel"] == "mfma"
    assert selected_attention_launch()["waves_per_head"] == 4
    _check_against_oracle(case, output.cpu(), NORTH_STAR_ATOL, NORTH_STAR_RTOL, f"cfg2 {dtype}")
    split = paged_gqa_decode_attention(
        gpu.query, gpu.key_cache, gpu.value_cache, gpu.block_tables, gpu.context_lengths,
        scale=case.scale, max_context_length=2048, attention_path="split_kv",
    )
    assert selected_attention_autotune_config()["split_size"] == 576
    _check_against_oracle(case, split.cpu(), NORTH_STAR_ATOL, NORTH_STAR_RTOL, f"cfg2 split {dtype}")


@pytest.mark.parametrize("split_size", [0, 256])
@pytest.mark.parametrize(("heads_per_wg", "waves_per_head", "tokens_per_wave"),
                         [(1, 2, 0), (1, 3, 0), (1, 4, 0), (1, 8, 0), (2, 2, 0), (2, 4, 0),
                          (4, 2, 0), (1, 3, 768), (1, 8, 256), (2, 4, 64)])
def test_grid_kernel_multi_wave_workgroups(device, heads_per_wg, waves_per_head,
                                           tokens_per_wave, split_size):
    """Workgroups of several kv heads and several wavefronts per head (their
    states combined in LDS), in one pass and with 256-token partitions, on
    ragged rows (including one shorter than a chunk and an empty one); with
    a token budget per wavefront, rows use only as many as they need."""

    lengths = [2048, 1, 700, 0, 1333, 31, 96, 2000]
    case = make_decode_attention_case(
        lengths, query_heads=32, kv_heads=4, head_dim=64, block_size=16, dtype=torch.bfloat16,
        seed=heads_per_wg * 10 + waves_per_head + tokens_per_wave,
    )
    gpu = case.to(device)
    workspace = PagedAttentionWorkspace.allocate(
        batch_capacity=len(lengths), query_heads=32, head_dim=64, max_context_length=2048,
        device=device,
    )
    flags = ((heads_per_wg << _native.TF_ATTENTION_HEADS_PER_WG_SHIFT)
             | (waves_per_head << _native.TF_ATTENTION_WAVES_PER_CU_SHIFT)
             | ((tokens_per_wave // 64) << _native.TF_ATTENTION_TOKENS_PER_WAVE_SHIFT))
    out = torch.full_like(gpu.query, float("nan"))
    if split_size == 0:
        _raw_decode(gpu, out, flags, gpu.block_tables.shape[1] * 16, 1, workspace)
    else:
        _raw_decode(gpu, out, flags, split_size, 2048 // split_size, workspace)
    _check_against_oracle(case, out.cpu(), NORTH_STAR_ATOL, NORTH_STAR_RTOL,
                          f"hpw {heads_per_wg} wph {waves_per_head} tpw {tokens_per_wave} "
                          f"split {split_size}")


@pytest.mark.parametrize(("head_dim", "dtype"), [(32, torch.float16), (64, torch.float16),
                                                 (128, torch.bfloat16), (128, torch.float16)])
def test_whole_row_loads_across_head_dims(device, head_dim, dtype):
    """Several wavefronts per kv head load K / V as whole token rows and
    stage K through LDS; every head_dim, both 16-bit types, ragged rows
    (partial chunks, a one-token row, an empty row) and GQA groups of 4."""

    lengths = [1000, 1, 577, 0, 1152, 33, 2047, 16]
    case = make_decode_attention_case(
        lengths, query_heads=16, kv_heads=4, head_dim=head_dim, block_size=16, dtype=dtype,
        seed=head_dim + (dtype == torch.float16),
    )
    gpu = case.to(device)
    workspace = PagedAttentionWorkspace.allocate(
        batch_capacity=len(lengths), query_heads=16, head_dim=head_dim, max_context_length=2048,
        device=device,
    )
    flags = ((1 << _native.TF_ATTENTION_HEADS_PER_WG_SHIFT)
             | (4 << _native.TF_ATTENTION_WAVES_PER_CU_SHIFT)
             | ((576 // 64) << _native.TF_ATTENTION_TOKENS_PER_WAVE_SHIFT))
    out = torch.full_like(gpu.query, float("nan"))
    _raw_decode(gpu, out, flags, gpu.block_tables.shape[1] * 16, 1, workspace)
    _check_against_oracle(case, out.cpu(), NORTH_STAR_ATOL, NORTH_STAR_RTOL,
                          f"whole rows D{head_dim} {dtype}")


def test_llama3_long_context_split_kv(device):
    """contexts 8k..32k, 512-token partitions + LSE merge."""

    case = llama3_long_context_case(seed=0)
    gpu = case.to(device)
    previous = set_attention_split_size(512)
    try:
        workspace = PagedAttentionWorkspace.allocate(
            batch_capacity=4, query_heads=32, head_dim=128, max_context_length=32768,
            device=device,
        )
        output = paged_gqa_decode_attention(
            gpu.query, gpu.key_cache, gpu.value_cache, gpu.block_tables, gpu.context_lengths,
            max_context_length=32768, workspace=workspace,
        )
        assert selected_attention_autotune_config() == {
            "path": "split_kv", "split_size": 512, "num_splits": 64,
        }
        # Two wavefronts stream each caller-fixed partition of <= 768 tokens.
        assert selected_attention_launch()["waves_per_head"] == 2
    finally:
        set_attention_split_size(previous)
    _check_against_oracle(case, output.cpu(), NORTH_STAR_ATOL, NORTH_STAR_RTOL, "cfg3")


def test_llama3_long_context_auto_plan(device):
    """BASELINE config 3 under the entry point's own plan: partitions sized
    on the device from the rows' lengths (at least 256 tokens, 128 slots per
    group of four kv heads) with two wavefronts per kv head (whole-row loads
    at D 128), then the merge launch."""

    case = llama3_long_context_case(seed=1)
    gpu = case.to(device)
    output = paged_gqa_decode_attention(
        gpu.query, gpu.key_cache, gpu.value_cache, gpu.block_tables, gpu.context_lengths,
        max_context_length=32768,
    )
    assert selected_attention_autotune_config() == {
        "path": "split_kv", "split_size": 256, "num_splits": 128,
    }
    assert selected_attention_launch()["waves_per_head"] == 2
    assert selected_attention_launch()["heads_per_workgroup"] == 4
    assert selected_attention_launch()["balanced_partitions"]
    _check_against_oracle(case, output.cpu(), NORTH_STAR_ATOL, NORTH_STAR_RTOL, "cfg3 auto")


@pytest.mark.parametrize("block_size", [1, 4, 8, 12, 16, 32, 48])
@pytest.mark.parametrize("path", ["one_pass", "split_kv"])
def test_ragged_rows_any_page_size(device, block_size, path):
    lengths = [1, 15, 16, 17, 33, 0, 250, 513, 64, 0]
    case = make_decode_attention_case(
        lengths, query_heads=16, kv_heads=2, head_dim=64, block_size=block_size,
        dtype=torch.bfloat16, seed=block_size, extra_pages=3,
    )
    gpu = case.to(device)
    previous = set_attention_split_size(64)
    try:
        workspace = PagedAttentionWorkspace.allocate(
            batch_capacity=len(lengths), query_heads=16, head_dim=64,
            max_context_length=4 * 513, device=device,
        )
        output = paged_gqa_decode_attention(
            gpu.query, gpu.key_cache, gpu.value_cache, gpu.block_tables, gpu.context_lengths,
            max_context_length=513, workspace=workspace, attention_path=path,
        )
    finally:
        set_attention_split_size(previous)
    _check_against_oracle(case, output.cpu(), NORTH_STAR_ATOL, NORTH_STAR_RTOL,
                          f"ragged page {block_size} {path}")


@pytest.mark.parametrize(("query_heads", "kv_heads", "head_dim"),
                         [(8, 2, 32), (32, 8, 128), (16, 1, 64), (4, 4, 64), (64, 2, 64)])
def test_group_and_head_dim_variants(device, query_heads, kv_heads, head_dim):
    lengths = [37, 300, 1]
    case = make_decode_attention_case(
        lengths, query_heads=query_heads, kv_heads=kv_heads, head_dim=head_dim, block_size=16,
        dtype=torch.float16, seed=query_heads + head_dim,
    )
    gpu = case.to(device)
    output = paged_gqa_decode_attention(
        gpu.query, gpu.key_cache, gpu.value_cache, gpu.block_tables, gpu.context_lengths,
    )
    _check_against_oracle(case, output.cpu(), 3e-3, 3e-3, f"G={query_heads // kv_heads} D={head_dim}")


def _raw_decode(gpu, out, flags, split_size, num_splits, workspace, counters=None, query=None):
    query = gpu.query if query is None else query
    head_bucket = workspace.partial_accumulator.shape[1]
    batch, query_heads, head_dim = query.shape
    num_blocks, block_size, kv_heads, _ = gpu.key_cache.shape
    status = _native.library().tf_paged_gqa_decode(
        query.data_ptr(), gpu.key_cache.data_ptr(), gpu.value_cache.data_ptr(),
        gpu.block_tables.data_ptr(), gpu.context_lengths.data_ptr(), out.data_ptr(),
        workspace.partial_max.data_ptr(), workspace.partial_sum.data_ptr(),
        workspace.partial_accumulator.data_ptr(), counters, workspace.partial_max.numel(),
        head_bucket,
        batch, query_heads, kv_heads, head_dim, num_blocks, block_size,
        gpu.block_tables.shape[1], split_size, num_splits, ctypes.c_float(gpu.scale),
        _native.dtype_code(gpu.query.dtype), flags, _native.current_stream(gpu.query.device),
    )
    _native.check(status, "tf_paged_gqa_decode")


def test_mfma_and_generic_kernels_agree_through_the_c_abi(device):
    lengths = [700, 2048, 5, 0, 1000]
    case = make_decode_attention_case(
        lengths, query_heads=32, kv_heads=4, head_dim=64, block_size=16, dtype=torch.bfloat16,
        seed=7,
    )
    gpu = case.to(device)
    workspace = PagedAttentionWorkspace.allocate(
        batch_capacity=len(lengths), query_heads=32, head_dim=64, max_context_length=2048,
        device=device,
    )
    counters = workspace.split_counters.data_ptr()
    outputs = {}
    for name, flags, counter_ptr in (
        ("mfma, merge kernel", 0, None),
        ("mfma grid, in-kernel merge", 0, counters),
        ("generic, merge kernel", _native.TF_ATTENTION_FLAG_FORCE_GENERIC, None),
        ("generic, in-kernel merge", _native.TF_ATTENTION_FLAG_FORCE_GENERIC, counters),
    ):
        out = torch.full_like(gpu.query, float("nan"))
        _raw_decode(gpu, out, flags, 256, 8, workspace, counter_ptr)
        torch.cuda.synchronize()
        outputs[name] = out.cpu()
        _check_against_oracle(case, outputs[name], NORTH_STAR_ATOL, NORTH_STAR_RTOL, name)
    assert int(workspace.split_counters.sum()) == 0, "arrival counters were not reset"
    assert_close(outputs["mfma, merge kernel"], outputs["generic, merge kernel"],
                 NORTH_STAR_ATOL, NORTH_STAR_RTOL, "mfma vs generic")
    assert_close(outputs["mfma, merge kernel"], outputs["mfma grid, in-kernel merge"],
                 1e-2, 1e-2, "merge kernel vs grid kernel with in-kernel merge")


def test_split_partials_follow_split_oracle(device):
    lengths = [129, 1000]
    case = make_decode_attention_case(
        lengths, query_heads=8, kv_heads=2, head_dim=64, block_size=16, dtype=torch.float32,
        seed=11,
    )
    gpu = case.to(device)
    previous = set_attention_split_size(128)
    try:
        workspace = PagedAttentionWorkspace.allocate(
            batch_capacity=2, query_heads=8, head_dim=64, max_context_length=2048, device=device,
        )
        output = paged_gqa_decode_attention(
            gpu.query, gpu.key_cache, gpu.value_cache, gpu.block_tables, gpu.context_lengths,
            max_context_length=1000, workspace=workspace,
        )
    finally:
        set_attention_split_size(previous)
    cpu = case.to("cpu")
    expected = paged_gqa_decode_split_reference(
        cpu.query, cpu.key_cache, cpu.value_cache, cpu.block_tables, cpu.context_lengths,
        split_size=128, scale=case.scale,
    )
    assert_close(output.cpu(), expected, 1e-5, 1e-5, "split fp32")


def test_graph_replay_is_address_stable_and_tracks_device_lengths(device):
    lengths = [300, 17, 1024, 64]
    case = make_decode_attention_case(
        lengths, query_heads=32, kv_heads=4, head_dim=64, block_size=16, dtype=torch.bfloat16,
        seed=3, table_width=64,
    )
    gpu = case.to(device)
    output = torch.empty_like(gpu.query)
    workspace = PagedAttentionWorkspace.allocate(
        batch_capacity=4, query_heads=32, head_dim=64, max_context_length=1024, device=device,
    )

    def run():
        paged_gqa_decode_attention(
            gpu.query, gpu.key_cache, gpu.value_cache, gpu.block_tables, gpu.context_lengths,
            scale=case.scale, max_context_length=1024, output=output, workspace=workspace,
        )

    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        run()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    for replay, new_lengths in enumerate(([300, 17, 1024, 0], [299, 16, 1000, 5], [1, 0, 1024, 64])):
        gpu.context_lengths.copy_(torch.tensor(new_lengths, dtype=torch.int32))
        graph.replay()
        torch.cuda.synchronize()
        replayed = output.clone()
        run()  # eager on the same buffers
        torch.cuda.synchronize()
        assert torch.equal(replayed.view(torch.int16), output.view(torch.int16)), (
            f"replay {replay} differs from eager"
        )
        case.context_lengths = torch.tensor(new_lengths, dtype=torch.int32)
        _check_against_oracle(case, replayed.cpu(), NORTH_STAR_ATOL, NORTH_STAR_RTOL,
                              f"replay {replay}")


def test_validation_matches_reference_messages(device):
    query = torch.randn(1, 4, 64, device=device)
    key_cache = torch.randn(3, 2, 2, 64, device=device)
    tables = torch.tensor([[2, 0]], dtype=torch.int32, device=device)
    lengths = torch.tensor([3], dtype=torch.int32, device=device)
    with pytest.raises(ValueError, match="CUDA"):
        paged_gqa_decode_attention(query.cpu(), key_cache, key_cache, tables, lengths)
    with pytest.raises(TypeError, match="int32"):
        paged_gqa_decode_attention(query, key_cache, key_cache, tables.long(), lengths)
    with pytest.raises(ValueError, match="attention_path"):
        paged_gqa_decode_attention(query, key_cache, key_cache, tables, lengths,
                                   attention_path="bogus")
    with pytest.raises(ValueError, match="table capacity"):
        paged_gqa_decode_attention(query, key_cache, key_cache, tables, lengths,
                                   max_context_length=5)
    small = PagedAttentionWorkspace.allocate(batch_capacity=1, query_heads=1, head_dim=64,
                                             max_context_length=1, device=device)
    with pytest.raises(ValueError, match="capacity"):
        paged_gqa_decode_attention(query, key_cache, key_cache, tables, lengths,
                                   attention_path="split_kv", workspace=small)
    grad_query = query.clone().requires_grad_(True)
    with pytest.raises(RuntimeError, match="inference-only"):
        paged_gqa_decode_attention(grad_query, key_cache, key_cache, tables, lengths)


def test_in_kernel_merge_is_fresh_on_every_call(device):
    """Back-to-back calls on one workspace with changing inputs: every call
    must merge its own partials (counters reset, no stale partial reads)."""

    lengths = [2048, 1500, 700, 129, 0, 1999, 256, 257]
    case = make_decode_attention_case(
        lengths, query_heads=32, kv_heads=4, head_dim=64, block_size=16, dtype=torch.bfloat16,
        seed=21,
    )
    gpu = case.to(device)
    workspace = PagedAttentionWorkspace.allocate(
        batch_capacity=len(lengths), query_heads=32, head_dim=64, max_context_length=2048,
        device=device,
    )
    plain = PagedAttentionWorkspace(workspace.partial_max.clone(), workspace.partial_sum.clone(),
                                    workspace.partial_accumulator.clone())
    generator = torch.Generator().manual_seed(5)
    queries = [torch.randn(case.query.shape, generator=generator).to(torch.bfloat16).to(device)
               for _ in range(6)]
    fused_out = [torch.empty_like(gpu.query) for _ in queries]
    for q, out in zip(queries, fused_out):
        # The C ABI's in-kernel merge: arrival counters given.
        _raw_decode(gpu, out, 0, 256, 8, workspace, workspace.split_counters.data_ptr(), query=q)
    for index, (q, out) in enumerate(zip(queries, fused_out)):
        separate = paged_gqa_decode_attention(q, gpu.key_cache, gpu.value_cache,
                                              gpu.block_tables, gpu.context_lengths,
                                              max_context_length=2048, workspace=plain)
        assert selected_attention_launch()["in_kernel_merge"] is False
        assert_close(out.cpu(), separate.cpu(), 1e-2, 1e-2, f"call {index}")
    torch.cuda.synchronize()
    assert int(workspace.split_counters.sum()) == 0
    case.query = queries[-1].cpu()
    _check_against_oracle(case, fused_out[-1].cpu(), NORTH_STAR_ATOL, NORTH_STAR_RTOL, "last call")


def test_merge_result_does_not_depend_on_its_wavefront_count(device):
    """The merge launch gives each (row, head) one wavefront per batch of 16
    partitions (up to four; one beyond 16 batches) and adds the batch sums
    in batch order, so the same partials merge to the same bits whatever
    the partition count the launch declares: here the partials of a call
    with 20 partitions of 64 tokens (two batches: two wavefronts), laid out
    again for 70 declared partitions (four wavefronts) and for 300 (one
    wavefront walking the batches), with NaN in every slot past the rows'
    own partitions (read ahead, never used)."""

    lengths = [1280, 1, 0, 700, 1279, 64, 65, 1024]
    case = make_decode_attention_case(lengths, query_heads=8, kv_heads=2, head_dim=64,
                                      block_size=16, dtype=torch.bfloat16, seed=31)
    gpu = case.to(device)
    lib = _native.library()
    batch, hq, d = gpu.query.shape
    blocks, page, hkv, _ = gpu.key_cache.shape
    split, used = 64, 20
    stream = _native.current_stream(device)
    partials = {}
    for declared in (used, 70, 300):
        rows = batch * hq * declared
        partials[declared] = (torch.full((rows,), float("nan"), device=device),
                              torch.full((rows,), float("nan"), device=device),
                              torch.full((rows, d), float("nan"), device=device))
    pm, ps, pa = partials[used]
    _native.check(lib.tf_paged_gqa_decode_partials(
        gpu.query.data_ptr(), gpu.key_cache.data_ptr(), gpu.value_cache.data_ptr(),
        gpu.block_tables.data_ptr(), gpu.context_lengths.data_ptr(), pm.data_ptr(),
        ps.data_ptr(), pa.data_ptr(), pm.numel(), d, batch, hq, hkv, d, blocks, page,
        gpu.block_tables.shape[1], split, used, gpu.scale, _native.dtype_code(torch.bfloat16), 0,
        stream), "partials")
    for declared in (70, 300):
        qm, qs, qa = partials[declared]
        qm.view(batch, hq, declared)[:, :, :used] = pm.view(batch, hq, used)
        qs.view(batch, hq, declared)[:, :, :used] = ps.view(batch, hq, used)
        qa.view(batch, hq, declared, d)[:, :, :used] = pa.view(batch, hq, used, d)
    outputs = {}
    for declared, (qm, qs, qa) in partials.items():
        out = torch.full_like(gpu.query, float("nan"))
        _native.check(lib.tf_paged_gqa_decode_merge(
            qm.data_ptr(), qs.data_ptr(), qa.data_ptr(), gpu.context_lengths.data_ptr(),
            out.data_ptr(), qm.numel(), d, batch, hq, d, split, declared, used * split,
            _native.dtype_code(torch.bfloat16), stream), f"merge of {declared}")
        outputs[declared] = out
    torch.cuda.synchronize()
    assert torch.equal(outputs[used].view(torch.int16), outputs[70].view(torch.int16))
    assert torch.equal(outputs[used].view(torch.int16), outputs[300].view(torch.int16))
    live = [r for r, c in enumerate(lengths) if c > 0]
    want = paged_gqa_decode_reference(case.query[live], case.key_cache, case.value_cache,
                                      case.block_tables[live], case.context_lengths[live],
                                      scale=case.scale)
    assert_close(outputs[used].cpu()[live], want, NORTH_STAR_ATOL, NORTH_STAR_RTOL, "merged")
    assert bool((outputs[used].cpu()[[2]] == 0).all())
