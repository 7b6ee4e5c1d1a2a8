"""The VALU form of the grid attention kernel (TF_ATTENTION_FLAG_VALU)
against the oracle, through the C ABI.

The VALU form keeps the MFMA kernel's grid, loads and LDS staging and
computes the two products on the VALU (packed two-element dot products for
the scores, fp32 FMAs for P.V); it exists to compare the two product forms
at group sizes 4 and 8.  Its results must match the oracle to the same
tolerance as the MFMA form's, with one and several wavefronts per kv head,
ragged and zero-length rows, and split partitions; geometries it does not
cover are rejected.
"""

from __future__ import annotations

import pytest
import torch

from helpers import NORTH_STAR_ATOL, NORTH_STAR_RTOL, assert_close
from oracle.reference import paged_gqa_decode_reference
from tensorforge_amd import _native
from tensorforge_amd.workloads import make_decode_attention_case, tinyllama_decode_case

pytestmark = pytest.mark.gpu


def _call(case, output, flags, *, split_size=None, stream=None):
    batch, query_heads, head_dim = case.query.shape
    num_blocks, block_size, kv_heads, _ = case.key_cache.shape
    width = case.block_tables.shape[1]
    capacity = (width * block_size + 31) // 32 * 32
    split = split_size or capacity
    splits = (capacity + split - 1) // split
    partials = None
    if splits > 1:
        rows = batch * query_heads * splits
        partials = (torch.empty(rows, device=case.query.device),
                    torch.empty(rows, device=case.query.device),
                    torch.empty((rows, head_dim), device=case.query.device))
    status = _native.library().tf_paged_gqa_decode(
        case.query.data_ptr(), case.key_cache.data_ptr(), case.value_cache.data_ptr(),
        case.block_tables.data_ptr(), case.context_lengths.data_ptr(), output.data_ptr(),
        partials[0].data_ptr() if partials else None, partials[1].data_ptr() if partials else None,
        partials[2].data_ptr() if partials else None, None,
        batch * query_heads * splits if partials else 0, head_dim, batch, query_heads, kv_heads,
        head_dim, num_blocks, block_size, width, split, splits, case.scale,
        _native.dtype_code(case.query.dtype), flags,
        stream if stream is not None else torch.cuda.current_stream().cuda_stream)
    return status, partials


def _merge(partials, lengths, split_size, query_heads, dtype):
    """Host log-sum-exp of the written partitions (ceil(ctx / split) per row;
    the kernel leaves partitions past a row's length unwritten)."""

    batch = len(lengths)
    splits = partials[0].numel() // (batch * query_heads)
    m, s, acc = (t.view(batch, query_heads, splits, -1) for t in partials)
    m, s = m[..., 0].clone(), s[..., 0]
    valid = torch.tensor([[j < (n + split_size - 1) // split_size for j in range(splits)]
                          for n in lengths], device=m.device)
    m = torch.where(valid.unsqueeze(1), m, torch.full_like(m, float("-inf")))
    s = torch.where(valid.unsqueeze(1), s, torch.zeros_like(s))
    acc = torch.where(valid.unsqueeze(1).unsqueeze(-1), acc, torch.zeros_like(acc))
    top = m.max(dim=2, keepdim=True).values
    weight = torch.where(m == float("-inf"), torch.zeros_like(m), torch.exp2(m - top))
    num = (weight.unsqueeze(-1) * acc).sum(2)
    den = (weight * s).sum(2).unsqueeze(-1)
    return torch.where(den > 0, num / den, torch.zeros_like(num)).to(dtype)


def _check(cpu, actual, what):
    rows = [r for r, n in enumerate(cpu.lengths) if n > 0]
    want = paged_gqa_decode_reference(cpu.query[rows], cpu.key_cache, cpu.value_cache,
                                      cpu.block_tables[rows], cpu.context_lengths[rows],
                                      scale=cpu.scale)
    assert_close(actual.cpu()[rows], want, NORTH_STAR_ATOL, NORTH_STAR_RTOL, what)
    empty = [r for r, n in enumerate(cpu.lengths) if n <= 0]
    if empty:
        assert bool((actual.cpu()[empty] == 0).all()), f"{what}: empty rows not zero"


# One pass with the entry point's multi-wavefront plan (4 per kv head, 576
# tokens each) and with one wavefront per (row, kv head).
PLANS = {
    "4 waves": (_native.TF_ATTENTION_FLAG_VALU | (1 << _native.TF_ATTENTION_HEADS_PER_WG_SHIFT)
                | (4 << _native.TF_ATTENTION_WAVES_PER_CU_SHIFT)
                | (9 << _native.TF_ATTENTION_TOKENS_PER_WAVE_SHIFT)),
    "1 wave": _native.TF_ATTENTION_FLAG_VALU,
}


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("plan", sorted(PLANS))
def test_config2_group8(device, dtype, plan):
    cpu = tinyllama_decode_case(seed=0, dtype=dtype)
    gpu = cpu.to(device)
    out = torch.full_like(gpu.query, float("nan"))
    status, _ = _call(gpu, out, PLANS[plan])
    assert status == 0, _native.library().tf_last_error()
    torch.cuda.synchronize()
    _check(cpu, out, f"valu cfg2 {dtype} {plan}")


@pytest.mark.parametrize(("heads", "lengths"), [
    ((16, 4), [0, 1, 15, 16, 17, 33, 700, 2048, 5]),   # group 4
    ((32, 4), [31, 32, 64, 129, 1000, 0, 3]),          # group 8
    ((32, 8), [100, 257, 1, 1500]),                    # group 4, 8 kv heads
])
def test_ragged_rows_groups_4_and_8(device, heads, lengths):
    query_heads, kv_heads = heads
    cpu = make_decode_attention_case(lengths, query_heads=query_heads, kv_heads=kv_heads,
                                     head_dim=64, block_size=16, dtype=torch.bfloat16,
                                     seed=len(lengths), table_width=128)
    gpu = cpu.to(device)
    for plan, flags in sorted(PLANS.items()):
        out = torch.full_like(gpu.query, float("nan"))
        status, _ = _call(gpu, out, flags)
        assert status == 0, _native.library().tf_last_error()
        torch.cuda.synchronize()
        _check(cpu, out, f"valu {heads} {plan}")


def test_split_partitions_merge_to_the_oracle(device):
    """Split-KV partials of the VALU form (512-token partitions), merged on
    the host by log-sum-exp, give the oracle's rows."""

    cpu = make_decode_attention_case([1800, 513, 40, 1024], query_heads=32, kv_heads=4,
                                     head_dim=64, block_size=16, dtype=torch.bfloat16, seed=7,
                                     table_width=128)
    gpu = cpu.to(device)
    out = torch.empty_like(gpu.query)
    status, partials = _call(gpu, out, _native.TF_ATTENTION_FLAG_VALU, split_size=512)
    assert status == 0, _native.library().tf_last_error()
    torch.cuda.synchronize()
    merged = _merge(partials, cpu.lengths, 512, 32, torch.bfloat16)
    _check(cpu, merged, "valu split 512")


def test_unsupported_geometries_are_rejected(device):
    cpu = make_decode_attention_case([100, 20], query_heads=16, kv_heads=4, head_dim=128,
                                     block_size=16, dtype=torch.bfloat16, seed=1)
    gpu = cpu.to(device)
    status, _ = _call(gpu, torch.empty_like(gpu.query), _native.TF_ATTENTION_FLAG_VALU)
    assert status == 2
    assert b"VALU attention form supports head_dim 64" in _native.library().tf_last_error()
