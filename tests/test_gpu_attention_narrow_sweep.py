"""Seeded sweep of the narrow split-KV plan (fewer than 192 (row, kv head)
workgroups, rows long enough to split) over drawn geometries and
workspace sizings.

Each case draws bf16 or fp16, head_dim 32 / 64 / 128, 1-8 kv heads with
groups of 1-8 query heads, pages of 16 or 32 tokens, 1-47 rows of ragged
lengths (zeros, single tokens, the longest row), a launch context of
512-6000 tokens, and the workspace: none (the entry point allocates one for
the plan), one sized as the reference sizes it (a partial per 256 tokens,
so partitions stay >= 256 tokens) or one sized as the decode executor sizes
it (a partial per 128 tokens).  The host test checks that the drawn cases
reach equal partitions with and without paired kv heads and the one-pass
fallback; the GPU test runs the entry point and compares with the oracle at
the reference's per-dtype tolerance (tests/test_decode_attention.py:60-104
of the reference), zero-length rows exactly zero, and checks that the
launch took the planned partitions and kv heads per workgroup.
"""

from __future__ import annotations

import random

import pytest
import torch

from helpers import REFERENCE_TOLERANCE, assert_close
from oracle.reference import paged_gqa_decode_reference
from tensorforge_amd.kernels import (
    PagedAttentionWorkspace,
    paged_gqa_decode_attention,
    selected_attention_autotune_config,
    selected_attention_launch,
)
from tensorforge_amd.kernels.attention import attention_plan
from tensorforge_amd.workloads import make_decode_attention_case

CASES = 24
WORKSPACES = ("none", "reference", "executor")


def draw(seed: int) -> dict:
    """One case of the sweep, a function of the seed only."""

    rng = random.Random(7919 * seed + 17)
    head_dim = rng.choice([32, 64, 128])
    kv_heads = rng.choice([1, 2, 4, 8])
    group = rng.choice([1, 2, 4, 8])
    rows = rng.choice([1, 2, 3, 8, 16, 31, 47, rng.randint(1, 47)])
    while rows * kv_heads >= 192:
        rows //= 2
    context = rng.choice([512, 1000, 1500, 2048, 3000, 4096, rng.randint(512, 6000)])
    while rows * context > 60000:  # keeps the CPU oracle to about a second
        context //= 2
    context = max(context, 256)
    lengths = []
    for _ in range(rows):
        pick = rng.random()
        lengths.append(0 if pick < 0.1 else 1 if pick < 0.15 else context if pick < 0.35
                       else rng.randint(1, context))
    lengths[rng.randrange(rows)] = context  # the launch context is reached
    return {
        "dtype": rng.choice([torch.bfloat16, torch.float16]),
        "head_dim": head_dim, "kv_heads": kv_heads, "query_heads": kv_heads * group,
        "block_size": rng.choice([16, 32]),
        "lengths": lengths, "context": context,
        "workspace": rng.choice(WORKSPACES),
    }


def _slot_limit(spec: dict) -> int | None:
    """Partials per (row, query head) of the drawn workspace (None: the
    entry point allocates one for the plan)."""

    if spec["workspace"] == "none":
        return None
    return -(-spec["context"] // (256 if spec["workspace"] == "reference" else 128))


def _plan(spec: dict):
    width = -(-spec["context"] // spec["block_size"])
    limit = _slot_limit(spec)
    return attention_plan(spec["context"], len(spec["lengths"]), spec["kv_heads"],
                          width * spec["block_size"],
                          slot_limit=limit if limit is not None else 1024,
                          head_dim=spec["head_dim"], element_bytes=2)


def test_the_sweep_reaches_every_narrow_form():
    """The drawn cases cover what the sweep is for (host only)."""

    cases = [draw(seed) for seed in range(CASES)]
    plans = [_plan(c) for c in cases]
    split = [p for p in plans if not p.one_pass and not p.balanced]
    assert len(split) >= CASES // 2
    assert any(p.heads_per_wg == 2 for p in split) and any(p.heads_per_wg == 1 for p in split)
    assert any(p.split_size == 128 for p in split) and any(p.split_size % 128 for p in split)
    assert any(p.one_pass for p in plans)
    assert {c["workspace"] for c in cases} == set(WORKSPACES)
    assert {c["head_dim"] for c in cases} == {32, 64, 128}
    # A reference-sized workspace keeps partitions of at least 256 tokens.
    for c, p in zip(cases, plans):
        if c["workspace"] == "reference" and not p.one_pass:
            assert p.num_splits <= -(-c["context"] // 256)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(CASES))
def test_drawn_narrow_call_matches_the_oracle(device, seed):
    spec = draw(seed)
    dtype, d, hq, hkv = spec["dtype"], spec["head_dim"], spec["query_heads"], spec["kv_heads"]
    lengths, context = spec["lengths"], spec["context"]
    width = -(-context // spec["block_size"])
    case = make_decode_attention_case(lengths, query_heads=hq, kv_heads=hkv, head_dim=d,
                                      block_size=spec["block_size"], dtype=dtype, seed=seed,
                                      table_width=width, extra_pages=3)
    gpu = case.to(device)
    workspace = None
    if spec["workspace"] != "none":
        sizing = context if spec["workspace"] == "reference" else 2 * context
        workspace = PagedAttentionWorkspace.allocate(batch_capacity=len(lengths), query_heads=hq,
                                                     head_dim=d, max_context_length=sizing,
                                                     device=device)
    plan = _plan(spec)
    out = paged_gqa_decode_attention(gpu.query, gpu.key_cache, gpu.value_cache, gpu.block_tables,
                                     gpu.context_lengths, max_context_length=context,
                                     workspace=workspace)
    torch.cuda.synchronize()
    record, launch = selected_attention_autotune_config(), selected_attention_launch()
    what = (f"seed {seed}: {dtype} D{d} {hq}/{hkv} heads, {len(lengths)} rows to {context}, pages "
            f"of {spec['block_size']}, workspace {spec['workspace']}, record {record}, "
            f"launch {launch}")
    if plan.one_pass:
        assert record["path"] == "one_pass", what
    else:
        assert record == {"path": "split_kv", "split_size": plan.split_size,
                          "num_splits": plan.num_splits}, what
        if launch["kernel"] == "mfma":
            assert launch["heads_per_workgroup"] == plan.heads_per_wg, what
    live = [r for r, c in enumerate(lengths) if c > 0]
    want = paged_gqa_decode_reference(case.query[live], case.key_cache, case.value_cache,
                                      case.block_tables[live], case.context_lengths[live],
                                      scale=case.scale)
    tol = REFERENCE_TOLERANCE[dtype]
    assert_close(out.cpu()[live], want, tol, tol, what)
    empty = [r for r, c in enumerate(lengths) if c == 0]
    assert bool((out.cpu()[empty] == 0).all()), what
