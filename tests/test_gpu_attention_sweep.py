"""Seeded sweep of the decode-attention entry point over drawn geometries.

Each case draws a dtype, head_dim (the MFMA sizes 32 / 64 / 128 and the
generic kernel's 80 / 96), kv heads, GQA group, page size (including pages
that straddle the 16-token MFMA tile), a batch and ragged lengths (zero,
one token, whole pages, the table's capacity), extra unused pages, a wider
block table than the rows need, a scale, and a plan: the entry point's own
choice, ``attention_path="one_pass"`` / ``"split_kv"``, or a caller-fixed
partition size (``set_attention_split_size``).  The regimes cover every
plan the entry point has: narrow one pass, wide one pass, narrow split-KV,
balanced partitions (>= 8192 tokens, 2..64 rows) and fixed partitions.

The check is the reference's own (tests/test_decode_attention.py:60-104 of
the reference: the oracle on the same inputs, the reference's per-dtype
tolerance) on the active rows, and exact zeros on zero-length rows.  The
launch record is in every failure message.

Every second case also runs, mapped onto the fused RoPE + KV append +
attention launch's geometries, through that launch and through the two
launches it replaces: output and both caches bit-identical, and the
output against the RoPE oracle followed by the attention oracle within
max-abs 2e-2 + rel 1e-2.
"""

from __future__ import annotations

import random

import pytest
import torch

from helpers import NORTH_STAR_ATOL, NORTH_STAR_RTOL, REFERENCE_TOLERANCE, assert_close
from oracle.model import rope_tables
from oracle.reference import paged_gqa_decode_reference, rope_kv_append_reference
from tensorforge_amd.kernels import (
    PagedAttentionWorkspace,
    paged_gqa_decode_attention,
    rope_paged_kv_append,
    selected_attention_launch,
    set_attention_split_size,
)
from tensorforge_amd.kernels.attention import (
    attention_plan,
    paged_gqa_decode_attention_rope_append,
)
from tensorforge_amd.workloads import make_decode_attention_case

CASES = 48


def _lengths(rng: random.Random, batch: int, longest: int, block_size: int) -> list[int]:
    lengths = []
    for _ in range(batch):
        pick = rng.random()
        if pick < 0.08:
            lengths.append(0)
        elif pick < 0.14:
            lengths.append(1)
        elif pick < 0.24:
            lengths.append(longest)
        elif pick < 0.34:
            lengths.append(max(block_size, longest // block_size * block_size))
        else:
            lengths.append(rng.randint(1, longest))
    if max(lengths) == 0:
        lengths[0] = longest
    return lengths


def draw(seed: int) -> dict:
    """One case of the sweep, a function of the seed only."""

    rng = random.Random(7919 * seed + 17)
    regime = ("short", "mid", "wide", "long", "balanced")[seed % 5]
    dtype = rng.choice([torch.bfloat16, torch.bfloat16, torch.float16, torch.float32])
    head_dim = rng.choice([32, 64, 64, 128, 80, 96, 256])
    kv_heads = rng.choice([1, 2, 4, 8])
    group = rng.choice([1, 2, 4, 8, 16])
    block_size = rng.choice([1, 5, 8, 16, 16, 32, 48, 64])
    if regime == "short":
        batch, longest = rng.randint(1, 16), rng.randint(1, 300)
    elif regime == "mid":
        batch, longest = rng.randint(1, 40), rng.randint(300, 2100)
    elif regime == "wide":
        # >= 192 (row, kv head) workgroups: the wide one-pass plan.
        kv_heads = rng.choice([4, 8])
        head_dim = min(head_dim, 128)
        batch = rng.randint(48, 80)
        longest = rng.randint(100, 2100 if kv_heads == 4 else 1200)
    elif regime == "long":
        head_dim = min(head_dim, 128)
        batch, longest = rng.randint(1, 6), rng.randint(2100, 6000)
    else:
        # 2..64 rows, the longest >= 8192 tokens, more slots (256 / 8 kv
        # heads) than rows, the MFMA kernel: the balanced partitions.
        kv_heads = 8
        group = rng.choice([1, 2, 4, 8])
        head_dim = rng.choice([32, 64, 128])
        dtype = rng.choice([torch.bfloat16, torch.float16])
        batch, longest = rng.randint(2, 6), rng.randint(8192, 10000)
        block_size = rng.choice([16, 32, 64])
    while kv_heads * group > 64:
        group //= 2
    if block_size == 1 and longest > 2100:
        block_size = 16
    lengths = _lengths(rng, batch, longest, block_size)
    lengths[rng.randrange(batch)] = longest
    plan = rng.random()
    path = "auto"
    split = None
    if regime == "balanced" and plan < 0.75:
        pass
    elif plan < 0.15:
        path = "one_pass"
    elif plan < 0.30:
        path = "split_kv"
    elif plan < 0.45:
        split = rng.choice([32, 64, 256, 512, 1024])
    scale = head_dim**-0.5 if rng.random() < 0.7 else rng.uniform(0.05, 0.3)
    return {
        "regime": regime, "dtype": dtype, "head_dim": head_dim, "kv_heads": kv_heads,
        "query_heads": kv_heads * group, "block_size": block_size, "lengths": lengths,
        "path": path, "split": split, "scale": scale,
        "extra_pages": rng.randint(0, 8), "extra_width": rng.randint(0, 3),
        "max_context": rng.choice(["none", "exact", "capacity"]),
    }


def _table_width(spec: dict) -> int:
    block_size = spec["block_size"]
    return (max((n + block_size - 1) // block_size for n in spec["lengths"])
            + spec["extra_width"])


def _launch_context(spec: dict) -> int | None:
    return {"none": None, "exact": max(spec["lengths"]),
            "capacity": _table_width(spec) * spec["block_size"]}[spec["max_context"]]


def test_the_sweep_reaches_every_regime_and_plan():
    """The drawn cases cover what the sweep is for (host only)."""

    cases = [draw(seed) for seed in range(CASES)]
    assert {c["regime"] for c in cases} == {"short", "mid", "wide", "long", "balanced"}
    assert {c["path"] for c in cases} == {"auto", "one_pass", "split_kv"}
    assert any(c["split"] for c in cases)
    assert {c["head_dim"] for c in cases} >= {32, 64, 128}
    assert {c["head_dim"] for c in cases} & {80, 96}
    assert any(0 in c["lengths"] for c in cases)
    assert any(c["block_size"] % 16 for c in cases)
    plans = []
    for c in cases:
        if c["split"] is None:
            context = _launch_context(c) or max(c["lengths"])
            plans.append(attention_plan(context, len(c["lengths"]), c["kv_heads"],
                                        _table_width(c) * c["block_size"], c["path"]))
    assert sum(p.balanced for p in plans) >= 3
    assert sum(p.one_pass and p.waves_per_head > 1 for p in plans) >= 3
    assert sum(not p.one_pass and not p.balanced for p in plans) >= 3


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(CASES))
def test_drawn_geometry_matches_the_oracle(device, seed):
    spec = draw(seed)
    lengths = spec["lengths"]
    block_size = spec["block_size"]
    width = _table_width(spec)
    case = make_decode_attention_case(
        lengths, query_heads=spec["query_heads"], kv_heads=spec["kv_heads"],
        head_dim=spec["head_dim"], block_size=block_size, dtype=spec["dtype"], seed=seed,
        table_width=width, extra_pages=spec["extra_pages"])
    max_context = _launch_context(spec)
    gpu = case.to(device)
    previous = set_attention_split_size(spec["split"])
    try:
        actual = paged_gqa_decode_attention(
            gpu.query, gpu.key_cache, gpu.value_cache, gpu.block_tables, gpu.context_lengths,
            scale=spec["scale"], max_context_length=max_context, attention_path=spec["path"])
        launch = selected_attention_launch()
    finally:
        set_attention_split_size(previous)
    torch.cuda.synchronize()
    what = (f"seed {seed} {spec['regime']} {spec['dtype']} hq {spec['query_heads']} "
            f"hkv {spec['kv_heads']} D {spec['head_dim']} page {block_size} "
            f"path {spec['path']} split {spec['split']} launch {launch} lengths {lengths}")
    rows = [row for row, n in enumerate(lengths) if n > 0]
    expected = paged_gqa_decode_reference(
        case.query[rows], case.key_cache, case.value_cache, case.block_tables[rows],
        case.context_lengths[rows], scale=spec["scale"])
    tol = REFERENCE_TOLERANCE[spec["dtype"]]
    assert_close(actual[rows], expected, tol, tol, what)
    for row, n in enumerate(lengths):
        if n == 0:
            assert bool((actual[row] == 0).all()), f"{what}: zero-length row {row} not zero"


def draw_fused(seed: int) -> dict:
    """A sweep case mapped onto what the fused RoPE + append + attention
    launch takes: the MFMA kernel's head dims and page multiples of 16,
    fp16 / bf16, the entry point's own plan (or a caller-fixed partition
    size)."""

    spec = draw(seed)
    if spec["dtype"] == torch.float32:
        spec["dtype"] = torch.bfloat16
    if spec["head_dim"] not in (32, 64, 128):
        spec["head_dim"] = 64
    if spec["block_size"] % 16:
        spec["block_size"] = 16 * (1 + spec["block_size"] // 16)
    spec["path"] = "auto"
    return spec


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(0, CASES, 2))
def test_drawn_geometry_fused_rope_append_equals_the_two_launches(device, seed):
    spec = draw_fused(seed)
    lengths, block_size, dtype = spec["lengths"], spec["block_size"], spec["dtype"]
    hq, hkv, d = spec["query_heads"], spec["kv_heads"], spec["head_dim"]
    width = _table_width(spec)
    case = make_decode_attention_case(
        lengths, query_heads=hq, kv_heads=hkv, head_dim=d, block_size=block_size, dtype=dtype,
        seed=seed, table_width=width, extra_pages=spec["extra_pages"])
    generator = torch.Generator().manual_seed(seed + 1)
    qkv = torch.randn(len(lengths), (hq + 2 * hkv) * d, generator=generator).to(dtype)
    positions = torch.tensor([max(n - 1, 0) for n in lengths], dtype=torch.int64)
    pages = torch.tensor([int(case.block_tables[r, (n - 1) // block_size]) if n > 0 else -1
                          for r, n in enumerate(lengths)], dtype=torch.int32)
    offsets = torch.tensor([(n - 1) % block_size if n > 0 else 0 for n in lengths],
                           dtype=torch.int32)
    active = torch.tensor([1 if n > 0 else 0 for n in lengths], dtype=torch.int32)
    cos, sin = rope_tables(d, 10000.0, torch.arange(max(lengths)))
    cos, sin = cos.to(dtype), sin.to(dtype)
    capacity = _launch_context(spec) or max(lengths)

    gpu = case.to(device)
    qkv_dev = qkv.to(device)
    rope = [t.to(device) for t in (positions, cos, sin)]
    append = [t.to(device) for t in (pages, offsets, active)]
    # Sized as the reference sizes it (256-token partitions over the table),
    # and for as many partitions as a smaller caller-fixed size makes.
    splits = -(-capacity // spec["split"]) if spec["split"] else 1
    workspace = PagedAttentionWorkspace.allocate(
        batch_capacity=len(lengths), query_heads=hq, head_dim=d,
        max_context_length=max(width * block_size, splits * 256), device=device)
    previous = set_attention_split_size(spec["split"])
    try:
        k1, v1 = gpu.key_cache.clone(), gpu.value_cache.clone()
        q = rope_paged_kv_append(qkv_dev, *rope, k1, v1, *append, query_heads=hq)
        out1 = paged_gqa_decode_attention(q, k1, v1, gpu.block_tables, gpu.context_lengths,
                                          max_context_length=capacity, workspace=workspace)
        launch = selected_attention_launch()
        k2, v2 = gpu.key_cache.clone(), gpu.value_cache.clone()
        out2 = torch.full_like(out1, float("nan"))
        paged_gqa_decode_attention_rope_append(
            qkv_dev, *rope, k2, v2, *append, gpu.block_tables, gpu.context_lengths,
            query_heads=hq, max_context_length=capacity, output=out2, workspace=workspace)
    finally:
        set_attention_split_size(previous)
    torch.cuda.synchronize()
    what = (f"seed {seed} {spec['regime']} {dtype} hq {hq} hkv {hkv} D {d} page {block_size} "
            f"split {spec['split']} launch {launch} lengths {lengths}")
    assert torch.equal(out2.view(torch.int16), out1.view(torch.int16)), what
    assert torch.equal(k2.view(torch.int16), k1.view(torch.int16)), what
    assert torch.equal(v2.view(torch.int16), v1.view(torch.int16)), what

    q_ref, k_ref, v_ref = rope_kv_append_reference(
        qkv, positions, cos, sin, case.key_cache, case.value_cache, pages, offsets, active,
        query_heads=hq)
    live = [r for r, n in enumerate(lengths) if n > 0]
    want = paged_gqa_decode_reference(q_ref.view(len(lengths), hq, d)[live], k_ref, v_ref,
                                      case.block_tables[live], case.context_lengths[live],
                                      scale=d ** -0.5)
    assert_close(out2.cpu()[live], want, NORTH_STAR_ATOL, NORTH_STAR_RTOL, what)
    dead = [r for r, n in enumerate(lengths) if n == 0]
    assert bool((out2.cpu()[dead] == 0).all()), what
