"""Packed causal GQA prefill attention against an fp32 CPU restatement of
the reference's masked SDPA (tensorforge/runtime/prefill.py:84-88,
109-118): each token attends to its own prompt's tokens up to itself.
Bar: the north-star max-abs 2e-2 + rel 1e-2 for bf16/fp16 outputs."""

from __future__ import annotations

import pytest
import torch

from helpers import NORTH_STAR_ATOL, NORTH_STAR_RTOL, assert_close
from tensorforge_amd.kernels.prefill import prefill_attention, prefill_tiles

pytestmark = pytest.mark.gpu


def _reference(q, k, v, lengths, hq, hkv, d, scale):
    """fp32 causal attention per prompt, GQA by index, on the CPU."""

    out = torch.zeros(q.shape[0], hq, d)
    group = hq // hkv
    start = 0
    for n in lengths:
        qs = q[start:start + n].float().view(n, hq, d)
        ks = k[start:start + n].float().view(n, hkv, d)
        vs = v[start:start + n].float().view(n, hkv, d)
        for h in range(hq):
            scores = (qs[:, h] @ ks[:, h // group].T) * scale
            scores = scores.masked_fill(torch.triu(torch.ones(n, n, dtype=torch.bool), 1), -float("inf"))
            out[start:start + n, h] = torch.softmax(scores, dim=-1) @ vs[:, h // group]
        start += n
    return out.view(q.shape[0], hq * d)


@pytest.mark.parametrize(("hq", "hkv", "d", "dtype"),
                         [(32, 4, 64, torch.bfloat16), (8, 2, 32, torch.float16),
                          (32, 8, 128, torch.bfloat16), (16, 1, 64, torch.float16),
                          (4, 4, 64, torch.bfloat16)])
@pytest.mark.parametrize("heads_per_wave", [0, 1, 8])
def test_prefill_attention_matches_fp32(device, hq, hkv, d, dtype, heads_per_wave):
    lengths = [1, 15, 16, 17, 33, 64, 300, 5]
    total = sum(lengths)
    generator = torch.Generator().manual_seed(hq * 31 + d + heads_per_wave)
    q = torch.randn(total, hq * d, generator=generator).to(dtype)
    # k and v as column slices of wider rows (strided, like the fused QKV rows)
    kv = torch.randn(total, 2 * hkv * d + 32, generator=generator).to(dtype)
    k, v = kv[:, :hkv * d], kv[:, hkv * d:2 * hkv * d]
    scale = d ** -0.5
    tiles = torch.from_numpy(prefill_tiles(lengths)).to(device)
    kv_dev = kv.to(device)
    out = torch.full((total, hq * d), float("nan"), dtype=dtype, device=device)
    prefill_attention(q.to(device), kv_dev[:, :hkv * d], kv_dev[:, hkv * d:2 * hkv * d], tiles,
                      query_heads=hq, kv_heads=hkv, scale=scale, output=out,
                      heads_per_wave=heads_per_wave)
    want = _reference(q, k, v, lengths, hq, hkv, d, scale)
    assert_close(out.cpu(), want, NORTH_STAR_ATOL, NORTH_STAR_RTOL,
                 f"prefill hq={hq} hkv={hkv} d={d} qh={heads_per_wave}")


def _draw(seed: int) -> dict:
    import random

    rng = random.Random(4409 * seed + 7)
    hkv = rng.choice([1, 2, 4, 8])
    group = rng.choice([1, 2, 4, 8])
    return {
        "hq": hkv * group, "hkv": hkv, "d": rng.choice([32, 64, 128]),
        "dtype": rng.choice([torch.bfloat16, torch.float16]),
        "heads_per_wave": rng.choice([0, 1, 2, 4, 8]),
        "lengths": [rng.choice([1, 15, 16, 17, 64, 65, rng.randint(1, 500)])
                    for _ in range(rng.randint(1, 8))],
    }


@pytest.mark.parametrize("seed", range(12))
def test_prefill_attention_drawn_geometries(device, seed):
    """Seeded sweep: 1-8 prompts of 1-500 tokens (tile remainders around 16
    and 64), head_dim 32 / 64 / 128, 1-8 kv heads with groups of 1-8, every
    query-heads-per-wavefront setting, fp16 and bf16."""

    spec = _draw(seed)
    hq, hkv, d, dtype, lengths = spec["hq"], spec["hkv"], spec["d"], spec["dtype"], spec["lengths"]
    total = sum(lengths)
    generator = torch.Generator().manual_seed(seed)
    q = torch.randn(total, hq * d, generator=generator).to(dtype)
    kv = torch.randn(total, 2 * hkv * d, generator=generator).to(dtype)
    k, v = kv[:, :hkv * d], kv[:, hkv * d:]
    scale = d ** -0.5
    tiles = torch.from_numpy(prefill_tiles(lengths)).to(device)
    kv_dev = kv.to(device)
    out = torch.full((total, hq * d), float("nan"), dtype=dtype, device=device)
    prefill_attention(q.to(device), kv_dev[:, :hkv * d], kv_dev[:, hkv * d:], tiles,
                      query_heads=hq, kv_heads=hkv, scale=scale, output=out,
                      heads_per_wave=spec["heads_per_wave"])
    want = _reference(q, k, v, lengths, hq, hkv, d, scale)
    assert_close(out.cpu(), want, NORTH_STAR_ATOL, NORTH_STAR_RTOL,
                 f"seed {seed}: prefill {spec}")
