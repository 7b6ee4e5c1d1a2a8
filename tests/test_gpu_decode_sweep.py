"""Seeded sweep of the graph-bucketed decode executor over drawn decoder
geometries.

Each case draws fp16 or bf16, head_dim 32 / 64 / 128, 1-4 kv heads and
1-8 query heads per kv head, an FFN of 1-3x the hidden size, 1-3 layers, a
vocabulary of 256-2048, pages of 16, 32 or 48 tokens on a seeded
permutation, batch and context buckets, and 2-5 prompts of 1-300 tokens
(some crossing a context bucket while they decode).  The executor prefills
and greedily decodes 8 tokens per request with the run's logits recorded,
and ``tests.helpers.GreedyParity`` checks them against the fp32 decoder
oracle teacher-forced on the run's own tokens: the largest logit deviation
within the reference's tolerance for the dtype at the run's logit
magnitude (fp16 4e-3 + 4e-3 L, tests/test_decode_bucket.py:119 of the
reference; bf16 3e-2 + 3e-2 L, tests/test_triton_model.py:37), and a token
may differ from the oracle's argmax only where the oracle's top-two margin
is within twice that deviation.
"""

from __future__ import annotations

import random

import pytest
import torch

from tensorforge_amd.cache import PagedKVCache, PagedKVCacheConfig
from tensorforge_amd.decode import (
    BucketedDecodeExecutor,
    DecoderConfig,
    DecoderWeights,
    greedy_decode,
)
from tests.helpers import GreedyParity

CASES = 10
TOLERANCE = {torch.float16: (4e-3, 4e-3), torch.bfloat16: (3e-2, 3e-2)}


def draw(seed: int) -> dict:
    """One case of the sweep, a function of the seed only."""

    rng = random.Random(1009 * seed + 41)
    head_dim = rng.choice([32, 64, 128])
    kv_heads = rng.choice([1, 2, 4])
    group = rng.choice([1, 2, 4, 8])
    while kv_heads * group * head_dim > 1024:
        group //= 2
    hidden = kv_heads * group * head_dim
    batch_buckets = rng.choice([(1, 2, 4), (4,), (2, 8)])
    prompts = [rng.randint(1, 300) for _ in range(rng.randint(2, 5))]
    prompts = prompts[: max(batch_buckets)]
    return {
        "dtype": rng.choice([torch.float16, torch.bfloat16]),
        "config": DecoderConfig(
            vocab_size=rng.choice([256, 1000, 2048]), hidden_size=hidden,
            intermediate_size=32 * ((hidden * rng.choice([1, 2, 3]) + 31) // 32),
            num_hidden_layers=rng.randint(1, 3), num_attention_heads=kv_heads * group,
            num_key_value_heads=kv_heads, max_position_embeddings=512),
        "block_size": rng.choice([16, 32, 48]),
        "batch_buckets": batch_buckets,
        "context_buckets": rng.choice([(512,), (128, 512), (256, 512)]),
        "prompts": prompts,
        "seed": seed,
    }


def test_the_sweep_reaches_every_head_dim_and_group():
    """The drawn geometries cover what the sweep is for (host only)."""

    cases = [draw(seed) for seed in range(CASES)]
    assert {c["config"].head_dim for c in cases} == {32, 64, 128}
    assert len({c["config"].num_attention_heads // c["config"].num_key_value_heads
                for c in cases}) >= 3
    assert {c["dtype"] for c in cases} == {torch.float16, torch.bfloat16}
    assert any(c["block_size"] != 16 for c in cases)
    assert any(min(c["context_buckets"]) < max(c["prompts"]) + 8 for c in cases)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(CASES))
def test_drawn_decoder_follows_the_oracle(device, seed):
    spec = draw(seed)
    config, dtype, block = spec["config"], spec["dtype"], spec["block_size"]
    what = (f"seed {seed}: {dtype} D{config.head_dim} {config.num_attention_heads}/"
            f"{config.num_key_value_heads} heads, hidden {config.hidden_size}, FFN "
            f"{config.intermediate_size}, {config.num_hidden_layers} layers, vocab "
            f"{config.vocab_size}, pages of {block}, prompts {spec['prompts']}")
    weights = DecoderWeights.random(config, seed=seed, dtype=dtype, device=device)
    pages = 4 * (512 // block + 1)
    order = list(range(pages))
    random.Random(seed).shuffle(order)
    cache = PagedKVCache(
        PagedKVCacheConfig(num_layers=config.num_hidden_layers, num_blocks=pages,
                           block_size=block, num_kv_heads=config.num_key_value_heads,
                           head_dim=config.head_dim, max_sequences=4 * len(spec["prompts"]),
                           max_sequence_length=512, dtype=dtype, device=device),
        page_order=order)
    executor = BucketedDecodeExecutor(weights, cache, batch_buckets=spec["batch_buckets"],
                                      context_buckets=spec["context_buckets"])
    rng = random.Random(seed)
    prompts = {f"r{i}": [rng.randrange(config.vocab_size) for _ in range(n)]
               for i, n in enumerate(spec["prompts"])}
    logits: dict[str, list[torch.Tensor]] = {}
    outputs = greedy_decode(executor, prompts, steps=8, logits=logits)
    parity = GreedyParity(weights, tolerance=TOLERANCE[dtype], device=device, name=what)
    for rid, prompt in prompts.items():
        assert len(outputs[rid]) == 8, what
        parity.check(rid, prompt, outputs[rid], logits[rid])
    parity.finish()
    assert executor.metrics().shape_fallbacks == 0, what
