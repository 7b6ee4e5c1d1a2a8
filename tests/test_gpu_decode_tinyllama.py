"""Greedy decoding at the real 22-layer TinyLlama geometry (bf16, random
init) against the fp32 decoder oracle: prefill of two prompts packed
together, then graph-captured decode steps with one step in flight.

bf16 weights and activations through 22 layers move the logits by about a
percent of their range, so a sampled token may differ from the oracle's
argmax only where the oracle's own top-two margin is within that
(the reference's margin rule, tests/test_triton_model.py:38-43).
"""

from __future__ import annotations

import random

import pytest
import torch

from oracle.model import decoder_forward
from tensorforge_amd.cache import PagedKVCache, PagedKVCacheConfig
from tensorforge_amd.decode import (
    BucketedDecodeExecutor,
    DecoderWeights,
    greedy_decode,
    tinyllama_config,
)

pytestmark = pytest.mark.gpu

MARGIN = 3e-2  # of the row's largest |logit|


def test_tinyllama_geometry_greedy_tokens_follow_the_oracle(device):
    config = tinyllama_config()
    weights = DecoderWeights.random(config, seed=0, dtype=torch.bfloat16, device=device)
    order = list(range(64))
    random.Random(1).shuffle(order)
    cache = PagedKVCache(
        PagedKVCacheConfig(num_layers=config.num_hidden_layers, num_blocks=64, block_size=16,
                           num_kv_heads=config.num_key_value_heads, head_dim=config.head_dim,
                           max_sequences=2, max_sequence_length=512, dtype=torch.bfloat16,
                           device=device),
        page_order=order)
    executor = BucketedDecodeExecutor(weights, cache, batch_buckets=(2,), context_buckets=(512,))
    rng = random.Random(0)
    prompts = {"a": [rng.randrange(config.vocab_size) for _ in range(40)],
               "b": [rng.randrange(config.vocab_size) for _ in range(23)]}
    outputs = greedy_decode(executor, prompts, steps=8)
    flips = 0
    for rid, prompt in prompts.items():
        generated = outputs[rid]
        assert len(generated) == 8
        logits = decoder_forward(weights, torch.tensor(prompt + generated[:-1]))
        for step, token in enumerate(generated):
            row = logits[len(prompt) - 1 + step]
            best = int(torch.argmax(row))
            if token != best:
                margin = float(row[best] - row[token])
                assert margin <= MARGIN * float(row.abs().max()), (rid, step, token, best, margin)
                flips += 1
    assert flips <= 2
