"""Continuous batching of the config-5 model on the GPU, at reduced size.

The 22-layer TinyLlama-geometry decoder (random init, seed 0, bf16) serves
40 requests through ``serving.ContinuousServer`` over the graph-bucketed
executor: 36 arrive at once and 4 later (Poisson gaps), prompts of
16..600 tokens, outputs of 8..30 tokens.  So the running batch passes
through every batch bucket {1, 2, 4, 8, 16, 32, 64} and contexts cross
from the 512- into the 1024-token bucket, with requests joining, leaving
and changing lanes while one step stays in flight.

Every request's tokens are checked against the fp32 decoder oracle,
teacher-forced on the run's own tokens (the reference checks its
scheduler's tokens against full-prefix greedy generation,
tests/test_gpu_continuous_scheduler.py:20-77).  The run is made twice:
pipelined (one step in flight, the serving mode), where a token may differ
from the oracle's argmax only where the oracle's top-two margin is within
twice the stated bf16 logit bound; and with every step read back with its
logits, where the largest logit deviation of that same run is measured,
must be within the stated bound, and a token may differ only where the
margin is within twice that measured deviation.  At the end of each run
every page and sequence slot is back in the pool.
"""

from __future__ import annotations

import dataclasses
import random

import numpy as np
import pytest
import torch

from tensorforge_amd.cache import PagedKVCache, PagedKVCacheConfig
from tensorforge_amd.decode import (
    BucketedDecodeExecutor,
    DecoderWeights,
    tinyllama_config,
)
from tensorforge_amd.serving import ContinuousServer, RequestSpec, summarize
from tests.helpers import GreedyParity
from tests.test_gpu_decode_tinyllama import BF16_22_LAYER_BOUND

pytestmark = pytest.mark.gpu

BATCH_BUCKETS = (1, 2, 4, 8, 16, 32, 64)
CONTEXT_BUCKETS = (512, 1024)


def _requests(vocab: int) -> list[RequestSpec]:
    rng = np.random.default_rng(5)
    count = 40
    prompts = np.clip(np.rint(rng.lognormal(np.log(256), 0.8, size=count)), 16, 600).astype(int)
    prompts[:3] = (600, 560, 530)  # contexts past 512 tokens
    outputs = rng.integers(8, 25, size=count)
    outputs[-6:] = (30, 29, 28, 27, 26, 25)  # a tail of 6, 5, ..., 1 running requests
    arrivals = np.zeros(count)
    arrivals[36:] = np.cumsum(rng.exponential(0.05, size=4))
    return [RequestSpec(f"s{i:02d}", tuple(int(t) for t in rng.integers(0, vocab, size=n)),
                        int(o), float(a))
            for i, (n, o, a) in enumerate(zip(prompts, outputs, arrivals))]


def _serve(weights, device, requests, logits=None):
    config = weights.config
    pages = 64 * (1024 // 16)
    order = list(range(pages))
    random.Random(0).shuffle(order)
    cache = PagedKVCache(
        PagedKVCacheConfig(num_layers=config.num_hidden_layers, num_blocks=pages, block_size=16,
                           num_kv_heads=config.num_key_value_heads, head_dim=config.head_dim,
                           max_sequences=64, max_sequence_length=1024, dtype=torch.bfloat16,
                           device=device),
        page_order=order)
    executor = BucketedDecodeExecutor(weights, cache, batch_buckets=BATCH_BUCKETS,
                                      context_buckets=CONTEXT_BUCKETS)
    traces = ContinuousServer(executor, max_batch=64, progress_s=0, logits=logits).run(requests)
    assert all(t.error is None for t in traces), [t.error for t in traces if t.error]
    stats = cache.stats()
    assert stats.active_sequences == 0 and stats.used_blocks == 0 and stats.reserved_tokens == 0
    return executor, traces


def _fp32(weights):
    """fp32 copies of the weights on their device, converted once."""

    return dataclasses.replace(
        weights,
        embedding=weights.embedding.float(), final_norm=weights.final_norm.float(),
        lm_head=weights.lm_head.float(),
        layers=[dataclasses.replace(layer, **{f.name: getattr(layer, f.name).float()
                                              for f in dataclasses.fields(layer)})
                for layer in weights.layers])


def test_continuous_batching_over_every_bucket_follows_the_oracle(device):
    config = tinyllama_config()
    weights = DecoderWeights.random(config, seed=0, dtype=torch.bfloat16, device=device)
    requests = _requests(config.vocab_size)
    executor, traces = _serve(weights, device, requests)

    # Every request served in full.
    for spec, trace in zip(requests, traces):
        assert len(trace.generated) == spec.max_new_tokens, spec.request_id
    # The batch passed through every batch bucket and both context buckets.
    used = {record.bucket for record in executor.step_records}
    assert {b for b, _ in used} == set(BATCH_BUCKETS), sorted(used)
    assert {c for _, c in used} == set(CONTEXT_BUCKETS), sorted(used)
    metrics = executor.metrics()
    assert metrics.shape_fallbacks == 0 and metrics.capture_count == len(used)
    summary = summarize(traces, executor)
    print(f"[serving] {summary['requests']} requests, {summary['generated_tokens']} tokens, "
          f"{summary['decode_steps']} decode steps, buckets {sorted(used)}")

    # Tokens against the fp32 oracle (run on the GPU; weights converted once).
    fp32 = _fp32(weights)
    parity = GreedyParity(fp32, bound=BF16_22_LAYER_BOUND, device=device,
                          name="cfg5 serving (pipelined), 40 requests, buckets 1..64")
    for spec, trace in zip(requests, traces):
        parity.check(spec.request_id, spec.prompt, trace.generated)
    parity.finish()

    # The same requests with every step read back with its logits.
    logits: dict[str, list[torch.Tensor]] = {}
    _, recorded = _serve(weights, device, requests, logits=logits)
    measured = GreedyParity(fp32, bound=BF16_22_LAYER_BOUND, device=device,
                            name="cfg5 serving (logits recorded), 40 requests")
    for spec, trace in zip(requests, recorded):
        assert len(trace.generated) == spec.max_new_tokens == len(logits[spec.request_id])
        measured.check(spec.request_id, spec.prompt, trace.generated, logits[spec.request_id])
    measured.finish()
