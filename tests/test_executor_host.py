"""Host-side checks of the decode executor's prefill contract (no GPU).

A prompt id outside the vocabulary must be rejected on the host before any
reservation or device work: on the device it would index the embedding
table out of range (the reference rejects such prompts first,
runtime/prefill.py:182-183).  ``prefill_requests`` reports such failures per
request, as ``BatchExecutionResult.errors`` (runtime/batch.py:11-31).
The cache and weights live on the CPU here, so any device work would fail
loudly: these tests pass only if the checks come first.
"""

from __future__ import annotations

import pytest
import torch

from tensorforge_amd.batch import BatchExecutionResult
from tensorforge_amd.cache import PagedKVCache, PagedKVCacheConfig
from tensorforge_amd.decode import DecoderWeights, prefill_batch, prefill_requests, small_config


def _host_model():
    config = small_config()
    weights = DecoderWeights.random(config, seed=0, dtype=torch.float32, device="cpu")
    cache = PagedKVCache(PagedKVCacheConfig(
        num_layers=config.num_hidden_layers, num_blocks=8, block_size=16,
        num_kv_heads=config.num_key_value_heads, head_dim=config.head_dim, max_sequences=3,
        max_sequence_length=64, dtype=torch.float32, device=torch.device("cpu")))
    return config, weights, cache


@pytest.mark.parametrize("bad", [1024, 5000, -1])
def test_prefill_batch_rejects_tokens_outside_the_vocabulary(bad: int) -> None:
    config, weights, cache = _host_model()
    assert config.vocab_size == 1024
    cache.create_sequence("a")
    cache.create_sequence("b")
    with pytest.raises(ValueError, match="outside the model vocabulary"):
        prefill_batch(weights, cache, {"a": [1, 2, 3], "b": [4, bad, 6]})
    stats = cache.stats()
    assert stats.reserved_tokens == 0 and stats.used_blocks == 0
    assert cache.sequence_layout("a").context_length == 0
    assert cache.sequence_layout("b").context_length == 0


def test_prefill_requests_reports_invalid_prompts_per_request() -> None:
    _, weights, cache = _host_model()
    for rid in ("a", "b", "c"):
        cache.create_sequence(rid)
    result = prefill_requests(weights, cache, {"a": [1, 2, 1024], "b": [], "c": [-3]})
    assert isinstance(result, BatchExecutionResult)
    assert result.logits == {}
    assert set(result.errors) == {"a", "b", "c"}
    assert "outside the model vocabulary" in result.errors["a"]
    assert "at least one token" in result.errors["b"]
    assert "outside the model vocabulary" in result.errors["c"]
    assert cache.stats().reserved_tokens == 0 and cache.stats().used_blocks == 0


def test_prefill_requests_reports_a_stale_sequence_and_an_exhausted_cache() -> None:
    _, weights, cache = _host_model()
    cache.create_sequence("long")
    # 8 pages of 16 tokens: a 200-token prompt exceeds the sequence limit (64).
    result = prefill_requests(weights, cache, {"long": list(range(200))})
    assert result.logits == {}
    assert "CacheExhaustedError" in result.errors["long"]
    assert cache.stats().reserved_tokens == 0
    with pytest.raises(ValueError):
        prefill_requests(weights, cache, {})
