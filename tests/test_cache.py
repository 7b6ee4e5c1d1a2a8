"""The paged cache's control plane on the CPU: allocation order,
transactional appends, rollback, partial commits, release and accounting.

Cases follow the reference's tests/test_paged_cache.py; page contents are
written only on the GPU (tests/test_gpu_cache.py), so here layers are
marked written with record_layer_write, the reference's hook for external
writers.
"""

from __future__ import annotations

import random

import pytest
import torch

from tensorforge_amd.cache import CacheExhaustedError, PagedKVCache, PagedKVCacheConfig


def _config(**overrides) -> PagedKVCacheConfig:
    values = dict(num_layers=1, num_blocks=4, block_size=2, num_kv_heads=2, head_dim=4,
                  max_sequences=2, max_sequence_length=8, dtype=torch.float32,
                  device=torch.device("cpu"))
    values.update(overrides)
    return PagedKVCacheConfig(**values)


def _write_all(cache: PagedKVCache, reservation) -> None:
    for layer in range(cache.config.num_layers):
        cache.record_layer_write(reservation, layer)


def test_config_validation() -> None:
    with pytest.raises(ValueError, match="num_blocks must be positive"):
        _config(num_blocks=0)
    with pytest.raises(TypeError, match="unsupported cache dtype"):
        _config(dtype=torch.int8)
    assert _config(max_sequence_length=9, block_size=4).max_blocks_per_sequence == 3


def test_append_crosses_logical_blocks() -> None:
    """tests/test_paged_cache.py:11-37: 3 tokens in 2-token pages -> [0, 1]."""

    cache = PagedKVCache(_config())
    cache.create_sequence("request-a")
    reservation = cache.begin_append("request-a", token_count=3)
    assert cache.layer_view("request-a", 0, reservation).context_length == 3
    _write_all(cache, reservation)
    cache.commit(reservation)
    view = cache.layer_view("request-a", layer_index=0)
    assert view.context_length == 3
    assert view.block_table.tolist()[:2] == [0, 1]
    assert int(cache.sequence_lengths[0]) == 3


def test_exhausted_append_is_atomic() -> None:
    """tests/test_paged_cache.py:40-70."""

    cache = PagedKVCache(_config(num_blocks=2, num_kv_heads=1))
    cache.create_sequence("owner")
    reservation = cache.begin_append("owner", 3)
    _write_all(cache, reservation)
    cache.commit(reservation)
    before = cache.stats()
    cache.create_sequence("waiting")
    with pytest.raises(CacheExhaustedError, match="only 0"):
        cache.begin_append("waiting", 1)
    after = cache.stats()
    assert after.used_blocks == before.used_blocks
    assert after.reserved_tokens == 0
    assert cache.layer_view("owner", 0).context_length == 3
    assert cache.layer_view("waiting", 0).context_length == 0


def test_rollback_returns_new_pages_for_deterministic_reuse() -> None:
    """tests/test_paged_cache.py:73-96."""

    cache = PagedKVCache(_config(num_blocks=3, num_kv_heads=1, max_sequence_length=6))
    cache.create_sequence("cancelled")
    cancelled = cache.begin_append("cancelled", 3)
    assert cache.layer_view("cancelled", 0, cancelled).block_table.tolist()[:2] == [0, 1]
    cache.rollback(cancelled)
    assert cache.stats().free_blocks == 3
    assert cache.layer_view("cancelled", 0).block_table.tolist()[:2] == [-1, -1]
    cache.create_sequence("replacement")
    replacement = cache.begin_append("replacement", 3)
    assert cache.layer_view("replacement", 0, replacement).block_table.tolist()[:2] == [0, 1]


def test_partial_commit_keeps_prefix_and_reclaims_tail_pages() -> None:
    """tests/test_paged_cache.py:99-121 (without the page contents)."""

    cache = PagedKVCache(_config(num_blocks=3, num_kv_heads=1, head_dim=2, max_sequences=1,
                                 max_sequence_length=6))
    cache.create_sequence("speculative")
    reservation = cache.begin_append("speculative", 3)
    _write_all(cache, reservation)
    cache.commit(reservation, accepted_tokens=1)
    assert cache.layer_view("speculative", 0).context_length == 1
    assert cache.stats().used_blocks == 1
    assert cache.layer_view("speculative", 0).block_table.tolist()[:2] == [0, -1]


def test_release_cancels_pending_append_and_returns_slot() -> None:
    """tests/test_paged_cache.py:124-150."""

    cache = PagedKVCache(_config(num_blocks=3, num_kv_heads=1, head_dim=2, max_sequences=1,
                                 max_sequence_length=6))
    cache.create_sequence("cancelled")
    committed = cache.begin_append("cancelled", 2)
    _write_all(cache, committed)
    cache.commit(committed)
    cache.begin_append("cancelled", 2)
    cache.release("cancelled")
    assert cache.stats().free_blocks == 3
    assert cache.stats().active_sequences == 0
    assert cache.block_owners() == (None, None, None)
    cache.create_sequence("replacement")
    assert cache.layer_view("replacement", 0).block_table.tolist() == [-1, -1, -1]


def test_optimized_writer_metadata_resolves_mapping() -> None:
    """tests/test_paged_cache.py:153-179."""

    cache = PagedKVCache(_config(num_layers=2, num_blocks=3, num_kv_heads=1, head_dim=2,
                                 max_sequences=1, max_sequence_length=6))
    cache.create_sequence("optimized")
    reservation = cache.begin_append("optimized", 3)
    assert cache.sequence_layout("optimized", reservation).physical_blocks == (0, 1)
    assert cache.sequence_layout("optimized", reservation).context_length == 3
    assert cache.append_location(reservation, 0).physical_block == 0
    assert cache.append_location(reservation, 2).physical_block == 1
    assert cache.append_location(reservation, 2).block_offset == 0
    with pytest.raises(RuntimeError, match="every cache layer"):
        cache.record_layer_write(reservation, 0)
        cache.commit(reservation)
    _write_all(cache, reservation)
    cache.commit(reservation)
    assert cache.sequence_layout("optimized").context_length == 3
    assert cache.stats().reserved_tokens == 0


def test_error_contract() -> None:
    cache = PagedKVCache(_config(max_sequences=1))
    with pytest.raises(ValueError, match="non-empty"):
        cache.create_sequence("")
    cache.create_sequence("a")
    with pytest.raises(ValueError, match="already exists"):
        cache.create_sequence("a")
    with pytest.raises(CacheExhaustedError, match="no free sequence slots"):
        cache.create_sequence("b")
    with pytest.raises(KeyError, match="unknown sequence"):
        cache.begin_append("zzz", 1)
    with pytest.raises(ValueError, match="positive"):
        cache.begin_append("a", 0)
    with pytest.raises(CacheExhaustedError, match="maximum sequence length"):
        cache.begin_append("a", 9)
    reservation = cache.begin_append("a", 2)
    with pytest.raises(RuntimeError, match="active append"):
        cache.begin_append("a", 1)
    with pytest.raises(IndexError, match="out of range"):
        cache.record_layer_write(reservation, 1)
    with pytest.raises(IndexError, match="outside the append reservation"):
        cache.append_location(reservation, 2)
    with pytest.raises(ValueError, match="within the reservation"):
        cache.commit(reservation, accepted_tokens=3)
    keys = torch.zeros(2, 2, 4)
    with pytest.raises(ValueError, match=r"must have shape \(2, 2, 4\)"):
        cache.write_layer(reservation, 0, keys[:1], keys[:1])
    with pytest.raises(ValueError, match="cache dtype and device"):
        cache.write_layer(reservation, 0, keys.half(), keys.half())
    with pytest.raises(ValueError, match="CUDA"):  # page writes run on the GPU only
        cache.write_layer(reservation, 0, keys, keys)
    cache.rollback(reservation)
    with pytest.raises(RuntimeError, match="no longer active"):
        cache.commit(reservation)


def test_seeded_request_churn_preserves_accounting() -> None:
    """tests/test_paged_cache.py:182-233, with layers recorded as written."""

    config = _config(num_layers=2, num_blocks=8, block_size=4, max_sequences=4,
                     max_sequence_length=16)
    cache = PagedKVCache(config)
    randomizer = random.Random(20260901)
    lengths: dict[str, int] = {}
    next_request = 0
    for _ in range(500):
        if len(lengths) < config.max_sequences and (not lengths or randomizer.random() < 0.3):
            request_id = f"request-{next_request}"
            next_request += 1
            cache.create_sequence(request_id)
            lengths[request_id] = 0
        else:
            request_id = randomizer.choice(list(lengths))
            if randomizer.random() < 0.25:
                cache.release(request_id)
                del lengths[request_id]
            else:
                remaining = config.max_sequence_length - lengths[request_id]
                if remaining:
                    token_count = randomizer.randint(1, min(5, remaining))
                    try:
                        reservation = cache.begin_append(request_id, token_count)
                    except CacheExhaustedError:
                        pass
                    else:
                        _write_all(cache, reservation)
                        accepted = randomizer.randint(0, token_count)
                        cache.commit(reservation, accepted_tokens=accepted)
                        lengths[request_id] += accepted
        stats = cache.stats()
        owners = cache.block_owners()
        assert stats.used_blocks == sum(owner is not None for owner in owners)
        assert stats.free_blocks + stats.used_blocks == stats.total_blocks
        assert stats.active_sequences == len(lengths)
        assert stats.committed_tokens == sum(lengths.values())
        assert stats.reserved_tokens == 0
        # The device table rows mirror the host page lists.
        for rid in lengths:
            layout = cache.sequence_layout(rid)
            row = cache.layer_view(rid, 0).block_table.tolist()
            assert row[:len(layout.physical_blocks)] == list(layout.physical_blocks)
            assert all(entry == -1 for entry in row[len(layout.physical_blocks):])
    for request_id in list(lengths):
        cache.release(request_id)
    assert cache.stats().free_blocks == config.num_blocks
