"""Host-side work list of the packed prefill attention (no GPU needed)."""

from __future__ import annotations

import numpy as np
import pytest

from tensorforge_amd.kernels.prefill import TILE, prefill_attention_supported, prefill_tiles


def test_prefill_tiles_cover_every_token_once():
    assert TILE == 64  # the kernel's work item: four wavefronts of 16 query tokens
    lengths = [1, 16, 17, 40, 64, 65, 200]
    tiles = prefill_tiles(lengths)
    covered = []
    for i0, s, e in tiles.tolist():
        assert s <= i0 < e and (i0 - s) % TILE == 0
        covered.extend(range(i0, min(i0 + TILE, e)))
    assert sorted(covered) == list(range(sum(lengths)))
    work = np.minimum(tiles[:, 0] + TILE, tiles[:, 2]) - tiles[:, 1]
    assert (np.diff(work) <= 0).all()  # heaviest first
    with pytest.raises(ValueError):
        prefill_tiles([3, 0])


def test_prefill_attention_geometry_gate():
    import torch

    assert prefill_attention_supported(torch.bfloat16, 32, 4, 64)
    assert prefill_attention_supported(torch.float16, 8, 2, 32)
    assert not prefill_attention_supported(torch.float32, 32, 4, 64)
    assert not prefill_attention_supported(torch.bfloat16, 12, 4, 64)  # group 3
    assert not prefill_attention_supported(torch.bfloat16, 4, 2, 80)
