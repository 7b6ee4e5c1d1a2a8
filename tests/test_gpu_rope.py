"""Parity of the fused decode RoPE + paged KV append with the CPU oracle.

Rotated query and key: within the elementwise tolerances of the reference
(tests/test_triton_kernels.py:21-26: fp32 1e-5, fp16 3e-3, bf16 3e-2 --
one rounding of an fp32 result, so at most one unit in the last place
apart); value rows and every cache row the step must not touch: bit-exact
(tests/test_decode_bucket.py:233-287 for padded lanes).
"""

from __future__ import annotations

import pytest
import torch

from helpers import assert_bit_exact
from oracle.model import rope_tables
from oracle.reference import rope_kv_append_reference
from tensorforge_amd.kernels import rope_paged_kv_append

pytestmark = pytest.mark.gpu

TOLERANCE = {torch.float32: 1e-5, torch.float16: 3e-3, torch.bfloat16: 3e-2}


def _case(batch, hq, hkv, d, dtype, seed, *, row_pad=0, num_blocks=40, block_size=16):
    generator = torch.Generator().manual_seed(seed)
    width = (hq + 2 * hkv) * d
    qkv = torch.randn(batch, width + row_pad, generator=generator).to(dtype)
    cos, sin = rope_tables(d, 10000.0, torch.arange(4096))
    positions = torch.randint(0, 4096, (batch,), generator=generator)
    slots = torch.randperm(num_blocks * block_size, generator=generator)[:batch]
    pages = (slots // block_size).to(torch.int32)
    offsets = (slots % block_size).to(torch.int32)
    active = (torch.rand(batch, generator=generator) < 0.8).to(torch.int32)
    key_cache = torch.randn(num_blocks, block_size, hkv, d, generator=generator).to(dtype)
    value_cache = torch.randn(num_blocks, block_size, hkv, d, generator=generator).to(dtype)
    return qkv, positions, cos.to(dtype), sin.to(dtype), key_cache, value_cache, pages, offsets, active


def _run(device, case, hq, width=None):
    """`width` < the buffer's row length slices the rows on the device, so
    the kernel sees a row stride longer than the row."""

    qkv, positions, cos, sin, key_cache, value_cache, pages, offsets, active = case
    k_dev, v_dev = key_cache.to(device), value_cache.to(device)
    qkv_dev = qkv.to(device)
    if width is not None:
        qkv_dev = qkv_dev[:, :width]
        assert qkv_dev.stride(0) > width
    q = rope_paged_kv_append(qkv_dev, positions.to(device), cos.to(device), sin.to(device),
                             k_dev, v_dev, pages.to(device), offsets.to(device),
                             active.to(device), query_heads=hq)
    return q, k_dev, v_dev


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize(("batch", "hq", "hkv", "d"),
                         [(72, 32, 4, 64), (4, 32, 8, 128), (9, 8, 2, 32), (3, 2, 1, 80)])
def test_rope_append_matches_the_oracle(device, dtype, batch, hq, hkv, d):
    case = _case(batch, hq, hkv, d, dtype, seed=batch * 7 + d)
    q, k_dev, v_dev = _run(device, case, hq)
    q_ref, k_ref, v_ref = rope_kv_append_reference(*case, hq)
    tol = TOLERANCE[dtype]
    torch.testing.assert_close(q.float().cpu(), q_ref, rtol=tol, atol=tol)
    torch.testing.assert_close(k_dev.float().cpu(), k_ref.float(), rtol=tol, atol=tol)
    assert_bit_exact(v_dev, v_ref, "value cache")
    # Rows no active lane targets: bit-identical to the input pool.
    key_cache, pages, offsets, active = case[4], case[6], case[7], case[8]
    touched = torch.zeros(key_cache.shape[:2], dtype=torch.bool)
    for lane in range(batch):
        if active[lane]:
            touched[pages[lane], offsets[lane]] = True
    assert_bit_exact(k_dev.cpu()[~touched], key_cache[~touched], "untouched key rows")


def test_rope_append_writes_dense_keys(device):
    """key_output receives every lane's rotated key, masked lanes included,
    bit-identical to what active lanes store in their pages."""

    case = _case(24, 8, 2, 64, torch.bfloat16, seed=5)
    qkv, positions, cos, sin, key_cache, value_cache, pages, offsets, active = \
        [t.to(device) for t in case]
    keys = torch.empty(24, 2, 64, dtype=torch.bfloat16, device=device)
    rope_paged_kv_append(qkv, positions, cos, sin, key_cache, value_cache, pages, offsets, active,
                         query_heads=8, key_output=keys)
    q_ref, k_ref, _ = rope_kv_append_reference(*case, 8)
    for lane in range(24):
        if case[8][lane]:
            assert_bit_exact(keys[lane], key_cache[pages[lane], offsets[lane]], f"lane {lane}")
    # The oracle's rotation of lane b's key equals q's formula on the k head.
    rows = case[0].float().view(24, 12, 64)
    half = 32
    cs = case[2].float()[case[1]][:, None, :]
    sn = case[3].float()[case[1]][:, None, :]
    k_in = rows[:, 8:10]
    expected = k_in * cs + torch.cat((-k_in[..., half:], k_in[..., :half]), -1) * sn
    torch.testing.assert_close(keys.float().cpu(), expected, rtol=3e-2, atol=3e-2)


def test_rope_append_reads_strided_rows(device):
    """qkv as a column slice of a wider projection output (row stride >
    row length), as when the projection is fused with another GEMM."""

    case = _case(16, 32, 4, 64, torch.bfloat16, seed=3, row_pad=96)
    width = (32 + 2 * 4) * 64
    q, k_dev, v_dev = _run(device, case, 32, width=width)
    q_ref, k_ref, v_ref = rope_kv_append_reference(case[0][:, :width], *case[1:], 32)
    torch.testing.assert_close(q.float().cpu(), q_ref, rtol=3e-2, atol=3e-2)
    assert_bit_exact(v_dev, v_ref, "value cache")


def test_rope_append_rejects_bad_arguments(device):
    case = _case(4, 8, 2, 32, torch.float16, seed=1)
    qkv, positions, cos, sin, key_cache, value_cache, pages, offsets, active = \
        [t.to(device) for t in case]
    with pytest.raises(ValueError, match="int64"):
        rope_paged_kv_append(qkv, positions.int(), cos, sin, key_cache, value_cache, pages,
                             offsets, active, query_heads=8)
    with pytest.raises(ValueError, match="shorter"):
        rope_paged_kv_append(qkv[:, :100], positions, cos, sin, key_cache, value_cache, pages,
                             offsets, active, query_heads=8)
    with pytest.raises(ValueError, match="share dtype"):
        rope_paged_kv_append(qkv, positions, cos.float(), sin.float(), key_cache, value_cache,
                             pages, offsets, active, query_heads=8)
