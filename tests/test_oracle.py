"""Pins of the CPU oracle (runs without a GPU).

Each oracle function is checked against something it does not restate: the
reference's own known-answer tests, an independent library routine, pure
Python brute force, closed forms and invariants.  The mutation tests at the
end plant plausible mistakes in the oracle (a wrong GQA head map, a dropped
scale, a reversed page order, a dropped eps, a mask ignored) and check that
at least one pin rejects each of them -- a pin that cannot fail pins nothing.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
from torch.nn import functional as F

from oracle.reference import (
    gather_sequence,
    paged_gqa_decode_reference,
    paged_gqa_decode_split_reference,
    paged_kv_write_slots_reference,
    paged_kv_write_token_reference,
    residual_rms_norm_fused_reference,
    residual_rms_norm_reference,
    rms_norm_reference,
    swiglu_fused_reference,
    swiglu_reference,
    write_layer_slots,
)
from tensorforge_amd.workloads import make_decode_attention_case

from helpers import assert_bit_exact


# ---------------------------------------------------------------------------
# Attention pins.  Each takes an attention implementation with the oracle's
# signature, so the mutation tests can run the same pins on planted mistakes.
# ---------------------------------------------------------------------------
def pin_reference_known_answer(attention) -> None:
    """tests/test_decode_attention.py:9-29 of the reference: two 2-token
    pages visited through the non-contiguous table [2, 0], 3 tokens, GQA
    group 2, expected by dense concatenation + repeat_interleave."""

    generator = torch.Generator().manual_seed(0)
    query = torch.randn(1, 4, 8, generator=generator)
    key_cache = torch.randn(3, 2, 2, 8, generator=generator)
    value_cache = torch.randn(3, 2, 2, 8, generator=generator)
    block_tables = torch.tensor([[2, 0]], dtype=torch.int32)
    context_lengths = torch.tensor([3], dtype=torch.int32)
    actual = attention(query, key_cache, value_cache, block_tables, context_lengths)
    dense_keys = torch.cat((key_cache[2], key_cache[0, :1]), dim=0).repeat_interleave(2, dim=1)
    dense_values = torch.cat((value_cache[2], value_cache[0, :1]), dim=0).repeat_interleave(2, dim=1)
    scores = torch.einsum("bhd,thd->bht", query, dense_keys) / 8**0.5
    expected = torch.einsum("bht,thd->bhd", scores.softmax(dim=-1), dense_values)
    torch.testing.assert_close(actual, expected)


def _sdpa_expected(case) -> torch.Tensor:
    """F.scaled_dot_product_attention(enable_gqa=True) over the gathered
    sequence, row by row (an independent library routine)."""

    rows = []
    tables = case.block_tables.tolist()
    for b, ctx in enumerate(case.lengths):
        keys, values = gather_sequence(case.key_cache, case.value_cache, tables[b], ctx)
        q = case.query[b].float()[:, None, :]  # [Hq, 1, D]
        k = keys.float().permute(1, 0, 2).contiguous()  # [Hkv, T, D]
        v = values.float().permute(1, 0, 2).contiguous()
        out = F.scaled_dot_product_attention(q, k, v, scale=case.scale, enable_gqa=True)
        rows.append(out[:, 0, :])
    return torch.stack(rows).to(case.query.dtype)


def pin_sdpa(attention) -> None:
    for lengths, hq, hkv, d, page in (
        ([1, 7, 33], 8, 2, 16, 4),
        ([129, 5], 8, 1, 32, 16),
        ([40, 17, 64], 12, 3, 8, 16),
    ):
        case = make_decode_attention_case(
            lengths, query_heads=hq, kv_heads=hkv, head_dim=d, block_size=page,
            dtype=torch.float32, seed=sum(lengths),
        )
        actual = attention(case.query, case.key_cache, case.value_cache, case.block_tables,
                           case.context_lengths, scale=case.scale)
        torch.testing.assert_close(actual, _sdpa_expected(case), rtol=1e-5, atol=1e-5)


def pin_brute_force(attention) -> None:
    """Pure-Python loops with math.exp on a tiny float64-exact case."""

    case = make_decode_attention_case(
        [5, 3], query_heads=4, kv_heads=2, head_dim=3, block_size=2, dtype=torch.float32, seed=5,
    )
    scale = 0.7
    actual = attention(case.query, case.key_cache, case.value_cache, case.block_tables,
                       case.context_lengths, scale=scale)
    q = case.query.tolist()
    kc = case.key_cache.tolist()
    vc = case.value_cache.tolist()
    tables = case.block_tables.tolist()
    group = 4 // 2
    for b, ctx in enumerate(case.lengths):
        for h in range(4):
            kvh = h // group
            scores = []
            for t in range(ctx):
                page, slot = tables[b][t // 2], t % 2
                scores.append(scale * sum(q[b][h][i] * kc[page][slot][kvh][i] for i in range(3)))
            top = max(scores)
            weights = [math.exp(s - top) for s in scores]
            total = sum(weights)
            for i in range(3):
                expected = sum(
                    w * vc[tables[b][t // 2]][t % 2][kvh][i] for t, w in enumerate(weights)
                ) / total
                assert abs(float(actual[b, h, i]) - expected) < 1e-5, (b, h, i)


def pin_closed_forms(attention) -> None:
    """Zero keys (or zero scale) weight every token equally, so the output is
    the mean of the row's values; one key aligned with q and scaled up takes
    all the weight, so the output is its value."""

    case = make_decode_attention_case(
        [9, 16, 1], query_heads=8, kv_heads=2, head_dim=16, block_size=4, dtype=torch.float32,
        seed=2,
    )
    tables = case.block_tables.tolist()
    means = []
    for b, ctx in enumerate(case.lengths):
        _, values = gather_sequence(case.key_cache, case.value_cache, tables[b], ctx)
        means.append(values.float().mean(dim=0).repeat_interleave(4, dim=0))  # [Hq, D]
    expected_mean = torch.stack(means)
    zero_keys = attention(case.query, torch.zeros_like(case.key_cache), case.value_cache,
                          case.block_tables, case.context_lengths, scale=case.scale)
    torch.testing.assert_close(zero_keys, expected_mean, rtol=1e-5, atol=1e-5)
    zero_scale = attention(case.query, case.key_cache, case.value_cache, case.block_tables,
                           case.context_lengths, scale=0.0)
    torch.testing.assert_close(zero_scale, expected_mean, rtol=1e-5, atol=1e-5)

    # Dominant key: token `hit` of row 0 is 100 * q for every kv head; all
    # other keys are tiny.
    key_cache = case.key_cache * 1e-3
    hit = 6
    page, slot = tables[0][hit // 4], hit % 4
    query = case.query.clone()
    # The four query heads of a group are equal, so all see the same dominant key.
    for kvh in range(2):
        query[0, 4 * kvh:4 * kvh + 4] = case.query[0, 4 * kvh]
        key_cache[page, slot, kvh] = 100.0 * query[0, 4 * kvh]
    out = attention(query, key_cache, case.value_cache, case.block_tables, case.context_lengths,
                    scale=1.0)
    expected = case.value_cache[page, slot].repeat_interleave(4, dim=0)
    torch.testing.assert_close(out[0], expected, rtol=1e-5, atol=1e-5)


def pin_gqa_head_map(attention) -> None:
    """Values constant per kv head: every query head h must return the
    constant of kv head h // group (softmax weights sum to one)."""

    case = make_decode_attention_case(
        [11, 30], query_heads=12, kv_heads=3, head_dim=8, block_size=8, dtype=torch.float32,
        seed=8,
    )
    constants = torch.tensor([-2.0, 0.5, 3.0])
    values = constants.view(1, 1, 3, 1).expand_as(case.value_cache).contiguous()
    out = attention(case.query, case.key_cache, values, case.block_tables, case.context_lengths,
                    scale=case.scale)
    expected = constants.repeat_interleave(4).view(1, 12, 1).expand(2, 12, 8)
    torch.testing.assert_close(out, expected, rtol=1e-6, atol=1e-6)


def pin_page_permutation(attention) -> None:
    """Moving pages to other physical slots and remapping the table gives the
    same output bit for bit; garbage in unused pages and past the length is
    never read."""

    case = make_decode_attention_case(
        [37, 64, 3], query_heads=8, kv_heads=2, head_dim=16, block_size=8, dtype=torch.float32,
        seed=4, extra_pages=5,
    )
    base = attention(case.query, case.key_cache, case.value_cache, case.block_tables,
                     case.context_lengths, scale=case.scale)
    pages = case.key_cache.shape[0]
    perm = torch.randperm(pages, generator=torch.Generator().manual_seed(9))
    inverse = torch.empty_like(perm)
    inverse[perm] = torch.arange(pages)
    key_cache = case.key_cache[perm].clone()
    value_cache = case.value_cache[perm].clone()
    tables = case.block_tables.clone()
    valid = tables >= 0
    tables[valid] = inverse[tables[valid].long()].to(torch.int32)
    # Poison tokens past each row's length inside its last page.
    for b, ctx in enumerate(case.lengths):
        last_page = int(tables[b, (ctx - 1) // 8])
        key_cache[last_page, (ctx - 1) % 8 + 1:] = float("nan")
        value_cache[last_page, (ctx - 1) % 8 + 1:] = float("nan")
    moved = attention(case.query, key_cache, value_cache, tables, case.context_lengths,
                      scale=case.scale)
    assert_bit_exact(moved, base, "page permutation")


ATTENTION_PINS = (
    pin_reference_known_answer,
    pin_sdpa,
    pin_brute_force,
    pin_closed_forms,
    pin_gqa_head_map,
    pin_page_permutation,
)


@pytest.mark.parametrize("pin", ATTENTION_PINS, ids=lambda pin: pin.__name__)
def test_attention_oracle_pins(pin) -> None:
    pin(paged_gqa_decode_reference)


@pytest.mark.parametrize("split_size", [1, 3, 16, 64, 4096])
def test_split_oracle_equals_one_pass(split_size: int) -> None:
    """The two-stage LSE merge reproduces one-pass softmax for any split."""

    case = make_decode_attention_case(
        [1, 17, 200, 64], query_heads=8, kv_heads=2, head_dim=32, block_size=16,
        dtype=torch.float32, seed=split_size,
    )
    args = (case.query, case.key_cache, case.value_cache, case.block_tables, case.context_lengths)
    one_pass = paged_gqa_decode_reference(*args, scale=case.scale)
    split = paged_gqa_decode_split_reference(*args, split_size=split_size, scale=case.scale)
    torch.testing.assert_close(split, one_pass, rtol=2e-6, atol=2e-6)


@pytest.mark.parametrize("pin", ATTENTION_PINS, ids=lambda pin: pin.__name__)
def test_split_oracle_pins(pin) -> None:
    pin(lambda *a, **k: paged_gqa_decode_split_reference(*a, split_size=3, **k))


def test_attention_oracle_rejects_what_the_reference_rejects() -> None:
    """reference.py:74-84: non-positive length, table overflow, bad page."""

    q = torch.zeros(1, 2, 4)
    cache = torch.zeros(2, 4, 1, 4)
    with pytest.raises(ValueError, match="positive"):
        paged_gqa_decode_reference(q, cache, cache, torch.tensor([[0]], dtype=torch.int32),
                                   torch.tensor([0], dtype=torch.int32))
    with pytest.raises(ValueError, match="capacity"):
        paged_gqa_decode_reference(q, cache, cache, torch.tensor([[0]], dtype=torch.int32),
                                   torch.tensor([5], dtype=torch.int32))
    with pytest.raises(ValueError, match="invalid physical block"):
        paged_gqa_decode_reference(q, cache, cache, torch.tensor([[2]], dtype=torch.int32),
                                   torch.tensor([3], dtype=torch.int32))


# ---------------------------------------------------------------------------
# RMSNorm / residual RMSNorm / SwiGLU
# ---------------------------------------------------------------------------
def pin_rms_norm(rms_norm) -> None:
    """F.rms_norm (library); the explicit formula of the reference's
    tests/test_layers.py:10-19; constant rows: y = c / sqrt(c^2 + eps) * w."""

    generator = torch.Generator().manual_seed(3)
    x = torch.randn(5, 96, generator=generator)
    w = torch.rand(96, generator=generator) + 0.5
    torch.testing.assert_close(rms_norm(x, w, 1e-5), F.rms_norm(x, (96,), w, 1e-5),
                               rtol=1e-6, atol=1e-6)
    for c in (-3.0, 1e-3, 250.0):
        row = torch.full((1, 64), c)
        expected = c / math.sqrt(c * c + 1e-6) * w[:64]
        torch.testing.assert_close(rms_norm(row, w[:64], 1e-6)[0], expected, rtol=1e-6, atol=1e-7)


def test_rms_norm_oracle_pins() -> None:
    pin_rms_norm(rms_norm_reference)


def test_rms_norm_oracle_rounds_once() -> None:
    """bf16 in, fp32 arithmetic, one rounding of the fp32 result."""

    x = torch.randn(4, 128).to(torch.bfloat16)
    w = (torch.randn(128) * 0.1 + 1).to(torch.bfloat16)
    exact = F.rms_norm(x.double(), (128,), w.double(), 1e-5)
    assert_bit_exact(rms_norm_reference(x, w, 1e-5), exact.float().to(torch.bfloat16), "rounding")


def test_residual_oracles() -> None:
    """The rounded residual sum is torch's bit for bit; the reference
    oracle normalises the rounded sum (reference.py:24-30); the fused form
    normalises the fp32 sum (triton_ops.py:89-97), recomputed in fp64."""

    x = torch.randn(6, 256).to(torch.bfloat16)
    r = torch.randn(6, 256).to(torch.bfloat16)
    w = (torch.randn(256) * 0.1 + 1).to(torch.bfloat16)
    summed, norm = residual_rms_norm_reference(x, r, w, 1e-5)
    assert_bit_exact(summed, x + r, "rounded sum")
    torch.testing.assert_close(norm, F.rms_norm(summed.float(), (256,), w.float(), 1e-5).to(
        torch.bfloat16))
    fused_sum, fused_norm = residual_rms_norm_fused_reference(x, r, w, 1e-5)
    assert_bit_exact(fused_sum, (x.float() + r.float()).to(torch.bfloat16), "fused sum")
    # The norm output against a library routine: F.rms_norm over the fp32
    # sum (not the rounded one), one rounding -- within one bf16 ulp, and it
    # must differ from the normalised rounded sum somewhere (the two
    # semantics the reference distinguishes, docs/kernel-design.md:33-39).
    s = x.float() + r.float()
    library = F.rms_norm(s.double(), (256,), w.double(), 1e-5).to(torch.bfloat16)
    ulp = (library.float().abs() * 2.0 ** -7).clamp_min(2.0 ** -133)
    assert bool(((fused_norm.float() - library.float()).abs() <= ulp).all())
    assert bool((fused_norm.float() == library.float()).float().mean() > 0.95)
    rounded_sum_norm = F.rms_norm(summed.double(), (256,), w.double(), 1e-5).to(torch.bfloat16)
    assert not torch.equal(fused_norm, rounded_sum_norm)
    # Cancellation (reference tests/test_triton_kernels.py:113-127): x + (-x) = 0 -> 0.
    zero_sum, zero_norm = residual_rms_norm_fused_reference(x, -x, w, 1e-5)
    assert not bool(zero_sum.float().abs().max()) and not bool(zero_norm.float().abs().max())


def pin_swiglu(swiglu) -> None:
    """F.silu (library) and per-element math.exp: g / (1 + e^-g) * u."""

    generator = torch.Generator().manual_seed(6)
    g = torch.randn(3, 40, generator=generator) * 4
    u = torch.randn(3, 40, generator=generator)
    torch.testing.assert_close(swiglu(g, u), F.silu(g) * u, rtol=1e-6, atol=1e-6)
    for gv, uv in ((0.0, 5.0), (1.5, -2.0), (-30.0, 1.0), (30.0, 0.5)):
        out = float(swiglu(torch.tensor([gv]), torch.tensor([uv]))[0])
        assert abs(out - gv / (1.0 + math.exp(-gv)) * uv) <= 1e-6 * max(1.0, abs(out))


def test_swiglu_oracle_pins() -> None:
    pin_swiglu(swiglu_reference)
    pin_swiglu(swiglu_fused_reference)


def test_swiglu_fused_oracle_rounds_once() -> None:
    g = torch.randn(4, 300).to(torch.float16)
    u = torch.randn(4, 300).to(torch.float16)
    exact = (g.double() * torch.sigmoid(g.double()) * u.double()).float().to(torch.float16)
    mismatch = (swiglu_fused_reference(g, u).float() - exact.float()).abs()
    # fp32 arithmetic may differ from fp64 by one fp16 ulp at a rounding tie.
    assert float(mismatch.max()) <= float(exact.float().abs().max()) * 2**-10


# ---------------------------------------------------------------------------
# KV writes
# ---------------------------------------------------------------------------
def test_write_slots_reference_known_answer() -> None:
    """tests/test_paged_cache.py:11-37 of the reference: 3 tokens of arange
    keys (values = keys + 100) into 2-token pages [0, 1] read back in order."""

    keys = torch.arange(24, dtype=torch.float32).view(3, 2, 4)
    values = keys + 100
    key_cache = torch.zeros(4, 2, 2, 4)
    value_cache = torch.zeros(4, 2, 2, 4)
    slots = torch.from_numpy(write_layer_slots([0, 1], 0, 3, 2))
    assert slots.tolist() == [0, 1, 2]
    k_out, v_out = paged_kv_write_slots_reference(keys, values, key_cache, value_cache, slots)
    got_k, got_v = gather_sequence(k_out, v_out, [0, 1], 3)
    torch.testing.assert_close(got_k, keys)
    torch.testing.assert_close(got_v, values)
    assert not bool(k_out[2:].any()) and not bool(v_out[2:].any())


def test_write_layer_slots_crosses_pages() -> None:
    """Positions start..start+T-1 map through the sequence's page list:
    slot = blocks[p // page] * page + p % page (cache/paged.py:221-233)."""

    blocks = [7, 2, 5]
    slots = write_layer_slots(blocks, start_position=3, token_count=6, block_size=4)
    expected = [blocks[p // 4] * 4 + p % 4 for p in range(3, 9)]
    assert slots.tolist() == expected == [31, 8, 9, 10, 11, 20]


def test_write_token_reference_is_bit_exact_and_masked() -> None:
    """Dense brute force: active lanes overwrite exactly one token row of
    each cache with their raw bits (NaN payloads and -0.0 survive);
    masked lanes write nothing."""

    kv_heads, head_dim, pages, page = 2, 8, 5, 4
    key_cache = torch.randn(pages, page, kv_heads, head_dim).to(torch.bfloat16)
    value_cache = torch.randn(pages, page, kv_heads, head_dim).to(torch.bfloat16)
    keys = torch.randn(3, kv_heads, head_dim).to(torch.bfloat16)
    values = torch.randn(3, kv_heads, head_dim).to(torch.bfloat16)
    keys.view(torch.int16)[0, 0, 0] = 0x7FC1  # NaN with a payload
    values.view(torch.int16)[0, 0, 1] = -32768  # -0.0
    phys = torch.tensor([4, 1, 1], dtype=torch.int32)
    offs = torch.tensor([3, 0, 2], dtype=torch.int32)
    mask = torch.tensor([1, 0, 1], dtype=torch.int32)
    k_out, v_out = paged_kv_write_token_reference(keys, values, key_cache, value_cache,
                                                  phys, offs, mask)
    k_expected, v_expected = key_cache.clone(), value_cache.clone()
    for lane in (0, 2):
        k_expected.view(torch.int16)[phys[lane], offs[lane]] = keys.view(torch.int16)[lane]
        v_expected.view(torch.int16)[phys[lane], offs[lane]] = values.view(torch.int16)[lane]
    assert_bit_exact(k_out, k_expected, "keys")
    assert_bit_exact(v_out, v_expected, "values")
    assert int(k_out.view(torch.int16)[4, 3, 0, 0]) == 0x7FC1
    assert int(v_out.view(torch.int16)[4, 3, 0, 1]) == -32768
    assert_bit_exact(k_out[1, 0], key_cache[1, 0], "masked lane untouched")


def test_write_slots_reference_skips_negative_and_out_of_range_slots() -> None:
    cache = torch.zeros(2, 2, 1, 2, dtype=torch.float16)
    rows = torch.tensor([[[1.0, 2.0]], [[3.0, 4.0]], [[5.0, 6.0]]], dtype=torch.float16)
    slots = torch.tensor([-1, 3, 4], dtype=torch.int64)
    k_out, v_out = paged_kv_write_slots_reference(rows, rows, cache, cache, slots)
    expected = torch.zeros_like(cache)
    expected[1, 1] = rows[1]
    assert_bit_exact(k_out, expected)
    assert_bit_exact(v_out, expected)


# ---------------------------------------------------------------------------
# Mutation tests: planted mistakes must fail at least one pin.
# ---------------------------------------------------------------------------
def _mutant_gqa_modulo(query, key_cache, value_cache, block_tables, context_lengths, scale=None):
    """Query head h reads kv head h % kv_heads instead of h // group."""

    hq, hkv = query.shape[1], key_cache.shape[2]
    group = hq // hkv
    sigma = torch.tensor([(h % hkv) * group + h // hkv for h in range(hq)])
    permuted = torch.empty_like(query)
    permuted[:, sigma] = query
    out = paged_gqa_decode_reference(permuted, key_cache, value_cache, block_tables,
                                     context_lengths, scale=scale)
    return out[:, sigma]


def _mutant_dropped_scale(query, key_cache, value_cache, block_tables, context_lengths,
                          scale=None):
    return paged_gqa_decode_reference(query, key_cache, value_cache, block_tables,
                                      context_lengths, scale=1.0)


def _mutant_reversed_pages(query, key_cache, value_cache, block_tables, context_lengths,
                           scale=None):
    """Logical pages visited in reverse order."""

    tables = block_tables.clone()
    page = key_cache.shape[1]
    for b, ctx in enumerate(context_lengths.tolist()):
        used = (ctx + page - 1) // page
        tables[b, :used] = block_tables[b, :used].flip(0)
    return paged_gqa_decode_reference(query, key_cache, value_cache, tables, context_lengths,
                                      scale=scale)


def _mutant_unmasked_tail(query, key_cache, value_cache, block_tables, context_lengths,
                          scale=None):
    """Whole last page attended, ignoring the length inside it."""

    page = key_cache.shape[1]
    padded = ((context_lengths + page - 1) // page) * page
    return paged_gqa_decode_reference(query, key_cache, value_cache, block_tables,
                                      padded.to(torch.int32), scale=scale)


@pytest.mark.parametrize(
    "mutant",
    [_mutant_gqa_modulo, _mutant_dropped_scale, _mutant_reversed_pages, _mutant_unmasked_tail],
    ids=lambda m: m.__name__,
)
def test_attention_pins_reject_planted_mistakes(mutant) -> None:
    failures = 0
    for pin in ATTENTION_PINS:
        try:
            pin(mutant)
        except (AssertionError, ValueError):
            failures += 1
    assert failures >= 1, f"no pin rejects {mutant.__name__}"


def test_norm_and_swiglu_pins_reject_planted_mistakes() -> None:
    def rms_without_eps(x, w, eps):
        return rms_norm_reference(x, w, 0.0)

    def rms_sum_not_mean(x, w, eps):
        return rms_norm_reference(x / math.sqrt(x.shape[-1]), w, eps)

    def swiglu_sigmoid_only(g, u):
        return torch.sigmoid(g) * u

    for mutant in (rms_without_eps, rms_sum_not_mean):
        with pytest.raises(AssertionError):
            pin_rms_norm(mutant)
    with pytest.raises(AssertionError):
        pin_swiglu(swiglu_sigmoid_only)


def test_gather_sequence_order_is_logical() -> None:
    """Tokens come out in logical order: page table[i] holds tokens
    [i * page, (i + 1) * page)."""

    cache = torch.arange(4 * 3, dtype=torch.float32).view(4, 3, 1, 1)
    keys, _ = gather_sequence(cache, cache, [2, 0, 3], 7)
    assert keys.flatten().tolist() == [6.0, 7.0, 8.0, 0.0, 1.0, 2.0, 9.0]
    assert np.array_equal(keys.flatten().numpy(), np.array([6, 7, 8, 0, 1, 2, 9], np.float32))
