"""Pins of the decoder oracle (oracle/model.py), on the CPU."""

from __future__ import annotations

import math

import pytest
import torch

from oracle.model import (
    apply_rope,
    decode_step_reference,
    decoder_forward,
    rope_tables,
    rotate_half,
)
from oracle.reference import (
    paged_gqa_decode_reference,
    rms_norm_reference,
    rope_kv_append_reference,
)
from tensorforge_amd.decode import DecoderConfig, DecoderWeights


def tiny_config() -> DecoderConfig:
    return DecoderConfig(vocab_size=50, hidden_size=32, intermediate_size=48, num_hidden_layers=2,
                         num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64)


def test_rope_closed_forms() -> None:
    """Position 0 is the identity; rotation keeps norms; q(m).k(n) depends
    only on m - n; a hand-rotated pair (x0, x_{D/2}) turns by p * theta^0."""

    d = 16
    cos, sin = rope_tables(d, 10000.0, torch.arange(40))
    x = torch.randn(3, d)
    assert torch.allclose(apply_rope(x, cos[:1], sin[:1]), x)
    rotated = apply_rope(x[:, None, :].expand(3, 40, d), cos, sin)
    assert torch.allclose(rotated.norm(dim=-1), x.norm(dim=-1)[:, None].expand(3, 40), atol=1e-5)
    q, k = torch.randn(d), torch.randn(d)
    rq = apply_rope(q.expand(40, d), cos, sin)
    rk = apply_rope(k.expand(40, d), cos, sin)
    assert math.isclose(float(rq[10] @ rk[7]), float(rq[33] @ rk[30]), rel_tol=1e-4, abs_tol=1e-5)
    assert math.isclose(float(rq[5] @ rk[5]), float(q @ k), rel_tol=1e-4, abs_tol=1e-5)
    e = torch.zeros(d)
    e[0] = 1.0
    out = apply_rope(e[None], cos[3:4], sin[3:4])[0]
    assert math.isclose(float(out[0]), math.cos(3.0), abs_tol=1e-6)
    assert math.isclose(float(out[d // 2]), math.sin(3.0), abs_tol=1e-6)
    assert torch.equal(rotate_half(torch.arange(4.0)), torch.tensor([-2.0, -3.0, 0.0, 1.0]))


def test_rope_tables_carry_the_references_fp32_angle_rounding() -> None:
    """The tables are built in fp32 as the reference builds them
    (layers.py:38-46), not from exact angles: against exact fp64 angles
    p * theta^(-2i/D) every entry is within the error that fp32 rounding of
    the frequency and of the product explains (and well outside a table of
    some other frequency law), while at large positions the rounding shows
    (entries differ from the exact-angle table by more than fp32 cos/sin
    rounding alone would)."""

    d, theta = 64, 10000.0
    positions = torch.arange(4096)
    cos, sin = rope_tables(d, theta, positions)
    assert cos.dtype == torch.float32 and cos.shape == (4096, d)
    exponent = torch.arange(0, d, 2, dtype=torch.float64) / d
    exact = positions.double()[:, None] * theta ** (-exponent)[None, :]
    exact = torch.cat((exact, exact), dim=-1)
    # fp32 inv_freq (pow and division: a few ulps) and the fp32 product.
    bound = exact.abs() * 6 * 2.0 ** -24 + 1e-6
    assert bool(((cos.double() - exact.cos()).abs() <= bound).all())
    assert bool(((sin.double() - exact.sin()).abs() <= bound).all())
    assert float((cos.double() - exact.cos()).abs().max()) > 1e-5
    # Identity at position 0, unit norm everywhere.
    assert torch.equal(cos[0], torch.ones(d)) and torch.equal(sin[0], torch.zeros(d))
    assert float((cos.double() ** 2 + sin.double() ** 2 - 1).abs().max()) < 1e-6


def _brute_force_logits(weights: DecoderWeights, tokens: list[int]) -> torch.Tensor:
    """The same decoder written as explicit per-position loops over heads
    and keys (math.exp softmax), fp64."""

    config = weights.config
    hq, hkv, d = config.num_attention_heads, config.num_key_value_heads, config.head_dim
    f64 = lambda t: t.detach().cpu().double()  # noqa: E731
    seq = len(tokens)
    x = f64(weights.embedding)[torch.tensor(tokens)]
    cos, sin = rope_tables(d, config.rope_theta, torch.arange(seq))
    cos, sin = cos.double(), sin.double()

    def norm(v, w):
        return v / torch.sqrt((v * v).mean(-1, keepdim=True) + config.rms_norm_eps) * f64(w)

    for layer in weights.layers:
        h = norm(x, layer.input_norm)
        qkv = h @ f64(layer.qkv).T
        q = apply_rope(qkv[:, :hq * d].view(seq, hq, d).transpose(0, 1), cos, sin)
        k = apply_rope(qkv[:, hq * d:(hq + hkv) * d].view(seq, hkv, d).transpose(0, 1), cos, sin)
        v = qkv[:, (hq + hkv) * d:].view(seq, hkv, d).transpose(0, 1)
        context = torch.zeros(seq, hq * d, dtype=torch.float64)
        for t in range(seq):
            for head in range(hq):
                kv = head // (hq // hkv)
                scores = [float(q[head, t] @ k[kv, s]) / math.sqrt(d) for s in range(t + 1)]
                top = max(scores)
                weights_t = [math.exp(s - top) for s in scores]
                total = sum(weights_t)
                for s, w in enumerate(weights_t):
                    context[t, head * d:(head + 1) * d] += (w / total) * v[kv, s]
        x = x + context @ f64(layer.o_proj).T
        h = norm(x, layer.post_norm)
        gate, up = h @ f64(layer.gate).T, h @ f64(layer.up).T
        x = x + (gate / (1 + torch.exp(-gate)) * up) @ f64(layer.down).T
    return norm(x, weights.final_norm) @ f64(weights.lm_head).T


def test_decoder_oracle_matches_brute_force() -> None:
    weights = DecoderWeights.random(tiny_config(), seed=3, dtype=torch.float32, device="cpu")
    for layer in weights.layers:  # non-trivial norm weights
        layer.input_norm.uniform_(0.5, 1.5)
        layer.post_norm.uniform_(0.5, 1.5)
    tokens = [3, 17, 42, 0, 9, 33, 8]
    expected = _brute_force_logits(weights, tokens).float()
    actual = decoder_forward(weights, torch.tensor(tokens))
    torch.testing.assert_close(actual, expected, rtol=1e-4, atol=1e-5)


def test_last_position_attention_is_the_decode_oracle() -> None:
    """The oracle's causal attention at the last position equals
    paged_gqa_decode_reference over the same (rotated) keys and values laid
    out in pages."""

    config = tiny_config()
    weights = DecoderWeights.random(config, seed=5, dtype=torch.float32, device="cpu")
    tokens = torch.tensor([1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11])
    seq, hq, hkv, d = len(tokens), 4, 2, config.head_dim
    layer = weights.layers[0]
    x = weights.embedding[tokens]
    h = rms_norm_reference(x, layer.input_norm, config.rms_norm_eps)
    qkv = h @ layer.qkv.T
    cos, sin = rope_tables(d, config.rope_theta, torch.arange(seq))
    q = apply_rope(qkv[:, :hq * d].view(seq, hq, d).transpose(0, 1), cos, sin)
    k = apply_rope(qkv[:, hq * d:(hq + hkv) * d].view(seq, hkv, d).transpose(0, 1), cos, sin)
    v = qkv[:, (hq + hkv) * d:].view(seq, hkv, d).transpose(0, 1)
    # Causal attention of the last position, as decoder_forward computes it.
    kk = k.repeat_interleave(2, dim=0)
    vv = v.repeat_interleave(2, dim=0)
    last = torch.softmax((q[:, -1:] @ kk.transpose(-1, -2)) * d ** -0.5, dim=-1) @ vv
    # The same keys/values in 4-token pages through a permuted table.
    pages = [2, 0, 1]
    key_cache = torch.zeros(3, 4, hkv, d)
    value_cache = torch.zeros(3, 4, hkv, d)
    for t in range(seq):
        key_cache[pages[t // 4], t % 4] = k[:, t]
        value_cache[pages[t // 4], t % 4] = v[:, t]
    decoded = paged_gqa_decode_reference(q[:, -1][None], key_cache, value_cache,
                                         torch.tensor([pages], dtype=torch.int32),
                                         torch.tensor([seq], dtype=torch.int32))
    torch.testing.assert_close(decoded[0], last[:, 0], rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------------------
# The fused decode RoPE + append oracle (rope_kv_append_reference).
# ---------------------------------------------------------------------------
def pin_rope_kv_append(fn) -> None:
    """Closed forms: position 0 is the identity; a unit vector e_0 at
    position p turns into (cos p, sin p) on the pair (0, D/2) and e_{D/2}
    into (-sin p, cos p); every pair keeps its norm; masked lanes leave the
    cache untouched; values are copied bit for bit."""

    hq, hkv, d, half = 4, 2, 8, 4
    generator = torch.Generator().manual_seed(11)
    cos, sin = rope_tables(d, 10000.0, torch.arange(16))
    qkv = torch.randn(3, (hq + 2 * hkv) * d, generator=generator)
    qkv[2, :d] = 0.0
    qkv[2, 0] = 1.0                                  # q head 0 of lane 2 = e_0
    qkv[2, d:2 * d] = 0.0
    qkv[2, d + half] = 1.0                           # q head 1 of lane 2 = e_{D/2}
    qkv[2, hq * d:(hq + 1) * d] = 0.0
    qkv[2, hq * d] = 1.0                             # k head 0 of lane 2 = e_0
    positions = torch.tensor([0, 5, 11])
    key_cache = torch.randn(5, 4, hkv, d, generator=generator)
    value_cache = torch.randn(5, 4, hkv, d, generator=generator)
    pages = torch.tensor([3, 0, 4], dtype=torch.int32)
    offsets = torch.tensor([1, 3, 0], dtype=torch.int32)
    active = torch.tensor([1, 0, 1], dtype=torch.int32)
    q, keys, values = fn(qkv, positions, cos, sin, key_cache, value_cache, pages, offsets, active,
                         hq)
    rows = qkv.view(3, hq + 2 * hkv, d)
    assert torch.equal(q[0], rows[0, :hq]), "position 0 is not the identity on q"
    assert torch.equal(keys[3, 1], rows[0, hq:hq + hkv]), "position 0 is not the identity on k"
    for got, want in ((q[2, 0, 0], math.cos(11)), (q[2, 0, half], math.sin(11)),
                      (q[2, 1, 0], -math.sin(11)), (q[2, 1, half], math.cos(11)),
                      (keys[4, 0, 0, 0], math.cos(11)), (keys[4, 0, 0, half], math.sin(11))):
        assert math.isclose(float(got), want, abs_tol=1e-6), (float(got), want)
    pair_in = rows[:, :hq].reshape(3, hq, 2, half).pow(2).sum(2)
    pair_out = q.reshape(3, hq, 2, half).pow(2).sum(2)
    assert torch.allclose(pair_in, pair_out, atol=1e-5), "rotation changed a pair's norm"
    assert torch.equal(keys[0, 3], key_cache[0, 3]) and torch.equal(values[0, 3], value_cache[0, 3])
    for lane, (page, offset) in ((0, (3, 1)), (2, (4, 0))):
        assert torch.equal(values[page, offset], rows[lane, hq + hkv:])
    untouched = torch.ones(5, 4, dtype=torch.bool)
    untouched[3, 1] = untouched[4, 0] = False
    assert torch.equal(keys[untouched], key_cache[untouched])


def test_rope_kv_append_oracle_pins() -> None:
    pin_rope_kv_append(rope_kv_append_reference)


def test_rope_kv_append_pins_reject_planted_mistakes() -> None:
    def negated_sin(qkv, pos, cos, sin, *rest):
        return rope_kv_append_reference(qkv, pos, cos, -sin, *rest)

    def position_off_by_one(qkv, pos, cos, sin, *rest):
        return rope_kv_append_reference(qkv, pos + 1, cos, sin, *rest)

    def key_not_rotated(qkv, pos, cos, sin, *rest):
        return rope_kv_append_reference(qkv, torch.zeros_like(pos), cos, sin, *rest)

    for mutant in (negated_sin, position_off_by_one, key_not_rotated):
        with pytest.raises(AssertionError):
            pin_rope_kv_append(mutant)


def test_incremental_decode_step_equals_the_full_prefix_forward() -> None:
    """decode_step_reference fed one token at a time (two rows of different
    lengths) reproduces decoder_forward's logits at every position."""

    config = tiny_config()
    weights = DecoderWeights.random(config, seed=7, dtype=torch.float32, device="cpu")
    for layer in weights.layers:
        layer.input_norm.uniform_(0.5, 1.5)
    sequences = [[3, 17, 42, 0, 9, 33, 8], [5, 5, 1, 49]]
    capacity = 8
    keys = [torch.zeros(2, capacity, config.num_key_value_heads, config.head_dim)
            for _ in weights.layers]
    values = [torch.zeros_like(k) for k in keys]
    expected = [decoder_forward(weights, torch.tensor(s)) for s in sequences]
    for step in range(len(sequences[0])):
        rows = [b for b, s in enumerate(sequences) if step < len(s)]
        # Rows that have finished keep decoding a pad token at a later slot.
        tokens = torch.tensor([sequences[b][step] if step < len(sequences[b]) else 0
                               for b in range(2)])
        positions = torch.tensor([step, min(step, capacity - 1)])
        logits = decode_step_reference(weights, keys, values, tokens, positions)
        for b in rows:
            torch.testing.assert_close(logits[b], expected[b][step], rtol=1e-4, atol=1e-5)
