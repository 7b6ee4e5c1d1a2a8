"""Pins of the decoder oracle (oracle/model.py), on the CPU."""

from __future__ import annotations

import math

import torch

from oracle.model import apply_rope, decoder_forward, rope_tables, rotate_half
from oracle.reference import paged_gqa_decode_reference, rms_norm_reference
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
