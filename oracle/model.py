"""CPU oracle of the Llama-style decoder the decode path serves.  TEST
INFRASTRUCTURE ONLY (same import rule as oracle/reference.py).

A full-prefix fp32 forward restating tensorforge/model/layers.py and
model/llama.py: embedding, pre-norm blocks (RMSNorm :14-30, grouped-query
causal attention with RoPE :33-143, SwiGLU MLP :146-158, residuals
:161-171), final RMSNorm and the LM head.  Weights come from the same
container the GPU path uses (tensorforge_amd.decode.DecoderWeights), read on
the CPU in fp32 (or, as a checker of long runs, on the GPU in fp32 or in
the model's own precision).

Pinning (tests/test_oracle_model.py): RoPE against its closed forms
(identity at position 0, norm preservation, dot products depending only on
the position difference, a hand-rotated pair); the last position's
attention against paged_gqa_decode_reference over the same keys and values;
the whole block against a pure-Python brute-force block on a tiny model;
the incremental decode step (decode_step_reference, the CPU baseline of the
decode-step benchmark) against decoder_forward, token by token.
"""

from __future__ import annotations

import torch
from torch import Tensor

from oracle.reference import rms_norm_reference


def rope_tables(head_dim: int, theta: float, positions: Tensor) -> tuple[Tensor, Tensor]:
    """cos/sin [len, head_dim] in fp32: angle(p, i) = p * theta^(-2i/D), the
    half-dimension table repeated twice, computed as the reference computes
    it (layers.py:33-46): inv_freq in fp32, the position/frequency outer
    product in fp32, cos and sin of those fp32 angles."""

    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    angles = torch.outer(positions.float(), inv_freq)
    angles = torch.cat((angles, angles), dim=-1)
    return angles.cos(), angles.sin()


def rotate_half(x: Tensor) -> Tensor:
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def apply_rope(x: Tensor, cos: Tensor, sin: Tensor) -> Tensor:
    """x [..., seq, D] with cos/sin [seq, D] (layers.py:49-60)."""

    return x * cos + rotate_half(x) * sin


def _rms_norm(x: Tensor, weight: Tensor, eps: float) -> Tensor:
    """rms_norm_reference's formula (fp32 mean of squares, rsqrt, scale by
    weight, one rounding to x's dtype) on x's own device."""

    xf = x.float()
    inv = torch.rsqrt(xf.square().mean(dim=-1, keepdim=True) + eps)
    return (xf * inv * weight.float()).to(x.dtype)


def decoder_forward(weights, tokens: Tensor, *, device: torch.device | str = "cpu",
                    dtype: torch.dtype = torch.float32) -> Tensor:
    """Logits [seq, vocab] of a full causal forward over `tokens` [seq].

    By default in fp32 on the CPU.  ``device`` runs the same math on another
    device (a checker for long sequences); ``dtype`` runs it in another
    precision (fp16 / bf16: every operand and every intermediate rounded to
    it, as a same-precision restatement of the model).  Logits are returned
    in fp32 on the CPU."""

    config = weights.config
    device = torch.device(device)
    f32 = lambda t: t.detach().to(device=device, dtype=dtype)  # noqa: E731
    hq, hkv, d = config.num_attention_heads, config.num_key_value_heads, config.head_dim
    group = hq // hkv
    seq = tokens.shape[0]
    x = f32(weights.embedding)[tokens.to(device)]
    cos, sin = rope_tables(d, config.rope_theta, torch.arange(seq))
    cos, sin = cos.to(device=device, dtype=dtype), sin.to(device=device, dtype=dtype)
    causal = torch.ones(seq, seq, dtype=torch.bool, device=device).triu(1)
    for layer in weights.layers:
        h = _rms_norm(x, f32(layer.input_norm), config.rms_norm_eps)
        qkv = h @ f32(layer.qkv).T
        q = qkv[:, : hq * d].view(seq, hq, d).transpose(0, 1)
        k = qkv[:, hq * d: (hq + hkv) * d].view(seq, hkv, d).transpose(0, 1)
        v = qkv[:, (hq + hkv) * d:].view(seq, hkv, d).transpose(0, 1)
        q, k = apply_rope(q, cos, sin), apply_rope(k, cos, sin)
        k = k.repeat_interleave(group, dim=0)
        v = v.repeat_interleave(group, dim=0)
        scores = (q @ k.transpose(-1, -2).contiguous()) * d**-0.5
        scores = scores.masked_fill(causal, float("-inf"))
        context = torch.softmax(scores.float(), dim=-1).to(dtype) @ v  # [hq, seq, d]
        x = x + context.transpose(0, 1).reshape(seq, hq * d) @ f32(layer.o_proj).T
        h = _rms_norm(x, f32(layer.post_norm), config.rms_norm_eps)
        gate = h @ f32(layer.gate).T
        up = h @ f32(layer.up).T
        x = x + (torch.nn.functional.silu(gate) * up) @ f32(layer.down).T
    h = _rms_norm(x, f32(weights.final_norm), config.rms_norm_eps)
    return (h @ f32(weights.lm_head).T).float().cpu()


def decode_step_reference(weights, keys: list[Tensor], values: list[Tensor], tokens: Tensor,
                          positions: Tensor) -> Tensor:
    """One incremental decode step on the CPU in fp32 (the reference's eager
    decode path, runtime/paged_decode.py, with dense per-row caches instead of
    pages): logits [B, vocab] for `tokens` [B] at `positions` [B].

    ``keys[layer]`` / ``values[layer]`` are fp32 [B, capacity, Hkv, D]
    buffers; row b's first positions[b] slots hold its earlier tokens, and
    the step writes the new token's k/v at slot positions[b] before
    attending over slots 0..positions[b].  Weights are read as given (call
    with fp32 CPU copies).
    """

    config = weights.config
    hq, hkv, d = config.num_attention_heads, config.num_key_value_heads, config.head_dim
    group = hq // hkv
    batch = tokens.shape[0]
    x = weights.embedding[tokens]
    cos, sin = rope_tables(d, config.rope_theta, positions)
    rows = torch.arange(batch)
    for index, layer in enumerate(weights.layers):
        h = rms_norm_reference(x, layer.input_norm, config.rms_norm_eps)
        qkv = h @ layer.qkv.T
        q = apply_rope(qkv[:, : hq * d].view(batch, hq, d), cos[:, None], sin[:, None])
        k = apply_rope(qkv[:, hq * d: (hq + hkv) * d].view(batch, hkv, d), cos[:, None],
                       sin[:, None])
        keys[index][rows, positions] = k
        values[index][rows, positions] = qkv[:, (hq + hkv) * d:].view(batch, hkv, d)
        context = torch.empty(batch, hq, d)
        for b in range(batch):
            n = int(positions[b]) + 1
            kk = keys[index][b, :n].repeat_interleave(group, dim=1).transpose(0, 1)  # [hq, n, d]
            vv = values[index][b, :n].repeat_interleave(group, dim=1).transpose(0, 1)
            scores = (kk @ q[b][:, :, None])[..., 0] * d ** -0.5                     # [hq, n]
            context[b] = (torch.softmax(scores, dim=-1)[:, None, :] @ vv)[:, 0]
        x = x + context.view(batch, hq * d) @ layer.o_proj.T
        h = rms_norm_reference(x, layer.post_norm, config.rms_norm_eps)
        gate = h @ layer.gate.T
        up = h @ layer.up.T
        x = x + (torch.nn.functional.silu(gate) * up) @ layer.down.T
    h = rms_norm_reference(x, weights.final_norm, config.rms_norm_eps)
    logits = h @ weights.lm_head.T
    return logits
