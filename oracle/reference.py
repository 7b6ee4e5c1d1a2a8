"""CPU oracle of the decode hot path.  TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker: the product
(``tensorforge_amd``) never imports it and has no CPU fallback.

Each function restates, from scratch, the algorithm of the reference file
and lines it cites (Kakarottoooo/TensorForge).  Floating-point work is done
in fp32 with torch on the CPU, as the reference oracle does; the KV writes
are byte scatters in numpy on the raw bit patterns, so they are exact for
every dtype.

Pinning (tests/test_oracle.py):
  paged_gqa_decode_reference   the reference's own known-answer case
                               (tests/test_decode_attention.py:9-29), an
                               independent library routine
                               (F.scaled_dot_product_attention, enable_gqa),
                               pure-Python brute force, closed forms (zero keys
                               -> mean of values; one dominant key -> its
                               value), page-permutation invariance
  paged_gqa_decode_split_reference  equality with the one-pass oracle
  rms_norm_reference           F.rms_norm; constant-row closed form
  residual_rms_norm_reference  torch addition (bit-exact) + rms_norm pins
  residual_rms_norm_fused_reference  fp64 recomputation of the same formula
  swiglu_reference             F.silu; per-element math.exp closed form
  swiglu_fused_reference       fp64 recomputation
  paged_kv_write_*_reference   the arange known answer of
                               tests/test_paged_cache.py:11-37, dense
                               recomputation by materialisation order
  rope_kv_append_reference     (tests/test_oracle_model.py) position-0
                               identity, unit vectors turning into
                               (cos p, sin p) / (-sin p, cos p), per-pair norm
                               preservation, masked lanes and untouched rows
                               bit-identical, values copied bit for bit
Mutation tests plant a wrong GQA map, a dropped scale and a reversed page
order in these functions (and a negated sine, an off-by-one position and an
unrotated key in the RoPE append) and check that the pins above reject them.
"""

from __future__ import annotations

import math

import numpy as np
import torch
from torch import Tensor
from torch.nn import functional as F

LOG2E = 1.0 / math.log(2.0)


# ---------------------------------------------------------------------------
# RMSNorm / residual RMSNorm / SwiGLU  (reference: kernels/reference.py:10-43)
# ---------------------------------------------------------------------------
def rms_norm_reference(inputs: Tensor, weight: Tensor, eps: float) -> Tensor:
    """fp32 mean of squares, rsqrt, scale by weight, one rounding.

    Follows kernels/reference.py:10-15.
    """

    x = inputs.detach().cpu().float()
    inv = torch.rsqrt(x.square().mean(dim=-1, keepdim=True) + eps)
    return (x * inv * weight.detach().cpu().float()).to(inputs.dtype)


def residual_rms_norm_reference(
    inputs: Tensor, residual: Tensor, weight: Tensor, eps: float
) -> tuple[Tensor, Tensor]:
    """Sum in storage dtype, then RMSNorm of the rounded sum.

    Follows kernels/reference.py:24-30.
    """

    summed = inputs.detach().cpu() + residual.detach().cpu()
    return summed, rms_norm_reference(summed, weight, eps)


def residual_rms_norm_fused_reference(
    inputs: Tensor, residual: Tensor, weight: Tensor, eps: float
) -> tuple[Tensor, Tensor]:
    """The reference *kernel's* semantics: the norm uses the fp32 sum.

    Follows kernels/triton_ops.py:68-97 (store rounded sum :89, normalise the
    fp32 sum :91-97).
    """

    s = inputs.detach().cpu().float() + residual.detach().cpu().float()
    inv = torch.rsqrt(s.square().mean(dim=-1, keepdim=True) + eps)
    norm = s * inv * weight.detach().cpu().float()
    return s.to(inputs.dtype), norm.to(inputs.dtype)


def swiglu_reference(gate: Tensor, up: Tensor) -> Tensor:
    """silu(gate) * up in the storage dtype (two roundings).

    Follows kernels/reference.py:40-43.
    """

    return F.silu(gate.detach().cpu()) * up.detach().cpu()


def swiglu_fused_reference(gate: Tensor, up: Tensor) -> Tensor:
    """g * sigmoid(g) * u in fp32, one rounding (kernels/triton_ops.py:106-122)."""

    g = gate.detach().cpu().float()
    return (g * torch.sigmoid(g) * up.detach().cpu().float()).to(gate.dtype)


# ---------------------------------------------------------------------------
# Paged GQA decode attention  (reference: kernels/reference.py:46-93)
# ---------------------------------------------------------------------------
def _check_attention_shapes(query: Tensor, key_cache: Tensor, value_cache: Tensor,
                            block_tables: Tensor, context_lengths: Tensor) -> None:
    if query.ndim != 3:
        raise ValueError("query must have shape [batch, query_heads, head_dim]")
    if key_cache.ndim != 4 or value_cache.shape != key_cache.shape:
        raise ValueError("key/value cache must share [blocks, block_size, kv_heads, head_dim]")
    batch, query_heads, head_dim = query.shape
    _, _, kv_heads, cache_head_dim = key_cache.shape
    if head_dim != cache_head_dim or query_heads % kv_heads != 0:
        raise ValueError("query/cache head dimensions do not form valid GQA groups")
    if block_tables.ndim != 2 or block_tables.shape[0] != batch:
        raise ValueError("block_tables must have one row per query")
    if tuple(context_lengths.shape) != (batch,):
        raise ValueError("context_lengths must have one value per query")


def gather_sequence(key_cache: Tensor, value_cache: Tensor, table_row: list[int],
                    context_length: int) -> tuple[Tensor, Tensor]:
    """Logical-order K/V rows [ctx, kv_heads, head_dim] of one sequence.

    Page ``table_row[i]`` holds logical tokens [i*page, (i+1)*page)
    (kernels/reference.py:76-87).
    """

    block_size = key_cache.shape[1]
    logical_blocks = (context_length + block_size - 1) // block_size
    if logical_blocks > len(table_row):
        raise ValueError("context length exceeds block table capacity")
    keys, values = [], []
    for logical in range(logical_blocks):
        physical = table_row[logical]
        if not 0 <= physical < key_cache.shape[0]:
            raise ValueError("block table contains an invalid physical block")
        valid = min(block_size, context_length - logical * block_size)
        keys.append(key_cache[physical, :valid])
        values.append(value_cache[physical, :valid])
    return torch.cat(keys, dim=0), torch.cat(values, dim=0)


def paged_gqa_decode_reference(
    query: Tensor,
    key_cache: Tensor,
    value_cache: Tensor,
    block_tables: Tensor,
    context_lengths: Tensor,
    scale: float | None = None,
) -> Tensor:
    """softmax(scale * q . K^T) V per row over its logical tokens, fp32.

    Query head h reads KV head h // (query_heads // kv_heads)
    (kernels/reference.py:68-93).  Raises on non-positive lengths like the
    reference; callers exclude zero-length rows.
    """

    query = query.detach().cpu()
    key_cache = key_cache.detach().cpu()
    value_cache = value_cache.detach().cpu()
    tables = block_tables.detach().cpu().tolist()
    lengths = context_lengths.detach().cpu().tolist()
    _check_attention_shapes(query, key_cache, value_cache, block_tables, context_lengths)
    batch, query_heads, head_dim = query.shape
    kv_heads = key_cache.shape[2]
    group = query_heads // kv_heads
    attention_scale = head_dim**-0.5 if scale is None else scale
    kv_index = torch.arange(query_heads) // group
    outputs = []
    for b in range(batch):
        ctx = int(lengths[b])
        if ctx <= 0:
            raise ValueError("context lengths must be positive")
        keys, values = gather_sequence(key_cache, value_cache, tables[b], ctx)
        keys = keys[:, kv_index].float()  # [ctx, Hq, D]
        values = values[:, kv_index].float()
        scores = torch.einsum("hd,thd->ht", query[b].float(), keys) * attention_scale
        probs = torch.softmax(scores, dim=-1)
        outputs.append(torch.einsum("ht,thd->hd", probs, values))
    return torch.stack(outputs).to(query.dtype)


def paged_gqa_decode_split_reference(
    query: Tensor,
    key_cache: Tensor,
    value_cache: Tensor,
    block_tables: Tensor,
    context_lengths: Tensor,
    split_size: int,
    scale: float | None = None,
) -> Tensor:
    """Two-stage split-KV restatement: per-split (max, sum, acc), then LSE merge.

    Follows triton_attention.py:173-266 (partials over [s*S, (s+1)*S)) and
    :268-316 (M = max m_s; out = sum acc_s e^{m_s-M} / sum l_s e^{m_s-M}),
    with empty splits contributing nothing.
    """

    query = query.detach().cpu()
    key_cache = key_cache.detach().cpu()
    value_cache = value_cache.detach().cpu()
    tables = block_tables.detach().cpu().tolist()
    lengths = context_lengths.detach().cpu().tolist()
    _check_attention_shapes(query, key_cache, value_cache, block_tables, context_lengths)
    batch, query_heads, head_dim = query.shape
    kv_heads = key_cache.shape[2]
    group = query_heads // kv_heads
    attention_scale = head_dim**-0.5 if scale is None else scale
    kv_index = torch.arange(query_heads) // group
    outputs = []
    for b in range(batch):
        ctx = int(lengths[b])
        if ctx <= 0:
            raise ValueError("context lengths must be positive")
        keys, values = gather_sequence(key_cache, value_cache, tables[b], ctx)
        keys = keys[:, kv_index].float()
        values = values[:, kv_index].float()
        q = query[b].float()
        maxima, sums, accs = [], [], []
        for start in range(0, ctx, split_size):
            k = keys[start:start + split_size]
            v = values[start:start + split_size]
            s = torch.einsum("hd,thd->ht", q, k) * attention_scale
            m = s.max(dim=-1).values
            p = torch.exp(s - m[:, None])
            maxima.append(m)
            sums.append(p.sum(dim=-1))
            accs.append(torch.einsum("ht,thd->hd", p, v))
        m_all = torch.stack(maxima)  # [splits, Hq]
        g_max = m_all.max(dim=0).values
        corr = torch.exp(m_all - g_max[None, :])
        den = (torch.stack(sums) * corr).sum(dim=0)
        num = (torch.stack(accs) * corr[:, :, None]).sum(dim=0)
        outputs.append(num / den[:, None])
    return torch.stack(outputs).to(query.dtype)


# ---------------------------------------------------------------------------
# Paged KV writes  (reference: kernels/triton_cache.py:23-63, cache/paged.py:221-235)
# ---------------------------------------------------------------------------
def _bits(tensor: Tensor) -> np.ndarray:
    """Raw bit patterns of a CPU tensor as an integer numpy array (a view)."""

    width = tensor.element_size()
    view_dtype = {2: torch.int16, 4: torch.int32, 8: torch.int64}[width]
    return tensor.view(view_dtype).numpy()


def paged_kv_write_token_reference(
    keys: Tensor,
    values: Tensor,
    key_cache: Tensor,
    value_cache: Tensor,
    physical_blocks: Tensor,
    block_offsets: Tensor,
    active_mask: Tensor,
) -> tuple[Tensor, Tensor]:
    """Return copies of the caches after the masked one-token-per-lane write.

    Lane b with active_mask[b] != 0 copies keys[b]/values[b] (all kv heads)
    to cache[physical_blocks[b], block_offsets[b]]; other lanes write
    nothing (triton_cache.py:41-63).
    """

    k_out = key_cache.detach().cpu().clone()
    v_out = value_cache.detach().cpu().clone()
    kb, vb = _bits(k_out), _bits(v_out)
    ks, vs = _bits(keys.detach().cpu().contiguous()), _bits(values.detach().cpu().contiguous())
    phys = physical_blocks.detach().cpu().numpy()
    offs = block_offsets.detach().cpu().numpy()
    mask = active_mask.detach().cpu().numpy()
    for lane in range(ks.shape[0]):
        if mask[lane] != 0:
            kb[phys[lane], offs[lane]] = ks[lane]
            vb[phys[lane], offs[lane]] = vs[lane]
    return k_out, v_out


def write_layer_slots(blocks: list[int], start_position: int, token_count: int,
                      block_size: int) -> np.ndarray:
    """Slot of each appended token: blocks[p // page] * page + p % page.

    The position -> (logical block, offset) -> physical mapping of
    cache/paged.py:221-233.
    """

    positions = np.arange(start_position, start_position + token_count, dtype=np.int64)
    physical = np.asarray(blocks, dtype=np.int64)[positions // block_size]
    return physical * block_size + positions % block_size


def paged_kv_write_slots_reference(
    keys: Tensor,
    values: Tensor,
    key_cache: Tensor,
    value_cache: Tensor,
    slot_mapping: Tensor,
) -> tuple[Tensor, Tensor]:
    """Return copies of the caches after scattering row t to token slot
    slot_mapping[t] (negative slots skipped); the index_put of
    cache/paged.py:234-235 expressed with flat token slots.
    """

    k_out = key_cache.detach().cpu().clone()
    v_out = value_cache.detach().cpu().clone()
    rows = k_out.shape[0] * k_out.shape[1]
    kb = _bits(k_out).reshape(rows, -1)
    vb = _bits(v_out).reshape(rows, -1)
    ks = _bits(keys.detach().cpu().contiguous()).reshape(keys.shape[0], -1)
    vs = _bits(values.detach().cpu().contiguous()).reshape(values.shape[0], -1)
    slots = slot_mapping.detach().cpu().numpy()
    for t, slot in enumerate(slots):
        if 0 <= slot < rows:
            kb[slot] = ks[t]
            vb[slot] = vs[t]
    return k_out, v_out



def rope_kv_append_reference(
    qkv: Tensor,
    positions: Tensor,
    cos_table: Tensor,
    sin_table: Tensor,
    key_cache: Tensor,
    value_cache: Tensor,
    physical_blocks: Tensor,
    block_offsets: Tensor,
    active_mask: Tensor,
    query_heads: int,
) -> tuple[Tensor, Tensor, Tensor]:
    """(rotated query [B, Hq, D] in fp32, key cache, value cache) after the
    fused decode-step RoPE and append.

    RoPE with the half-split rotation (model/layers.py:46-69), evaluated in
    fp32 from the storage-dtype cos/sin rows of each lane's position; the
    rotated key is rounded once to the cache dtype and, with the value
    (copied bit for bit), written by the masked one-token write
    (paged_kv_write_token_reference).
    """

    num_blocks, block_size, kv_heads, head_dim = key_cache.shape
    half = head_dim // 2
    rows = qkv.detach().cpu().float()
    pos = positions.detach().cpu().long()
    cos = cos_table.detach().cpu().float()[pos][:, None, :]
    sin = sin_table.detach().cpu().float()[pos][:, None, :]

    def rotate(x: Tensor) -> Tensor:
        rotated = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
        return x * cos + rotated * sin

    batch = rows.shape[0]
    q = rotate(rows[:, : query_heads * head_dim].reshape(batch, query_heads, head_dim))
    k = rotate(rows[:, query_heads * head_dim:(query_heads + kv_heads) * head_dim]
               .reshape(batch, kv_heads, head_dim))
    v = qkv.detach().cpu()[:, (query_heads + kv_heads) * head_dim:
                           (query_heads + 2 * kv_heads) * head_dim]
    keys = k.to(key_cache.dtype)
    values = v.reshape(batch, kv_heads, head_dim).contiguous()
    key_out, value_out = paged_kv_write_token_reference(
        keys, values, key_cache, value_cache, physical_blocks, block_offsets, active_mask)
    return q, key_out, value_out
