"""Bucketed, HIP-graph-captured batched decode over the paged cache.

The caller of the hot path (reference: runtime/decode_bucket.py:175-666).
One decode step of a Llama-style decoder for up to ``batch_capacity``
sequences runs as ONE captured HIP graph.  Per layer, five launches:

* the fused QKV projection with the input RMSNorm applied to its products
  (the norm gain folded into an executor-held copy of the weight);
* RoPE on q and k, k and v into their pages, and
  ``paged_gqa_decode_attention`` (one pass for wide buckets, split-KV with
  its merge otherwise) -- one fused launch where the MFMA attention kernel
  serves the geometry, else ``rope_paged_kv_append`` then attention;
* the output projection added to the residual stream;
* the fused gate|up projection with the post-attention RMSNorm and SwiGLU;
* the down projection added to the residual stream;

then the final RMSNorm, the LM head and the greedy argmax.  With
``fuse_norms=False`` the norms run as launches of their own
(``residual_rms_norm`` over split-K partials of the o and down
projections).

The gfx950 kernels of this package do the norm, cache and attention work
and the projections (the K-split weight stream for qkv, o, gate|up and
down, the weight stream for the LM head up to 32 rows); only the LM head of
larger buckets is a library GEMM (torch -> hipBLASLt).  Every per-step
input lives in one device "control" slab, filled from one pinned host slab
with one asynchronous copy per step.  So the graph's addresses never
change, and a step needs no host synchronisation beyond reading back the
sampled tokens.

Lanes past the live batch are padded: context length 0, masked cache
write.  Their attention output is zero and their sampled token is ignored.
The model math follows tensorforge/model/layers.py (RMSNorm, RoPE with the
half-split rotation, grouped-query attention, SwiGLU MLP, pre-norm
residuals); weights are random (N(0, 0.02), norms 1), as in the reference's
initialize_weights (layers.py:174-176).
"""

from __future__ import annotations

import time
from collections.abc import Callable
from contextlib import suppress
from dataclasses import asdict, dataclass, field

import numpy as np
import torch
from torch import Tensor
from torch.nn import functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

from tensorforge_amd import _native
from tensorforge_amd.batch import BatchExecutionResult
from tensorforge_amd.cache import AppendReservation, PagedKVCache
from tensorforge_amd.kernels import (
    argmax_rows,
    embedding_rms_norm,
    PagedAttentionWorkspace,
    linear_kstream,
    linear_rows,
    linear_rows_supported,
    linear_stream,
    linear_swiglu,
    paged_gqa_decode_attention,
    residual_rms_norm,
    rms_norm,
    rope_paged_kv_append,
    swiglu_gate_up,
)
from tensorforge_amd.kernels.attention import (
    paged_gqa_decode_attention_rope_append,
    set_attention_split_size,
)
from tensorforge_amd.kernels.linear import (
    default_splits,
    fold_norm_gain,
    linear_partials_supported,
)
from tensorforge_amd.kernels.ops import residual_rms_norm_partials
from tensorforge_amd.kernels.prefill import (
    prefill_attention,
    prefill_attention_supported,
    prefill_tiles,
)


@dataclass(frozen=True, slots=True)
class DecoderConfig:
    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    rms_norm_eps: float = 1e-5
    rope_theta: float = 10000.0
    max_position_embeddings: int = 4096

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads


def tinyllama_config() -> DecoderConfig:
    """TinyLlama-1.1B geometry."""

    return DecoderConfig(vocab_size=32000, hidden_size=2048, intermediate_size=5632,
                         num_hidden_layers=22, num_attention_heads=32, num_key_value_heads=4)


def small_config() -> DecoderConfig:
    """4 layers, d_model 256, 8/2 heads (head_dim 32), FFN 768,
    vocab 1024."""

    return DecoderConfig(vocab_size=1024, hidden_size=256, intermediate_size=768,
                         num_hidden_layers=4, num_attention_heads=8, num_key_value_heads=2,
                         max_position_embeddings=512)


@dataclass(slots=True)
class LayerWeights:
    input_norm: Tensor  # [H]
    qkv: Tensor         # [(Hq + 2 Hkv) D, H]: q, k, v projections stacked
    o_proj: Tensor      # [H, Hq D]
    post_norm: Tensor   # [H]
    gate_up: Tensor     # [2F, H]: gate and up projections stacked (one GEMM)
    down: Tensor        # [H, F]

    @property
    def gate(self) -> Tensor:
        return self.gate_up[: self.gate_up.shape[0] // 2]

    @property
    def up(self) -> Tensor:
        return self.gate_up[self.gate_up.shape[0] // 2:]


@dataclass(slots=True)
class DecoderWeights:
    config: DecoderConfig
    embedding: Tensor   # [V, H]
    layers: list[LayerWeights]
    final_norm: Tensor  # [H]
    lm_head: Tensor     # [V, H]
    rope_cos: Tensor    # [max_position, D] in the model dtype
    rope_sin: Tensor

    @classmethod
    def random(cls, config: DecoderConfig, *, seed: int = 0, dtype: torch.dtype = torch.bfloat16,
               device: torch.device | str = "cuda") -> DecoderWeights:
        device = torch.device(device)
        generator = torch.Generator(device=device).manual_seed(seed)

        def normal(*shape: int) -> Tensor:
            return (torch.randn(*shape, generator=generator, device=device,
                                dtype=torch.float32) * 0.02).to(dtype)

        def ones(size: int) -> Tensor:
            return torch.ones(size, device=device, dtype=dtype)

        h, f, d = config.hidden_size, config.intermediate_size, config.head_dim
        hq, hkv = config.num_attention_heads, config.num_key_value_heads
        layers = [
            LayerWeights(input_norm=ones(h), qkv=normal((hq + 2 * hkv) * d, h),
                         o_proj=normal(h, hq * d), post_norm=ones(h), gate_up=normal(2 * f, h),
                         down=normal(h, f))
            for _ in range(config.num_hidden_layers)
        ]
        # RoPE tables as the reference builds them (layers.py:38-46): inv_freq
        # and the position/frequency outer product in fp32, cos/sin of those
        # fp32 angles rounded once to the model dtype.
        inv_freq = 1.0 / (config.rope_theta ** (
            torch.arange(0, d, 2, dtype=torch.float32) / d))
        angles = torch.outer(torch.arange(config.max_position_embeddings, dtype=torch.float32),
                             inv_freq)
        angles = torch.cat((angles, angles), dim=-1)
        return cls(config=config, embedding=normal(config.vocab_size, h), layers=layers,
                   final_norm=ones(h), lm_head=normal(config.vocab_size, h),
                   rope_cos=angles.cos().to(dtype).to(device),
                   rope_sin=angles.sin().to(dtype).to(device))


def _project(x: Tensor, weight: Tensor, output: Tensor | None = None) -> Tensor:
    """x @ weight.T for a decode step (measured on MI355X at the TinyLlama
    shapes).  Weights of >= 16384 rows (the LM head) up to 32 rows and of
    >= 8192 rows (the stacked gate|up) up to 16 rows go through the
    LDS-staged weight stream (linear_stream: 24.6-25.0 us against 30.4-30.7
    for hipBLASLt at 32000 x 2048; 12.6-12.8 us against 12.5-14.7 at
    11264 x 2048).  Narrower weights with K >= 1024 (the stacked q/k/v)
    take the K-split weight stream (linear_kstream: 4.7-7.9 us at 1..64 rows
    against 5.7-12.9 for linear_rows and 11.2-11.9 for hipBLASLt at
    2560 x 2048).  Other weights up to 16 rows use the K-split MFMA kernel
    (linear_rows) when small (<= 8M elements), where the library GEMM
    launches too few workgroups; otherwise hipBLASLt."""

    rows = x.shape[0]
    if (linear_rows_supported(x, weight)
            and ((weight.shape[0] >= 16384 and rows <= 32)
                 or (weight.shape[0] >= 8192 and rows <= 16))):
        return linear_stream(x, weight, output=output)
    if linear_rows_supported(x, weight) and weight.shape[0] < 8192 and weight.shape[1] >= 1024:
        return linear_kstream(x, weight, output=output)
    rows_kernel = (rows <= 16 and linear_rows_supported(x, weight)
                   and (weight.numel() <= 8 * 1024 * 1024 or weight.shape[0] >= 16384
                        or (rows <= 8 and weight.shape[0] >= 8192)))
    if rows_kernel:
        return linear_rows(x, weight, output=output)
    if output is None:
        return F.linear(x, weight)
    return torch.matmul(x, weight.t(), out=output)


class DecodeGraphBucket:
    """Static buffers and one captured HIP graph for a decode step of up to
    ``batch_capacity`` sequences whose contexts stay within
    ``context_capacity`` tokens (reference: _DecodeBucket,
    decode_bucket.py:175-528).

    Control state per lane: the input token (taken either from the host or,
    on the device, from ``token_state[source_lane]`` -- the token the previous
    step sampled in that lane, so a running request never round-trips its
    token through the host), the position, the block-table row, the context
    length, the append page/offset and the active flag.  The host keeps a
    master copy and rewrites only what changed: a lane that decodes the same
    request as last time gets just its newly appended pages.  Each step
    copies the master into one of two pinned byte slabs (the int64 rows and
    the int32 segments back to back) and from there, with one asynchronous
    copy, to the device; a slab is reused only after its previous copy has
    completed.
    """

    def __init__(self, weights: DecoderWeights, cache: PagedKVCache, *, batch_capacity: int,
                 context_capacity: int, token_state: Tensor | None = None, graph: bool = True,
                 metrics: _MutableMetrics | None = None,
                 folded: Callable[[], list[tuple[Tensor, Tensor]]] | None = None) -> None:
        config = weights.config
        self.weights = weights
        self.cache = cache
        self.batch_capacity = batch_capacity
        self.context_capacity = context_capacity
        # graph=False runs every step eagerly (the executor's fallback for
        # steps no bucket holds); the step's work is the same.
        self.graph = graph
        self._metrics = metrics
        device = cache.config.device
        dtype = cache.config.dtype
        width = cache.config.max_blocks_per_sequence
        b = batch_capacity
        self.device = device
        # Long rows: host token, position, source lane.  Int32 segments: block
        # tables [b, width], context lengths, append pages, page offsets,
        # active flags.
        self._ctl_long = np.zeros((3, b), dtype=np.int64)
        self._ctl_int = np.zeros(b * (width + 4), dtype=np.int32)
        self._ctl_int[:b * width] = -1
        cuts = [b * width, b * (width + 1), b * (width + 2), b * (width + 3)]
        self._host_views = (self._ctl_int[:cuts[0]].reshape(b, width), self._ctl_int[cuts[0]:cuts[1]],
                            self._ctl_int[cuts[1]:cuts[2]], self._ctl_int[cuts[2]:cuts[3]],
                            self._ctl_int[cuts[3]:])
        # One byte slab holds both segments (the int64 rows first), so a step
        # stages its controls with a single host-to-device copy.
        long_bytes = 3 * b * 8
        slab_bytes = long_bytes + self._ctl_int.size * 4
        self._pinned = []
        for _ in range(2):
            slab = torch.zeros(slab_bytes, dtype=torch.uint8, pin_memory=True)
            self._pinned.append((slab, slab.numpy()[:long_bytes].view(np.int64).reshape(3, b),
                                 slab.numpy()[long_bytes:].view(np.int32)))
        self._copied = [torch.cuda.Event(), torch.cuda.Event()]
        self._copy_recorded = [False, False]
        self._flip = 0
        self._slab = torch.zeros(slab_bytes, dtype=torch.uint8, device=device)
        self._long = self._slab[:long_bytes].view(torch.int64).view(3, b)
        self._int = self._slab[long_bytes:].view(torch.int32)
        self.host_tokens = self._long[0]
        self.positions = self._long[1]
        self.source_lanes = self._long[2]
        self.block_tables = self._int[:cuts[0]].view(b, width)
        self.context_lengths = self._int[cuts[0]:cuts[1]]
        self.physical_blocks = self._int[cuts[1]:cuts[2]]
        self.block_offsets = self._int[cuts[2]:cuts[3]]
        self.active_mask = self._int[cuts[3]:]
        self._lane_rows: list[tuple[tuple[int, int], int] | None] = [None] * b
        self._max_position = weights.rope_cos.shape[0]
        if token_state is None:
            token_state = torch.zeros(b, dtype=torch.long, device=device)
        if token_state.numel() < b or token_state.dtype != torch.long:
            raise ValueError("token_state must be an int64 tensor of at least batch_capacity")
        self.token_state = token_state
        hq, hkv, d = config.num_attention_heads, config.num_key_value_heads, config.head_dim
        # Partials for one partition per 128 tokens of the context (twice the
        # reference's sizing), so narrow buckets can take the 128-token
        # partitions of the attention plan.
        self.workspace = PagedAttentionWorkspace.allocate(
            batch_capacity=b, query_heads=hq, head_dim=d, max_context_length=2 * context_capacity,
            device=device)
        self.query = torch.empty((b, hq, d), dtype=dtype, device=device)
        self.attention_output = torch.empty((b, hq, d), dtype=dtype, device=device)
        self.norm_output = torch.empty((b, config.hidden_size), dtype=dtype, device=device)
        self.embedding_output = torch.empty((b, config.hidden_size), dtype=dtype, device=device)
        self.swiglu_output = torch.empty((b, config.intermediate_size), dtype=dtype,
                                         device=device)
        self.logits = torch.empty((b, config.vocab_size), dtype=dtype, device=device)
        self.next_tokens = self.token_state[:b]
        # RoPE, the KV append and attention in one launch where the MFMA
        # attention kernel serves the geometry.
        self.fused_rope = _native.library().tf_paged_gqa_decode_variant(
            _native.dtype_code(dtype), d, hq // hkv, cache.config.block_size,
            0) == _native.TF_ATTENTION_MFMA
        # Output and down projections at up to 64 rows: split-K partials of
        # the LDS-staged weight stream, whose K-slice sum is fused into the
        # residual RMSNorm that consumes them (measured faster than
        # linear_rows and hipBLASLt at 1..64 rows for the TinyLlama o and
        # down shapes: at 64 rows 6.1 / 10.6 us against 10.9 / 18.2 for
        # hipBLASLt; at up to 16 rows only for weights of >= 1M elements --
        # smaller ones make too few 64-column workgroups and stay on
        # linear_rows).  Above 32 rows an output projection with K >= 1024
        # instead takes the K-split weight stream with a rounded output and
        # the plain residual RMSNorm (TinyLlama b64 step 1.559 -> 1.549 ms;
        # at 16-32 rows the partials stay as fast or faster).
        self.split_o = self.split_down = 0
        layer0 = weights.layers[0]
        large = min(layer0.o_proj.numel(), layer0.down.numel()) >= 1024 * 1024
        if (b <= 64 and (b > 16 or large)
                and dtype in (torch.float16, torch.bfloat16)):
            probe_o = torch.empty((b, hq * d), dtype=dtype, device=device)
            probe_d = torch.empty((b, config.intermediate_size), dtype=dtype, device=device)
            if (linear_partials_supported(probe_o, layer0.o_proj)
                    and linear_partials_supported(probe_d, layer0.down)):
                kstream_o = b > 32 and layer0.o_proj.shape[1] >= 1024
                self.split_o = 0 if kstream_o else default_splits(*layer0.o_proj.shape)
                self.split_down = default_splits(*layer0.down.shape)
                self.partials_o = torch.empty((self.split_o, b, config.hidden_size),
                                              dtype=torch.float32, device=device)
                self.partials_down = torch.empty((self.split_down, b, config.hidden_size),
                                                 dtype=torch.float32, device=device)
        # The MLP's gate|up projection with SwiGLU in its epilogue, K split
        # over 16-column workgroups (TinyLlama 11264 x 2048: 11.0-13.9 us at
        # 1..32 rows and 18.2 at 64, against 14.7-16.8 and 18.8 for the best
        # projection + SwiGLU pair).
        probe_h = torch.empty((b, config.hidden_size), dtype=dtype, device=device)
        self.fused_gate_up = linear_rows_supported(probe_h, layer0.gate_up)
        # Norms fused into the projections around them (every weight through
        # the K-split stream): qkv and gate|up scale their products by the
        # RMSNorm of their input rows, with the norm gains folded into
        # copies of their weights (`folded`, shared by the executor's
        # buckets), and o and down add their products to the residual
        # stream -- five launches per layer instead of seven, and no
        # normalised activations written.  The LM head keeps the final norm.
        probe_a = torch.empty((b, hq * d), dtype=dtype, device=device)
        probe_f = torch.empty((b, config.intermediate_size), dtype=dtype, device=device)
        self.fused_norms = (folded is not None and self.fused_gate_up
                            and linear_rows_supported(probe_h, layer0.qkv)
                            and linear_rows_supported(probe_a, layer0.o_proj)
                            and linear_rows_supported(probe_f, layer0.down))
        self._folded = folded if self.fused_norms else None
        if self.fused_norms:
            self.split_o = self.split_down = 0
        self._graph: torch.cuda.CUDAGraph | None = None

    def addresses(self) -> dict[str, int]:
        """Device addresses the captured graph depends on (decode_bucket.py:330-369)."""

        return {name: getattr(self, name).data_ptr() for name in (
            "host_tokens", "positions", "source_lanes", "block_tables", "context_lengths",
            "physical_blocks", "block_offsets", "active_mask", "attention_output",
            "norm_output", "swiglu_output", "logits", "next_tokens")}

    def prepare(self, request_ids: list[str], reservations: dict[str, AppendReservation], *,
                tokens: dict[str, int] | None = None,
                source_lanes: dict[str, int] | None = None) -> None:
        """Stage one step: lane i decodes request_ids[i] at its one-token
        reservation, with input token ``tokens[rid]`` if given, else the
        token the previous step sampled in lane ``source_lanes[rid]``."""

        b = self.batch_capacity
        if len(request_ids) > b:
            raise ValueError("more requests than the bucket's batch capacity")
        tokens = tokens or {}
        source_lanes = source_lanes or {}
        block_size = self.cache.config.block_size
        tables, lengths, pages, offsets, active = self._host_views
        host_tokens, positions, sources = self._ctl_long
        for lane, request_id in enumerate(request_ids):
            reservation = reservations[request_id]
            if reservation.request_id != request_id or reservation.token_count != 1:
                raise ValueError("each lane needs a one-token reservation of its own request")
            page_list, version = self.cache.page_list(request_id)
            start = reservation.start_position
            if start + 1 > self.context_capacity:
                raise ValueError("context exceeds the bucket's context capacity")
            if start >= self._max_position:
                raise ValueError("position exceeds the model's RoPE table")
            logical, offset = divmod(start, block_size)
            if logical >= len(page_list):
                raise RuntimeError("reservation is not backed by a page")
            row = self._lane_rows[lane]
            count = len(page_list)
            if row is None or row[0] != version or row[1] > count:
                tables[lane, :count] = page_list
                tables[lane, count:] = -1
            elif row[1] < count:
                tables[lane, row[1]:count] = page_list[row[1]:]
            self._lane_rows[lane] = (version, count)
            lengths[lane] = start + 1
            pages[lane] = page_list[logical]
            offsets[lane] = offset
            active[lane] = 1
            positions[lane] = start
            if request_id in tokens:
                host_tokens[lane] = tokens[request_id]
                sources[lane] = -1
            else:
                host_tokens[lane] = 0
                sources[lane] = source_lanes[request_id]
        live = len(request_ids)
        lengths[live:] = 0
        pages[live:] = 0
        offsets[live:] = 0
        active[live:] = 0
        positions[live:] = 0
        host_tokens[live:] = 0
        sources[live:] = -1
        self._stage()

    def _stage(self) -> None:
        k = self._flip
        self._flip ^= 1
        if self._copy_recorded[k]:
            self._copied[k].synchronize()  # the slab's previous copy has landed
        slab, host_long, host_int = self._pinned[k]
        np.copyto(host_long, self._ctl_long)
        np.copyto(host_int, self._ctl_int)
        self._slab.copy_(slab, non_blocking=True)
        self._copied[k].record()
        self._copy_recorded[k] = True

    def execute(self) -> Tensor:
        """Run the step (capturing the graph on first use, or eagerly when
        the bucket has no graph); returns the device tensor of greedy next
        tokens, one per lane."""

        metrics = self._metrics
        if not self.graph:
            self._forward()
            if metrics is not None:
                metrics.eager_calls += 1
            return self.next_tokens
        if self._graph is None:
            begin = time.perf_counter()
            stream = torch.cuda.current_stream(self.device)
            # The eager warm-up (library handles and plans) samples into
            # token_state; restore it so the replay reads the previous step's
            # tokens.  Its cache writes equal the replay's.
            saved = self.token_state.clone()
            side = torch.cuda.Stream(self.device)
            side.wait_stream(stream)
            with torch.cuda.stream(side):
                self._forward()
            stream.wait_stream(side)
            self.token_state.copy_(saved)
            torch.cuda.synchronize(self.device)
            warm = time.perf_counter()
            self._graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self._graph):
                self._forward()
            if metrics is not None:
                metrics.capture_count += 1
                metrics.capture_warmup_time_ms += (warm - begin) * 1e3
                metrics.capture_time_ms += (time.perf_counter() - begin) * 1e3
                metrics.graph_misses += 1
        elif metrics is not None:
            metrics.graph_hits += 1
        if metrics is not None:
            metrics.graph_calls += 1
        self._graph.replay()
        return self.next_tokens

    def _forward(self) -> None:
        config = self.weights.config
        hq, hkv, d = config.num_attention_heads, config.num_key_value_heads, config.head_dim
        b = self.batch_capacity
        eps = config.rms_norm_eps
        # The attention plan is chosen per call from the bucket's sizes (one
        # pass for wide buckets, split-KV otherwise), whatever partition size
        # a caller may have fixed globally.
        previous = set_attention_split_size(None)
        try:
            # Token feedback, embedding and the first input norm in one launch.
            residual, h = embedding_rms_norm(
                self.token_state, self.source_lanes, self.host_tokens, self.weights.embedding,
                self.weights.layers[0].input_norm, eps, x_output=self.embedding_output,
                norm_output=self.norm_output)
            folded = self._folded() if self._folded is not None else None
            for index, layer in enumerate(self.weights.layers):
                if folded is not None:
                    qkv = linear_kstream(residual, folded[index][0], norm_eps=eps)
                else:
                    qkv = _project(h, layer.qkv)
                key_cache = self.cache.key_cache[index]
                value_cache = self.cache.value_cache[index]
                if self.fused_rope:
                    # RoPE, k and v into their pages, and attention: one launch.
                    paged_gqa_decode_attention_rope_append(
                        qkv, self.positions, self.weights.rope_cos, self.weights.rope_sin,
                        key_cache, value_cache, self.physical_blocks, self.block_offsets,
                        self.active_mask, self.block_tables, self.context_lengths,
                        query_heads=hq, max_context_length=self.context_capacity,
                        output=self.attention_output, workspace=self.workspace,
                        scale=d ** -0.5)
                else:
                    # RoPE on q and k, k and v into their pages: one launch.
                    q = rope_paged_kv_append(qkv, self.positions, self.weights.rope_cos,
                                             self.weights.rope_sin, key_cache, value_cache,
                                             self.physical_blocks, self.block_offsets,
                                             self.active_mask, query_heads=hq,
                                             query_output=self.query)
                    paged_gqa_decode_attention(
                        q, key_cache, value_cache, self.block_tables, self.context_lengths,
                        scale=d ** -0.5, max_context_length=self.context_capacity,
                        output=self.attention_output, workspace=self.workspace)
                attention = self.attention_output.view(b, hq * d)
                if folded is not None:
                    residual = linear_kstream(attention, layer.o_proj, residual=residual)
                    act = linear_swiglu(residual, folded[index][1], output=self.swiglu_output,
                                        k_split=True, norm_eps=eps)
                    residual = linear_kstream(act, layer.down, residual=residual)
                    continue
                if self.split_o:
                    linear_stream(attention, layer.o_proj, splits=self.split_o,
                                  partials=self.partials_o)
                    residual, h = residual_rms_norm_partials(
                        self.partials_o, residual, layer.post_norm, eps,
                        residual_output=torch.empty_like(residual), norm_output=self.norm_output)
                else:
                    attn = _project(attention, layer.o_proj)
                    residual, h = residual_rms_norm(attn, residual, layer.post_norm, eps,
                                                    residual_output=torch.empty_like(attn),
                                                    norm_output=self.norm_output)
                if self.fused_gate_up:
                    act = linear_swiglu(h, layer.gate_up, output=self.swiglu_output,
                                        k_split=True)
                else:
                    act = swiglu_gate_up(_project(h, layer.gate_up), output=self.swiglu_output)
                next_norm = (self.weights.layers[index + 1].input_norm
                             if index + 1 < len(self.weights.layers) else self.weights.final_norm)
                if self.split_down:
                    linear_stream(act, layer.down, splits=self.split_down,
                                  partials=self.partials_down)
                    residual, h = residual_rms_norm_partials(
                        self.partials_down, residual, next_norm, eps,
                        residual_output=torch.empty_like(residual), norm_output=self.norm_output)
                else:
                    mlp = _project(act, layer.down)
                    residual, h = residual_rms_norm(mlp, residual, next_norm, eps,
                                                    residual_output=torch.empty_like(mlp),
                                                    norm_output=self.norm_output)
            if folded is not None:
                h = rms_norm(residual, self.weights.final_norm, eps, output=self.norm_output)
            _project(h, self.weights.lm_head, output=self.logits)
            argmax_rows(self.logits, output=self.next_tokens)
        finally:
            set_attention_split_size(previous)


def prefill(weights: DecoderWeights, cache: PagedKVCache, request_id: str,
            prompt: list[int]) -> tuple[int, Tensor]:
    """One prompt: (greedy next token, last-position logits) -- the
    reference's prefill_request (runtime/prefill.py:19-34)."""

    return prefill_batch(weights, cache, {request_id: prompt})[request_id]


def _causal_attention(q: Tensor, k: Tensor, v: Tensor, scale: float) -> Tensor:
    """q [S, Hq, D], k/v [S, Hkv, D] of one prompt -> context [S, Hq * D]:
    causal attention through torch's fused (flash / memory-efficient) SDPA
    kernels with contiguous operands, kv heads expanded to the query heads.
    The math backend is excluded: it would run batched products on
    transposed views."""

    seq, hq, d = q.shape
    group = hq // k.shape[1]
    qh = q.transpose(0, 1).unsqueeze(0).contiguous()                           # [1, Hq, S, D]
    kh = k.repeat_interleave(group, dim=1).transpose(0, 1).unsqueeze(0).contiguous()
    vh = v.repeat_interleave(group, dim=1).transpose(0, 1).unsqueeze(0).contiguous()
    with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        context = F.scaled_dot_product_attention(qh, kh, vh, is_causal=True, scale=scale)
    return context[0].transpose(0, 1).reshape(seq, hq * d)


def _validate_prompt(weights: DecoderWeights, cache: PagedKVCache, request_id: str,
                     prompt) -> None:
    """Host-side checks of one prompt before any reservation or device work
    (runtime/prefill.py:175-185): an id outside the vocabulary would index
    the embedding table out of range on the device."""

    if len(prompt) == 0:
        raise ValueError("prompt must contain at least one token")
    ids = np.asarray(prompt, dtype=np.int64)
    if ids.ndim != 1 or bool(((ids < 0) | (ids >= weights.config.vocab_size)).any()):
        raise ValueError("prompt token is outside the model vocabulary")
    if cache.sequence_layout(request_id).context_length != 0:
        raise ValueError("prefill ingests fresh sequences only")
    if len(prompt) > weights.rope_cos.shape[0]:
        raise ValueError("prompt exceeds the model's RoPE table")


def _prefill_packed(weights: DecoderWeights, cache: PagedKVCache, prompts: dict[str, list[int]],
                    ) -> Tensor:
    """Run the packed prefill of reserved, validated prompts; last-position
    logits [len(prompts), vocab] in prompt order.  Writes every layer's
    pages; commit or rollback is the caller's."""

    config = weights.config
    hq, hkv, d = config.num_attention_heads, config.num_key_value_heads, config.head_dim
    device = cache.config.device
    block_size = cache.config.block_size
    request_ids = list(prompts)
    lengths = [len(prompts[r]) for r in request_ids]
    bounds = np.concatenate(([0], np.cumsum(lengths)))
    total = int(bounds[-1])
    longs = np.empty((2, total), dtype=np.int64)   # token ids, positions
    ints = np.ones((3, total), dtype=np.int32)     # pages, offsets, active
    for i, request_id in enumerate(request_ids):
        lo, hi = bounds[i], bounds[i + 1]
        positions = np.arange(hi - lo, dtype=np.int64)
        pages = np.asarray(cache.page_list(request_id)[0], dtype=np.int32)
        longs[0, lo:hi] = prompts[request_id]
        longs[1, lo:hi] = positions
        ints[0, lo:hi] = pages[positions // block_size]
        ints[1, lo:hi] = positions % block_size
    longs_dev = torch.from_numpy(longs).to(device)
    ints_dev = torch.from_numpy(ints).to(device)
    packed_attention = prefill_attention_supported(weights.embedding.dtype, hq, hkv, d)
    if packed_attention:
        tiles = torch.from_numpy(prefill_tiles(lengths)).to(device)
    tokens, positions_dev = longs_dev[0], longs_dev[1]
    eps = config.rms_norm_eps
    residual = F.embedding(tokens, weights.embedding)
    h = rms_norm(residual, weights.layers[0].input_norm, eps)
    q = torch.empty((total, hq, d), dtype=residual.dtype, device=device)
    k = torch.empty((total, hkv, d), dtype=residual.dtype, device=device)
    context = torch.empty((total, hq * d), dtype=residual.dtype, device=device)
    for index, layer in enumerate(weights.layers):
        qkv = F.linear(h, layer.qkv)
        rope_paged_kv_append(qkv, positions_dev, weights.rope_cos, weights.rope_sin,
                             cache.key_cache[index], cache.value_cache[index], ints_dev[0],
                             ints_dev[1], ints_dev[2], query_heads=hq, query_output=q,
                             key_output=k)
        if packed_attention:  # every prompt's causal attention in one launch
            prefill_attention(q.view(total, hq * d), k.view(total, hkv * d),
                              qkv[:, (hq + hkv) * d:], tiles, query_heads=hq,
                              kv_heads=hkv, scale=d ** -0.5, output=context)
        else:
            v = qkv[:, (hq + hkv) * d:].view(total, hkv, d)
            for i in range(len(request_ids)):
                lo, hi = int(bounds[i]), int(bounds[i + 1])
                context[lo:hi] = _causal_attention(q[lo:hi], k[lo:hi], v[lo:hi], d ** -0.5)
        attn = F.linear(context, layer.o_proj)
        residual, h = residual_rms_norm(attn, residual, layer.post_norm, eps)
        act = swiglu_gate_up(F.linear(h, layer.gate_up))
        next_norm = (weights.layers[index + 1].input_norm
                     if index + 1 < len(weights.layers) else weights.final_norm)
        residual, h = residual_rms_norm(F.linear(act, layer.down), residual, next_norm, eps)
    last = torch.from_numpy(bounds[1:] - 1).to(device)
    return F.linear(h.index_select(0, last), weights.lm_head)


def prefill_requests(weights: DecoderWeights, cache: PagedKVCache,
                     prompts: dict[str, list[int]]) -> BatchExecutionResult:
    """Prefill fresh prompts together, each in a transaction of its own
    (runtime/prefill.py:37-149): the last position's logits of every prompt
    that ran, and an error message for every prompt that could not.

    A prompt with an id outside the vocabulary, a sequence that is not
    fresh or a reservation the cache cannot make fails alone, before any
    device work; the others run.  A failure of the packed launch itself
    rolls back every reservation and fails every request of the call.

    The reference pads the prompts into one [batch, longest] causal batch
    and writes each request's K/V with its own write_layer per layer.  Here
    the prompts' tokens are packed into one [total, H] stream with no
    padding: every projection is one GEMM over all tokens, and one
    rope_paged_kv_append launch per layer rotates q and k of every token and
    writes k, v straight into the pages each token's position maps to.
    Attention is one packed causal launch per layer over all prompts
    (prefill_attention; torch's fused causal SDPA per prompt for geometries
    that kernel does not serve).
    """

    if not prompts:
        raise ValueError("prefill requires at least one prompt")
    errors: dict[str, str] = {}
    reservations: dict[str, AppendReservation] = {}
    for request_id, prompt in prompts.items():
        try:
            _validate_prompt(weights, cache, request_id, prompt)
            reservations[request_id] = cache.begin_append(request_id, len(prompt))
        except Exception as error:  # noqa: BLE001 - reported per request
            errors[request_id] = f"{type(error).__name__}: {error}"
    if not reservations:
        return BatchExecutionResult(logits={}, errors=errors)
    try:
        logits = _prefill_packed(weights, cache, {r: list(prompts[r]) for r in reservations})
    except Exception as error:  # noqa: BLE001 - the whole launch failed
        message = f"{type(error).__name__}: {error}"
        for request_id, reservation in reservations.items():
            with suppress(RuntimeError):
                cache.rollback(reservation)
            errors[request_id] = message
        return BatchExecutionResult(logits={}, errors=errors)
    for reservation in reservations.values():
        cache.record_all_layers_written(reservation)
        cache.commit(reservation)
    return BatchExecutionResult(
        logits={request_id: logits[i] for i, request_id in enumerate(reservations)},
        errors=errors)


def prefill_batch(weights: DecoderWeights, cache: PagedKVCache,
                  prompts: dict[str, list[int]]) -> dict[str, tuple[int, Tensor]]:
    """Prefill several fresh prompts together, all or nothing: {request_id:
    (greedy next token, last-position logits)}.  Every prompt is validated
    on the host and every reservation made before any device work; any
    failure rolls back the reservations made and raises."""

    if not prompts:
        raise ValueError("prefill_batch requires at least one prompt")
    for request_id, prompt in prompts.items():
        _validate_prompt(weights, cache, request_id, prompt)
    reservations: dict[str, AppendReservation] = {}
    try:
        for request_id, prompt in prompts.items():
            reservations[request_id] = cache.begin_append(request_id, len(prompt))
        logits = _prefill_packed(weights, cache, {r: list(p) for r, p in prompts.items()})
        first_tokens = torch.argmax(logits, dim=-1).tolist()
    except Exception:
        for reservation in reservations.values():
            cache.rollback(reservation)
        raise
    for reservation in reservations.values():
        cache.record_all_layers_written(reservation)
        cache.commit(reservation)
    return {request_id: (first_tokens[i], logits[i]) for i, request_id in enumerate(prompts)}


DEFAULT_BATCH_BUCKETS = (1, 2, 4, 8, 16, 32, 64)
DEFAULT_CONTEXT_BUCKETS = (512, 1024, 2048, 4096)


@dataclass(frozen=True, slots=True)
class DecodeExecutionMetrics:
    """Counters of the executor's step dispatch (the graph and fallback
    fields of decode_bucket.py:140-154).  ``graph_misses`` counts steps
    that captured their bucket's graph and steps that fell back to an
    eager step because no bucket holds them; ``fallback_reasons`` counts
    the latter by "batch_overflow", "context_overflow" or
    "batch_and_context_overflow"."""

    eager_calls: int
    graph_calls: int
    graph_hits: int
    graph_misses: int
    shape_fallbacks: int
    eager_fallback_calls: int
    capture_count: int
    capture_time_ms: float
    capture_warmup_time_ms: float
    padded_lanes: int
    fallback_reasons: dict[str, int]


@dataclass(slots=True)
class _MutableMetrics:
    eager_calls: int = 0
    graph_calls: int = 0
    graph_hits: int = 0
    graph_misses: int = 0
    shape_fallbacks: int = 0
    eager_fallback_calls: int = 0
    capture_count: int = 0
    capture_time_ms: float = 0.0
    capture_warmup_time_ms: float = 0.0
    padded_lanes: int = 0
    fallback_reasons: dict[str, int] = field(default_factory=dict)


@dataclass(slots=True)
class DecodeTicket:
    """One launched decode step whose sampled tokens have not been read yet.
    ``request_ids`` are the requests that run in it, in lane order;
    ``errors`` the requests of the launch that could not run, with why.
    A launch in which no request could run has no slot (-1)."""

    request_ids: tuple[str, ...]
    bucket: tuple[int, int]
    slot: int
    errors: dict[str, str] = field(default_factory=dict)


@dataclass(frozen=True, slots=True)
class DecodeStepRecord:
    bucket: tuple[int, int]
    lanes: int
    device_ms: float
    graph: bool = True


class BucketedDecodeExecutor:
    """Decode executor over graph buckets (reference:
    BucketedPagedDecodeExecutor, decode_bucket.py:532-666).

    ``launch`` stages and replays one step and returns at once; ``collect``
    returns that step's sampled tokens.  A request that ran in the previously
    launched step needs no host token: its lane's sample is fed back on the
    device.  So a serving loop can launch step n+1 before reading step n's
    tokens and keep the GPU one step ahead of the host.  ``append_tokens``
    and ``prefill_prompts`` are the reference's synchronous contract (host
    tokens or prompts in, ``BatchExecutionResult`` of logits and per-request
    errors out).

    Failures are per request: a token outside the vocabulary, a missing
    input token, a position past the RoPE table or a reservation the cache
    cannot make fails that request alone, before anything is staged, and
    the others run.  A step that no bucket holds (more requests than the
    largest batch bucket, or a context past the largest context bucket) runs
    eagerly on buffers sized for it, counted in ``metrics()`` with its
    reason (decode_bucket.py:597-614).
    """

    _RING = 4

    def __init__(self, weights: DecoderWeights, cache: PagedKVCache, *,
                 batch_buckets: tuple[int, ...] = DEFAULT_BATCH_BUCKETS,
                 context_buckets: tuple[int, ...] = DEFAULT_CONTEXT_BUCKETS,
                 fuse_norms: bool = True) -> None:
        if not batch_buckets or any(value <= 0 for value in batch_buckets):
            raise ValueError("batch_buckets must contain positive capacities")
        if not context_buckets or any(value <= 0 for value in context_buckets):
            raise ValueError("context_buckets must contain positive capacities")
        self.weights = weights
        self.cache = cache
        self.batch_buckets = tuple(sorted(set(batch_buckets)))
        self.context_buckets = tuple(sorted(set(context_buckets)))
        if self.batch_buckets[-1] > cache.config.max_sequences:
            raise ValueError("batch bucket exceeds cache sequence capacity")
        if self.context_buckets[-1] > cache.config.max_sequence_length:
            raise ValueError("context bucket exceeds cache sequence capacity")
        device = cache.config.device
        # One sampled-token slot per lane of any step: a step never holds
        # more requests than the cache has sequences, fallback steps included.
        lanes = max(self.batch_buckets[-1], cache.config.max_sequences)
        self.token_state = torch.zeros(lanes, dtype=torch.long, device=device)
        self._buckets: dict[tuple[int, int], DecodeGraphBucket] = {}
        self._fallbacks: dict[tuple[int, int], DecodeGraphBucket] = {}
        self._last_lanes: dict[str, int] = {}
        self._readback = [torch.zeros(lanes, dtype=torch.long, pin_memory=True)
                          for _ in range(self._RING)]
        self._events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True),
                         torch.cuda.Event()) for _ in range(self._RING)]
        self._busy = [False] * self._RING
        self._slot_bucket: list[DecodeGraphBucket | None] = [None] * self._RING
        self._next_slot = 0
        self._metrics = _MutableMetrics()
        self.step_records: list[DecodeStepRecord] = []
        self._folded_weights: list[tuple[Tensor, Tensor]] | None = None
        self._folded_sources: list[Tensor] = []
        self._folded_version = 0
        # Requests whose logits every pipelined step copies to the host
        # (``watch_logits``), per ring slot: pinned rows and the lanes held.
        self.watch_logits: set[str] = set()
        self._watch_host: list[Tensor | None] = [None] * self._RING
        self._watch_lanes: list[list[tuple[int, str]]] = [[] for _ in range(self._RING)]
        # fuse_norms=False keeps the RMSNorm launches between the
        # projections (the split-K partials path) in every bucket.
        self._fold = self._folded if fuse_norms else None

    def _folded(self) -> list[tuple[Tensor, Tensor]]:
        """Per layer, the qkv and gate|up weights with the input and
        post-attention norm gains folded in (made on first use, shared by
        every bucket of this executor)."""

        if self._folded_weights is None:
            self._folded_weights = [(fold_norm_gain(layer.qkv, layer.input_norm),
                                     fold_norm_gain(layer.gate_up, layer.post_norm))
                                    for layer in self.weights.layers]
            self._folded_sources = [tensor for layer in self.weights.layers
                                    for tensor in (layer.qkv, layer.input_norm, layer.gate_up,
                                                   layer.post_norm)]
            self._folded_version = sum(t._version for t in self._folded_sources)
        return self._folded_weights

    def refresh_weights(self) -> bool:
        """Remake the folded qkv and gate|up copies, in place (the captured
        graphs keep their addresses), if a weight or norm gain they come from
        was changed in place since they were made (``layer.qkv.copy_(...)``,
        a reload into the same tensors: torch counts such writes in each
        tensor's version, which only grows).  Called by ``launch`` before
        every step (about 8 us of host time at 22 layers); returns whether
        the copies were remade.  Weights replaced by new tensors are not seen
        by graphs captured before; build a new executor for them."""

        if self._folded_weights is None:
            return False
        version = sum(t._version for t in self._folded_sources)
        if version == self._folded_version:
            return False
        for (qkv, gate_up), layer in zip(self._folded_weights, self.weights.layers):
            qkv.copy_(fold_norm_gain(layer.qkv, layer.input_norm))
            gate_up.copy_(fold_norm_gain(layer.gate_up, layer.post_norm))
        self._folded_version = version
        return True

    @property
    def vocab_size(self) -> int:
        return self.weights.config.vocab_size

    def metrics(self) -> DecodeExecutionMetrics:
        values = asdict(self._metrics)
        values["fallback_reasons"] = dict(self._metrics.fallback_reasons)
        return DecodeExecutionMetrics(**values)

    def create_request(self, request_id: str) -> None:
        self.cache.create_sequence(request_id)

    def release_request(self, request_id: str) -> None:
        self._last_lanes.pop(request_id, None)
        self.cache.release(request_id)

    def prefill_prompts(self, prompts: dict[str, tuple[int, ...]]) -> BatchExecutionResult:
        """Prefill the prompts together; the last position's logits of each
        that ran and the errors of those that could not
        (decode_bucket.py:567-570, runtime/prefill.py:37-149)."""

        return prefill_requests(self.weights, self.cache, {r: list(p) for r, p in prompts.items()})

    def prefill_tokens(self, prompts: dict[str, tuple[int, ...]],
                       ) -> tuple[dict[str, int], dict[str, str]]:
        """``prefill_prompts`` with the greedy first token of each prompt that
        ran (one device-to-host copy) instead of its logits."""

        result = self.prefill_prompts(prompts)
        if not result.logits:
            return {}, dict(result.errors)
        ids = list(result.logits)
        tokens = torch.argmax(torch.stack([result.logits[r] for r in ids]), dim=-1).tolist()
        return dict(zip(ids, tokens)), dict(result.errors)

    def buffer_addresses(self) -> dict[str, dict[str, int]]:
        return {f"b{batch}-c{context}": bucket.addresses()
                for (batch, context), bucket in self._buckets.items()}

    def _capacities(self, batch: int, context: int) -> tuple[int | None, int | None]:
        batch_capacity = next((v for v in self.batch_buckets if v >= batch), None)
        context_capacity = next((v for v in self.context_buckets if v >= context), None)
        return batch_capacity, context_capacity

    def bucket(self, batch: int, context: int) -> DecodeGraphBucket:
        batch_capacity, context_capacity = self._capacities(batch, context)
        if batch_capacity is None or context_capacity is None:
            raise ValueError(f"no decode bucket holds batch {batch} at context {context}")
        key = (batch_capacity, context_capacity)
        if key not in self._buckets:
            self._buckets[key] = DecodeGraphBucket(
                self.weights, self.cache, batch_capacity=batch_capacity,
                context_capacity=context_capacity, token_state=self.token_state,
                metrics=self._metrics, folded=self._fold)
        return self._buckets[key]

    def _fallback_bucket(self, batch: int, context: int) -> DecodeGraphBucket:
        """Eager buffers for a step no graph bucket holds: batch rounded up
        to a multiple of 16 (within the cache's sequences), context up to
        the cache's maximum sequence length."""

        config = self.cache.config
        capacity = min(-(-batch // 16) * 16, config.max_sequences)
        key = (capacity, config.max_sequence_length)
        if key not in self._fallbacks:
            self._fallbacks[key] = DecodeGraphBucket(
                self.weights, self.cache, batch_capacity=capacity,
                context_capacity=config.max_sequence_length, token_state=self.token_state,
                graph=False, metrics=self._metrics, folded=self._fold)
        return self._fallbacks[key]

    def capture_all(self) -> None:
        """Capture every (batch, context) bucket now, with all lanes padded,
        so no capture lands inside a timed run.  Only between requests: it
        overwrites the sampled-token state."""

        if any(self._busy):
            raise RuntimeError("capture_all with decode steps in flight")
        for batch in self.batch_buckets:
            for context in self.context_buckets:
                bucket = self.bucket(batch, context)
                bucket.prepare([], {})
                bucket.execute()
        self._last_lanes = {}
        torch.cuda.synchronize(self.cache.config.device)

    def launch(self, request_ids: list[str], tokens: dict[str, int] | None = None) -> DecodeTicket:
        """Append one token to each request and enqueue the step.  Requests in
        ``tokens`` take that input token; the others must have run in the
        previously launched step, whose sample they continue from.  Requests
        that cannot run are left out of the step and listed in the ticket's
        ``errors`` with nothing of theirs reserved."""

        tokens = tokens or {}
        if not request_ids:
            raise ValueError("launch requires at least one request")
        self.refresh_weights()
        slot = self._next_slot
        if self._busy[slot]:
            raise RuntimeError("too many decode steps launched without collect()")
        errors: dict[str, str] = {}
        reservations: dict[str, AppendReservation] = {}
        max_position = self.weights.rope_cos.shape[0]
        for request_id in request_ids:
            if request_id in tokens:
                if not 0 <= tokens[request_id] < self.vocab_size:
                    errors[request_id] = "token_id is outside the model vocabulary"
                    continue
            elif request_id not in self._last_lanes:
                errors[request_id] = "no input token (the request was not in the previous step)"
                continue
            try:
                reservation = self.cache.begin_append(request_id, 1)
            except Exception as error:  # noqa: BLE001 - reported per request
                errors[request_id] = f"{type(error).__name__}: {error}"
                continue
            if reservation.start_position >= max_position:
                self.cache.rollback(reservation)
                errors[request_id] = "position exceeds the model's RoPE table"
                continue
            reservations[request_id] = reservation
        staged = list(reservations)
        if not staged:
            return DecodeTicket((), (0, 0), -1, errors)
        context = max(r.end_position for r in reservations.values())
        batch_capacity, context_capacity = self._capacities(len(staged), context)
        try:
            if batch_capacity is None or context_capacity is None:
                reason = ("batch_and_context_overflow" if batch_capacity is None
                          and context_capacity is None else
                          "batch_overflow" if batch_capacity is None else "context_overflow")
                metrics = self._metrics
                metrics.shape_fallbacks += 1
                metrics.eager_fallback_calls += 1
                metrics.graph_misses += 1
                metrics.fallback_reasons[reason] = metrics.fallback_reasons.get(reason, 0) + 1
                bucket = self._fallback_bucket(len(staged), context)
            else:
                bucket = self.bucket(len(staged), context)
            bucket.prepare(staged, reservations, tokens=tokens, source_lanes=self._last_lanes)
        except Exception as error:  # noqa: BLE001 - nothing was launched
            message = f"{type(error).__name__}: {error}"
            for request_id, reservation in reservations.items():
                self.cache.rollback(reservation)
                errors[request_id] = message
            return DecodeTicket((), (0, 0), -1, errors)
        self._metrics.padded_lanes += bucket.batch_capacity - len(staged)
        begin, end, copied = self._events[slot]
        begin.record()
        try:
            bucket.execute()
        except Exception as error:  # noqa: BLE001
            # Nothing of this step is committed; its lanes' previous samples
            # are no longer trusted as inputs either.
            message = f"{type(error).__name__}: {error}"
            for request_id, reservation in reservations.items():
                with suppress(RuntimeError):
                    self.cache.rollback(reservation)
                errors[request_id] = message
            self._last_lanes = {}
            return DecodeTicket((), (0, 0), -1, errors)
        end.record()
        lanes = len(staged)
        self._readback[slot][:lanes].copy_(self.token_state[:lanes], non_blocking=True)
        watched = [(lane, request_id) for lane, request_id in enumerate(staged)
                   if request_id in self.watch_logits]
        if watched:
            host = self._watch_host[slot]
            if host is None or host.shape[0] < len(watched) or host.dtype != bucket.logits.dtype:
                host = torch.empty((max(len(watched), 8), self.vocab_size),
                                   dtype=bucket.logits.dtype, pin_memory=True)
                self._watch_host[slot] = host
            # Ordered on the stream before any later step rewrites the rows.
            for index, (lane, _) in enumerate(watched):
                host[index].copy_(bucket.logits[lane], non_blocking=True)
        self._watch_lanes[slot] = watched
        copied.record()
        # Host bookkeeping only: the step's device work is ordered before any
        # later reader of these pages on this stream.
        for reservation in reservations.values():
            self.cache.record_all_layers_written(reservation)
            self.cache.commit(reservation)
        self._last_lanes = {request_id: lane for lane, request_id in enumerate(staged)}
        self._slot_bucket[slot] = bucket
        self._busy[slot] = True
        self._next_slot = (slot + 1) % self._RING
        return DecodeTicket(tuple(staged), (bucket.batch_capacity, bucket.context_capacity),
                            slot, errors)

    def collect(self, ticket: DecodeTicket) -> list[int]:
        """Wait for a launched step; its sampled token per request, in order."""

        if ticket.slot < 0:
            return []
        if not self._busy[ticket.slot]:
            raise RuntimeError("decode ticket was already collected")
        begin, end, copied = self._events[ticket.slot]
        copied.synchronize()
        lanes = len(ticket.request_ids)
        sampled = self._readback[ticket.slot][:lanes].tolist()
        bucket = self._slot_bucket[ticket.slot]
        self.step_records.append(DecodeStepRecord(ticket.bucket, lanes, begin.elapsed_time(end),
                                                  bucket is not None and bucket.graph))
        self._busy[ticket.slot] = False
        return sampled

    def watched_logits(self, ticket: DecodeTicket) -> dict[str, Tensor]:
        """Host copies (the model dtype) of the logits behind a collected
        step's tokens for its requests in ``watch_logits`` -- valid in the
        pipelined mode too, where the bucket's own buffer has moved on.
        Call after ``collect`` of the ticket and before its slot is reused
        (``_RING`` launches later)."""

        if ticket.slot < 0 or self._busy[ticket.slot]:
            return {}
        host = self._watch_host[ticket.slot]
        return {request_id: host[index].clone()
                for index, (_, request_id) in enumerate(self._watch_lanes[ticket.slot])}

    def logits_of(self, ticket: DecodeTicket) -> dict[str, Tensor]:
        """The collected step's logits per request: views into its bucket's
        logits buffer, valid until the bucket runs again."""

        if ticket.slot < 0:
            return {}
        bucket = self._slot_bucket[ticket.slot]
        return {request_id: bucket.logits[lane] for lane, request_id in enumerate(ticket.request_ids)}

    def append_tokens(self, tokens: dict[str, int]) -> BatchExecutionResult:
        """The reference's synchronous step (decode_bucket.py:582-666): logits
        of every request that ran (views into the bucket's logits buffer,
        valid until the next step) and the errors of those that could not."""

        if not tokens:
            raise ValueError("append_tokens requires at least one request")
        ticket = self.launch(list(tokens), tokens)
        self.collect(ticket)
        return BatchExecutionResult(logits=self.logits_of(ticket), errors=dict(ticket.errors))


def greedy_decode(executor: BucketedDecodeExecutor, prompts: dict[str, list[int]],
                  steps: int, *, logits: dict[str, list[Tensor]] | None = None,
                  ) -> dict[str, list[int]]:
    """Prefill each prompt, then decode ``steps - 1`` more greedy tokens for
    all of them together, keeping one step in flight: step n+1 is launched
    (its inputs fed back on the device) before step n's tokens are read.
    Raises on the first request that fails.

    With ``logits`` (a dict to fill) every step is read back before the next
    is launched -- the inputs are still fed back on the device -- and the
    fp32 logits row behind each sampled token is appended per request."""

    outputs: dict[str, list[int]] = {}
    for request_id, prompt in prompts.items():
        executor.create_request(request_id)
    if logits is None:
        first, errors = executor.prefill_tokens(prompts)
    else:
        result = executor.prefill_prompts(prompts)
        errors = dict(result.errors)
        first = {}
        for request_id, row in result.logits.items():
            logits[request_id] = [row.float().cpu()]
            first[request_id] = int(torch.argmax(row))
    if errors:
        raise RuntimeError(f"prefill failed: {errors}")
    for request_id in prompts:
        outputs[request_id] = [first[request_id]]
    order = list(prompts)
    pending: DecodeTicket | None = None
    for step in range(steps - 1):
        ticket = executor.launch(order, first if step == 0 else None)
        if ticket.errors:
            raise RuntimeError(f"decode step failed: {ticket.errors}")
        if logits is not None:
            for request_id, token in zip(order, executor.collect(ticket)):
                outputs[request_id].append(token)
            for request_id, row in executor.logits_of(ticket).items():
                logits[request_id].append(row.float().cpu())
            continue
        if pending is not None:
            for request_id, token in zip(order, executor.collect(pending)):
                outputs[request_id].append(token)
        pending = ticket
    if pending is not None:
        for request_id, token in zip(order, executor.collect(pending)):
            outputs[request_id].append(token)
    return outputs
