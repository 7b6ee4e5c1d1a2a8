"""Paged GQA decode attention over a paged KV cache, on gfx950 HIP kernels.

Drop-in counterpart of ``tensorforge/kernels/triton_attention.py``: the
public names, the call signature, the validation order, exception types and
messages, the caller-owned ``output``/``workspace`` contract and the dispatch
record are those of the reference (file:line cited per function).  The
kernels behind it are the hand-written HIP kernels of
``tensorforge_amd/csrc/tf_paged_attention.hip`` called through the C ABI on
torch's current stream; nothing here synchronises with the device when
``max_context_length`` is given, so a call can be captured in a HIP graph.
"""

from __future__ import annotations

import dataclasses
from dataclasses import dataclass
from typing import Any

import torch
from torch import Tensor

from tensorforge_amd import _native

# Tokens per split-KV partition of the reference (triton_attention.py:46,406).
# The workspace capacity contract is sized for this value, so a smaller split
# needs a workspace allocated for it; larger ones fit any reference-sized
# workspace.
REFERENCE_SPLIT_SIZE = 256

# None: choose the partition size per call (attention_split_size_for).
_SPLIT_SIZE: int | None = None
_LAST_ATTENTION_CONFIG: dict[str, Any] | None = None
_LAST_ATTENTION_LAUNCH: dict[str, Any] | None = None


def _next_power_of_2(value: int) -> int:
    return 1 << (value - 1).bit_length() if value > 1 else 1


@dataclass(frozen=True, slots=True)
class PagedAttentionWorkspace:
    """Caller-owned split-KV buffers whose addresses can remain graph-stable.

    Same fields and capacity rule as ``triton_attention.py:25-57``: buffers
    hold ``batch_capacity * query_heads * ceil(max_context_length / 256)``
    fp32 partial rows, accumulator rows padded to ``next_pow2(head_dim)``.
    ``split_counters`` (no reference counterpart; optional, so workspaces
    built from the three reference fields still work) holds one zeroed int32
    arrival counter per (row, head): with it the last workgroup of a row
    merges the partials inside the split kernel and resets its counter, so
    the call is one launch and stays graph-replay safe.
    """

    partial_max: Tensor
    partial_sum: Tensor
    partial_accumulator: Tensor
    split_counters: Tensor | None = None

    @classmethod
    def allocate(
        cls,
        *,
        batch_capacity: int,
        query_heads: int,
        head_dim: int,
        max_context_length: int,
        device: torch.device,
    ) -> PagedAttentionWorkspace:
        dimensions = (batch_capacity, query_heads, head_dim, max_context_length)
        if any(value <= 0 for value in dimensions):
            raise ValueError("workspace dimensions must be positive")
        num_splits = (max_context_length + REFERENCE_SPLIT_SIZE - 1) // REFERENCE_SPLIT_SIZE
        programs = batch_capacity * query_heads * num_splits
        head_bucket = _next_power_of_2(head_dim)
        partial_max = torch.empty(programs, device=device, dtype=torch.float32)
        return cls(
            partial_max=partial_max,
            partial_sum=torch.empty_like(partial_max),
            partial_accumulator=torch.empty(
                (programs, head_bucket), device=device, dtype=torch.float32
            ),
            split_counters=torch.zeros(
                batch_capacity * query_heads, device=device, dtype=torch.int32
            ),
        )


def is_hip_attention_available() -> bool:
    """True when the gfx950 attention library is built and loadable."""

    return _native.is_available()


def set_attention_split_size(split_size: int | None) -> int | None:
    """Fix the split-KV partition size (tokens) and return the previous one.

    A positive multiple of 32, or None for the per-call choice of
    :func:`attention_split_size_for`.  Sizes below 256 need a workspace
    allocated with at least ``ceil(context / split_size)`` partials per head.
    """

    global _SPLIT_SIZE
    if split_size is not None and (split_size <= 0 or split_size % 32 != 0):
        raise ValueError("split_size must be a positive multiple of 32")
    previous = _SPLIT_SIZE
    _SPLIT_SIZE = split_size
    return previous


def attention_split_size() -> int | None:
    """The fixed partition size, or None when it is chosen per call."""

    return _SPLIT_SIZE


def attention_split_size_for(max_context_length: int, batch: int, kv_heads: int) -> int:
    """Partition size chosen from host-known sizes only (no device sync).

    One wavefront streams one (row, kv head, split) and the merge reads every
    split's partial, so the size balances three things: enough wavefronts to
    cover the GPU, few enough that their loads do not congest HBM (measured
    best near 500-1300 wavefronts in flight on MI355X), and at most 16 splits
    per row.  ``max(256, ceil64(L * B * Hkv / 1024), ceil64(L / 16))``: 576
    for 72 rows x 4 kv heads at 2k, 2048 for 4 x 8 at 32k, and the
    reference's 256 for short batches.
    """

    def ceil64(value: int) -> int:
        return (value + 63) // 64 * 64

    return max(
        REFERENCE_SPLIT_SIZE,
        ceil64(max_context_length * max(batch, 1) * kv_heads // 1024),
        ceil64((max_context_length + 15) // 16),
    )


# One pass (no split-KV, no merge launch) when a call has at least this many
# (row, kv head) workgroups to spread over the 256 CUs (measured on MI355X at
# 2k contexts, 4 kv heads: 48 rows 20.5 us one pass vs 21.7 split; 32 rows
# 18.7 vs 16.1).
ONE_PASS_MIN_WORKGROUPS = 192
# Tokens per wavefront that set the one-pass wavefronts per kv head (swept
# on MI355X at config 2, three seeds: 576 with up to 4 wavefronts per 2k row
# beats 448 / 512 / 640 and the 768 / 3 of the operand-layout loads).
ONE_PASS_TOKENS_PER_WAVE = 576
# Narrow calls (fewer workgroups than ONE_PASS_MIN_WORKGROUPS).  Measured on
# MI355X with the K/V read from HBM (one 1 GB page pool, tables rotated over
# disjoint pages; TinyLlama 32/4 heads at D 64 and Llama-3 32/8 at D 128,
# 1-47 rows of 64-32768 tokens), graph-timed through the C ABI:
# * split-KV (narrow_split_plan) wins once a (row, kv head) holds >=
#   NARROW_SPLIT_MIN_BYTES of K and V (NARROW_SPLIT_MIN_BYTES_WIDE above
#   NARROW_SPLIT_WIDE_GRID one-pass workgroups), in partitions of equal size
#   that put about one workgroup on each compute unit, two wavefronts each,
#   kv heads paired in a workgroup (256-byte slices of each token row) where
#   one head's slice is narrower.  1 x 1000 at D 64: 7.7 us against 10.4 for
#   one pass with eight wavefronts of 64 tokens; 8 x 1000 8.6 against 11.3;
#   32 x 2048 15.3 against 19.7; 32 x 3000 20.0 (four partitions of pairs)
#   against 22.7 for two partitions of one kv head and 27.6 for one pass;
#   47 x 3000 23.9 (three of pairs) against 28.3; 4 x 1000 at D 128 10.7
#   against 19.0; 1 x 32k at D 128 29.1 against 38.5 for 2048-token
#   partitions of four wavefronts.  Below the byte floor one pass is as
#   fast or faster (1 x 256 at D 64: 5.3 against 7.2 us with two partitions;
#   32 x 800: 9.6 against 10.2);
# * otherwise one pass with up to NARROW_WAVES wavefronts per kv head, a row
#   using one per max(64, head_dim, ceil64(context / 4)) of its tokens (1-47
#   rows x 64 / 200 / 512 tokens at D 64: 3.7-3.9 / 5.1-5.7 / 6.9-7.5 us,
#   against 4.5-4.8 / 5.3-6.0 / 7.6-8.4 with eight wavefronts of 64 tokens).
NARROW_WAVES = 4
NARROW_SPLIT_WAVES = 2
NARROW_SPLIT_WAVES_SMALL_GRID = 4  # partitions of >= 256 tokens on <= 128 workgroups
NARROW_SPLIT_MIN_SIZE = 128
NARROW_SPLIT_MIN_BYTES = 192 * 1024
NARROW_SPLIT_MIN_BYTES_WIDE = 256 * 1024
NARROW_SPLIT_WIDE_GRID = 64
NARROW_TOKENS_PER_WAVE = 64
# Narrow split-KV calls of at least this context and 2..64 rows size their
# partitions on the device from the rows' lengths (balanced_geometry); the
# compact grid holds one workgroup per compute unit, each partition streamed
# by BALANCED_WAVES wavefronts per kv head (config 3 on MI355X, one kv head
# per workgroup: 64.4-64.6 us with 2, 65.4-65.7 with 4, 67.7-68.2 with 6 or
# 8, 92.5 with 1; fixed 4096-token partitions with 4: 70.8-71.9).  A
# workgroup serves up to BALANCED_MAX_HEADS_PER_WG kv heads of a partition
# at once, so its wavefronts read whole token rows (one kv head's slice is
# a quarter or less of a row) and the partitions are that many times
# shorter (MI355X, graph-timed: config 3 64.4 -> 62.7 -> 61.8 us with 1, 2,
# 4 kv heads per workgroup; 8 x 16k 99.6 -> 91.5 with 2; 4 x 32k at 32/4
# heads, D 64 36.5 -> 31.1 with 2; 6 ragged rows of 8k-31k 75.9 -> 72.5).
BALANCED_MIN_CONTEXT = 8192
BALANCED_WAVES = 2
BALANCED_MAX_HEADS_PER_WG = 4
# Partitions of a caller-fixed size (set_attention_split_size, or
# attention_path="split_kv") are streamed by two wavefronts each, four
# above 768 tokens, all of them on every partition (measured on MI355X
# against one wavefront per partition, merge launch included: config 3 in
# the BASELINE's 512-token partitions 119.7 -> 85.1 us; config 2 at 256 /
# 512 / 1024 tokens 32.6 / 33.3 / 34.0 -> 27.0 / 25.1 / 24.3 us (2) and
# 25.9 (4 at 1024); 16 x 4096 and 4 x 2048 rows 10-30% faster).  Partitions
# of 512-768 tokens go to workgroups of two kv heads, so their wavefronts
# read whole token rows (config 3 at 512 tokens 76.1 -> 71.6 us, config 2
# 25.4 -> 24.5; at 256 tokens config 2 is 26.4 against 26.9, so shorter
# partitions keep one kv head per workgroup).
FIXED_SPLIT_WAVES = 2
FIXED_SPLIT_WAVES_WIDE = 4
FIXED_SPLIT_WIDE = 768
FIXED_SPLIT_PAIRED = 512
COMPUTE_UNITS = 256  # MI355X


@dataclass(frozen=True, slots=True)
class AttentionPlan:
    """Launch shape of one decode-attention call: one pass or split-KV
    (``num_splits`` partitions of ``split_size`` tokens and a merge), with
    ``waves_per_head`` wavefronts per (row, kv head, split), a row using one
    per ``tokens_per_wave`` of its tokens in the partition."""

    one_pass: bool
    split_size: int
    num_splits: int
    waves_per_head: int
    tokens_per_wave: int = ONE_PASS_TOKENS_PER_WAVE
    # Split-KV with partitions sized on the device from the rows' lengths
    # (TF_ATTENTION_FLAG_BALANCED): split_size is then the smallest partition
    # and num_splits the slots per group of heads_per_wg kv heads over all
    # rows together.
    balanced: bool = False
    # kv heads one workgroup serves (its wavefronts: heads_per_wg x
    # waves_per_head).
    heads_per_wg: int = 1

    @property
    def flags(self) -> int:
        """The C ABI's launch flags: several wavefronts per kv head (none for
        one), several kv heads per workgroup and the balanced partitions."""

        flags = _native.TF_ATTENTION_FLAG_BALANCED if self.balanced else 0
        if self.waves_per_head <= 1 and self.heads_per_wg <= 1:
            return flags
        return (flags | (self.heads_per_wg << _native.TF_ATTENTION_HEADS_PER_WG_SHIFT)
                | (self.waves_per_head << _native.TF_ATTENTION_WAVES_PER_CU_SHIFT)
                | ((self.tokens_per_wave // 64) << _native.TF_ATTENTION_TOKENS_PER_WAVE_SHIFT))


def wide_tokens_per_wave(max_context_length: int) -> int:
    """Token budget per wavefront of a wide one-pass call: 576 above 1536
    tokens (config 2's ragged rows up to 2k: four wavefronts for the
    longest), else about a quarter of the context and at least 128, so a
    row gets ~4 wavefronts (measured on MI355X with the fused RoPE + append
    at 64 rows: 512 tokens 9.5 us with 4 against 13.7 with 1; 1000 tokens
    16.3 us with 4 against 17.0 with 2)."""

    if max_context_length > 1536:
        return ONE_PASS_TOKENS_PER_WAVE
    return max(128, (-(-max_context_length // 4) + 63) // 64 * 64)


def narrow_one_pass_tokens(max_context_length: int, head_dim: int) -> int:
    """Token budget per wavefront of a narrow one-pass call: a row gets up to
    NARROW_WAVES wavefronts of max(64, head_dim, ceil64(context / 4))
    tokens."""

    quarter = (-(-max_context_length // NARROW_WAVES) + 63) // 64 * 64
    return max(NARROW_TOKENS_PER_WAVE, head_dim, quarter)


def narrow_split_plan(max_context_length: int, batch: int, kv_heads: int, head_dim: int,
                      element_bytes: int, slot_limit: int | None = None) -> AttentionPlan | None:
    """Split-KV launch of a narrow call, or None where one pass is faster.

    With R = rows x kv heads one-pass workgroups, the partitions aim at
    about COMPUTE_UNITS workgroups: round(COMPUTE_UNITS x pair / R) per row,
    where pair = 2 when kv heads can pair up (an even count whose slice of a
    token row is narrower than 256 bytes) and a workgroup then serves two kv
    heads of its partition once the unpaired grid would exceed the compute
    units.  Partitions are of equal size (a multiple of 32 tokens, at least
    NARROW_SPLIT_MIN_SIZE), as many per row as the workspace's partials per
    (row, query head) allow (``slot_limit``).  Two wavefronts per partition,
    four for partitions of >= 256 tokens on at most 128 workgroups.  One
    pass instead when a (row, kv head) holds less than NARROW_SPLIT_MIN_BYTES
    of K and V (NARROW_SPLIT_MIN_BYTES_WIDE above 64 one-pass workgroups), or
    when a row would not take two partitions."""

    rows_heads = max(batch, 1) * kv_heads
    row_bytes = 2 * max_context_length * head_dim * element_bytes
    floor_bytes = (NARROW_SPLIT_MIN_BYTES if rows_heads <= NARROW_SPLIT_WIDE_GRID
                   else NARROW_SPLIT_MIN_BYTES_WIDE)
    if row_bytes < floor_bytes:
        return None
    pair = 2 if kv_heads % 2 == 0 and head_dim * element_bytes < 256 else 1
    target = max(1, round(COMPUTE_UNITS * pair / rows_heads))
    if slot_limit is not None:
        target = min(target, slot_limit)
    size = max(NARROW_SPLIT_MIN_SIZE, (-(-max_context_length // max(target, 1)) + 31) // 32 * 32)
    splits = -(-max_context_length // size)
    if splits < 2:
        return None
    units = rows_heads * splits
    heads = pair if units > COMPUTE_UNITS else 1
    waves = (NARROW_SPLIT_WAVES_SMALL_GRID if units <= COMPUTE_UNITS // 2 and size >= 256
             else NARROW_SPLIT_WAVES)
    return AttentionPlan(False, size, splits, waves, NARROW_TOKENS_PER_WAVE,
                         heads_per_wg=heads)


def balanced_geometry(max_context_length: int, batch: int, kv_heads: int,
                      slot_limit: int | None = None) -> tuple[int, int]:
    """Slots and kv heads per workgroup of a balanced split-KV call, or
    (0, 1) where the call keeps fixed partitions.

    A workgroup serves ``heads_per_wg`` kv heads of one partition (the
    largest of BALANCED_MAX_HEADS_PER_WG, ..., 2, 1 that divides kv_heads
    and fits), and there is one slot per compute unit and group of kv heads
    (``COMPUTE_UNITS * heads_per_wg // kv_heads``), so the compact grid is
    one workgroup per compute unit.  Only for 2..64 rows of at least
    BALANCED_MIN_CONTEXT tokens, where rows of unequal length leave fixed
    partitions unevenly spread (config 3: rows of 8k..32k in 4096-token
    partitions give 160 of 256 workgroups work); the slots must outnumber
    the rows (the device-side partition size needs it) and fit the
    workspace, whose partials keep the fixed-partition layout ([row][query
    head][slot]): ``slot_limit`` slots per (row, query head), by default one
    per 256 tokens of the context, what the workspace the reference sizes
    for 256-token partitions holds."""

    if batch < 2 or batch > 64 or max_context_length < BALANCED_MIN_CONTEXT:
        return 0, 1
    limit = (-(-max_context_length // REFERENCE_SPLIT_SIZE) if slot_limit is None
             else slot_limit)
    heads = BALANCED_MAX_HEADS_PER_WG
    while heads >= 1:
        if kv_heads % heads == 0:
            slots = COMPUTE_UNITS * heads // max(kv_heads, 1)
            if batch < slots <= limit:
                return slots, heads
        heads //= 2
    return 0, 1


def balanced_slots_for(max_context_length: int, batch: int, kv_heads: int) -> int:
    """Slots per group of kv heads of a balanced split-KV call, or 0 where
    the call keeps fixed partitions (balanced_geometry)."""

    return balanced_geometry(max_context_length, batch, kv_heads)[0]


def attention_plan(launch_context: int, batch: int, kv_heads: int, context_capacity: int,
                   attention_path: str = "auto", slot_limit: int | None = None, *,
                   head_dim: int = 64, element_bytes: int = 2) -> AttentionPlan:
    """The launch of a call from host-known sizes only.

    The reference runs one pass unless the batch has few programs
    (``triton_attention.py:400-404``: split-KV only for contexts >= 1024 with
    batch * query heads <= 32).  Here (measured on MI355X, TinyLlama
    geometry unless noted):

    * at least 192 (row, kv head) workgroups and no caller-fixed partition
      size: one pass, each workgroup splitting its row over up to 8
      wavefronts (one per wide_tokens_per_wave tokens of the row) that
      combine in LDS -- no partials, no merge launch (72 rows x 4 kv heads
      x 2k: 21.3 us against 26.0 us for split 576 plus merge);
    * fewer workgroups: for 2..64 rows of >= 8k the balanced partitions of
      balanced_geometry, sized on the device from the rows' lengths, with
      up to four kv heads per workgroup and two wavefronts per kv head
      (config 3: 58.7 us, against 70.8 for fixed 4096-token partitions);
      otherwise split-KV by narrow_split_plan where a row's K and V are
      large enough to pay for the merge launch, else one pass with up to
      four wavefronts per kv head (narrow_one_pass_tokens);
    * a partition size fixed by the caller (set_attention_split_size) or
      ``attention_path="split_kv"``: split-KV (size attention_split_size_for
      unless fixed) with two wavefronts per partition, four above 768
      tokens; ``"one_pass"`` forces one pass.

    ``slot_limit`` is the number of partials per (row, query head) the
    workspace holds (None: no limit beyond the plan's own); ``head_dim`` and
    ``element_bytes`` size a token row's slice per kv head.
    """

    fixed = _SPLIT_SIZE is not None
    split_size = (_SPLIT_SIZE if fixed
                  else attention_split_size_for(launch_context, batch, kv_heads))
    workgroups = batch * kv_heads
    capacity32 = (context_capacity + 31) // 32 * 32
    if fixed or attention_path == "split_kv":
        if attention_path == "one_pass" or (attention_path == "auto"
                                            and launch_context <= split_size):
            return AttentionPlan(True, capacity32, 1, 1)
        waves = FIXED_SPLIT_WAVES if split_size <= FIXED_SPLIT_WIDE else FIXED_SPLIT_WAVES_WIDE
        heads = 2 if FIXED_SPLIT_PAIRED <= split_size <= FIXED_SPLIT_WIDE and kv_heads % 2 == 0 else 1
        return AttentionPlan(False, split_size, (launch_context + split_size - 1) // split_size,
                             waves, 0, heads_per_wg=heads)
    if workgroups >= ONE_PASS_MIN_WORKGROUPS:
        tokens = wide_tokens_per_wave(launch_context)
        waves = max(1, min(8, -(-launch_context // tokens)))
        return AttentionPlan(True, capacity32, 1, waves, tokens)
    narrow_tokens = narrow_one_pass_tokens(launch_context, head_dim)
    one_pass = AttentionPlan(True, capacity32, 1,
                             max(1, min(NARROW_WAVES, -(-launch_context // narrow_tokens))),
                             narrow_tokens)
    if attention_path == "one_pass":
        return one_pass
    slots, heads = balanced_geometry(launch_context, batch, kv_heads, slot_limit)
    if slots:
        smallest = (-(-launch_context // slots) + 63) // 64 * 64
        return AttentionPlan(False, smallest, slots, BALANCED_WAVES, NARROW_TOKENS_PER_WAVE,
                             balanced=True, heads_per_wg=heads)
    split = narrow_split_plan(launch_context, batch, kv_heads, head_dim, element_bytes, slot_limit)
    return split if split is not None else one_pass


def paged_gqa_decode_attention(
    query: Tensor,
    key_cache: Tensor,
    value_cache: Tensor,
    block_tables: Tensor,
    context_lengths: Tensor,
    *,
    scale: float | None = None,
    max_context_length: int | None = None,
    output: Tensor | None = None,
    workspace: PagedAttentionWorkspace | None = None,
    attention_path: str = "auto",
) -> Tensor:
    """Attend one query token per sequence over logically ordered physical KV pages.

    Mirrors ``triton_attention.py:326-518``.  Differences, all on inputs the
    reference leaves undefined: rows with ``context_lengths <= 0`` produce
    zeros (reference: 0/0); tokens whose block-table entry lies outside the
    cache are skipped instead of read out of bounds.
    """

    global _LAST_ATTENTION_CONFIG, _LAST_ATTENTION_LAUNCH
    if not _native.is_available():
        raise RuntimeError(
            "the gfx950 attention library is unavailable; build it with "
            "`python -m tensorforge_amd.build`"
        )
    tensors = (query, key_cache, value_cache, block_tables, context_lengths)
    if any(not tensor.is_cuda for tensor in tensors):
        raise ValueError("paged GQA attention requires CUDA tensors")
    if any(not tensor.is_contiguous() for tensor in tensors):
        raise ValueError("paged GQA attention requires contiguous tensors")
    if query.ndim != 3:
        raise ValueError("query must have shape [batch, query_heads, head_dim]")
    if key_cache.ndim != 4 or value_cache.shape != key_cache.shape:
        raise ValueError("key/value cache must share [blocks, block_size, kv_heads, head_dim]")
    if query.dtype not in _native.DTYPE_CODES:
        raise TypeError(f"unsupported query dtype: {query.dtype}")
    if key_cache.dtype != query.dtype or value_cache.dtype != query.dtype:
        raise ValueError("query, key cache, and value cache must share dtype")
    if block_tables.dtype != torch.int32 or context_lengths.dtype != torch.int32:
        raise TypeError("block tables and context lengths must use torch.int32")
    batch, query_heads, head_dim = query.shape
    num_blocks, block_size, kv_heads, cache_head_dim = key_cache.shape
    if head_dim != cache_head_dim or query_heads % kv_heads != 0:
        raise ValueError("query/cache head dimensions do not form valid GQA groups")
    if head_dim > 256:
        raise ValueError("decode attention supports head dimensions up to 256")
    if block_tables.ndim != 2 or block_tables.shape[0] != batch:
        raise ValueError("block_tables must have one row per query")
    if context_lengths.shape != (batch,):
        raise ValueError("context_lengths must have one value per query")
    if query.requires_grad and torch.is_grad_enabled():
        raise RuntimeError("TensorForge HIP kernels are inference-only")
    if attention_path not in {"auto", "one_pass", "split_kv"}:
        raise ValueError("attention_path must be auto, one_pass, or split_kv")

    table_width = block_tables.shape[1]
    context_capacity = table_width * block_size
    if max_context_length is None:
        # Host synchronisation, as in the reference (:375); give a bucket to
        # keep the call capture-safe.
        launch_context = int(context_lengths.max().item()) if batch > 0 else 0
        if launch_context <= 0:
            raise ValueError("context lengths must be positive")
    else:
        launch_context = max_context_length
    if launch_context <= 0 or launch_context > context_capacity:
        raise ValueError("max_context_length must be positive and within table capacity")
    head_bucket = _next_power_of_2(head_dim)
    if output is None:
        output = torch.empty_like(query)
    elif (
        output.shape != query.shape
        or output.dtype != query.dtype
        or output.device != query.device
        or not output.is_contiguous()
    ):
        raise ValueError("output must be contiguous and share query shape, dtype, and device")
    attention_scale = head_dim**-0.5 if scale is None else scale

    # Balanced partitions may take as many slots as the partials' workspace
    # holds per (row, query head): the caller's, or the one allocated below.
    if workspace is not None:
        slot_limit = min(workspace.partial_max.numel(), workspace.partial_sum.numel(),
                         workspace.partial_accumulator.shape[0]) // max(batch * query_heads, 1)
    else:
        slot_limit = COMPUTE_UNITS * BALANCED_MAX_HEADS_PER_WG
    plan = attention_plan(launch_context, batch, kv_heads, context_capacity, attention_path,
                          slot_limit, head_dim=head_dim, element_bytes=query.element_size())
    use_split_kv = not plan.one_pass
    split_size = plan.split_size
    dtype = _native.dtype_code(query.dtype)
    group = query_heads // kv_heads
    variant = _native.library().tf_paged_gqa_decode_variant(dtype, head_dim, group, block_size, 0)
    kernel = "mfma" if variant == _native.TF_ATTENTION_MFMA else "generic"
    if plan.balanced and kernel != "mfma":
        # The generic kernel takes fixed partitions: the same slots of the
        # smallest size still cover the context.
        plan = dataclasses.replace(plan, balanced=False, heads_per_wg=1)
    device = query.device
    stream = _native.current_stream(device)
    counters_ptr = None
    if use_split_kv:
        num_splits = plan.num_splits
        partial_programs = batch * query_heads * num_splits
        if workspace is None:
            workspace = PagedAttentionWorkspace.allocate(
                batch_capacity=max(batch, 1),
                query_heads=query_heads,
                head_dim=head_dim,
                max_context_length=num_splits * REFERENCE_SPLIT_SIZE,
                device=device,
            )
        if (
            workspace.partial_max.device != device
            or workspace.partial_sum.device != device
            or workspace.partial_accumulator.device != device
            or workspace.partial_max.dtype != torch.float32
            or workspace.partial_sum.dtype != torch.float32
            or workspace.partial_accumulator.dtype != torch.float32
            or workspace.partial_max.numel() < partial_programs
            or workspace.partial_sum.numel() < partial_programs
            or workspace.partial_accumulator.shape[0] < partial_programs
            or workspace.partial_accumulator.shape[1] != head_bucket
            or not workspace.partial_max.is_contiguous()
            or not workspace.partial_sum.is_contiguous()
            or not workspace.partial_accumulator.is_contiguous()
        ):
            raise ValueError("split-KV workspace has insufficient or incompatible capacity")
        capacity = min(
            workspace.partial_max.numel(),
            workspace.partial_sum.numel(),
            workspace.partial_accumulator.shape[0],
        )
        # The partials are merged by a second launch: measured faster on
        # MI355X than the in-kernel merge that the workspace's arrival
        # counters enable (the C ABI keeps both).
        counters_ptr = None
        _native.check(
            _native.library().tf_paged_gqa_decode(
                query.data_ptr(),
                key_cache.data_ptr(),
                value_cache.data_ptr(),
                block_tables.data_ptr(),
                context_lengths.data_ptr(),
                output.data_ptr(),
                workspace.partial_max.data_ptr(),
                workspace.partial_sum.data_ptr(),
                workspace.partial_accumulator.data_ptr(),
                counters_ptr,
                capacity,
                head_bucket,
                batch,
                query_heads,
                kv_heads,
                head_dim,
                num_blocks,
                block_size,
                table_width,
                split_size,
                num_splits,
                attention_scale,
                dtype,
                plan.flags,
                stream,
            ),
            "paged_gqa_decode_attention",
        )
        # The reference's record, key for key (triton_attention.py:475-479;
        # its test compares it with ==); launch details go to
        # selected_attention_launch().
        _LAST_ATTENTION_CONFIG = {
            "path": "split_kv",
            "split_size": split_size,
            "num_splits": num_splits,
        }
    else:
        # One partition spanning the whole table: every present token of a
        # row is visited by one workgroup per (row, kv head), split over its
        # plan.waves_per_head wavefronts.
        one_pass_size = plan.split_size
        num_splits = 1
        _native.check(
            _native.library().tf_paged_gqa_decode(
                query.data_ptr(),
                key_cache.data_ptr(),
                value_cache.data_ptr(),
                block_tables.data_ptr(),
                context_lengths.data_ptr(),
                output.data_ptr(),
                None,
                None,
                None,
                None,
                0,
                head_bucket,
                batch,
                query_heads,
                kv_heads,
                head_dim,
                num_blocks,
                block_size,
                table_width,
                one_pass_size,
                1,
                attention_scale,
                dtype,
                plan.flags,
                stream,
            ),
            "paged_gqa_decode_attention",
        )
        _LAST_ATTENTION_CONFIG = {
            "path": "one_pass",
            "kernel": kernel,
            "workgroup": "sequence x kv_head",
        }
    heads = plan.heads_per_wg if kernel == "mfma" else 1
    _LAST_ATTENTION_LAUNCH = {
        "kernel": kernel,
        "waves_per_head": plan.waves_per_head if kernel == "mfma" else 1,
        "grid": ((kv_heads // heads * num_splits, 1) if use_split_kv and plan.balanced
                 else (batch * kv_heads // heads, num_splits)),
        "heads_per_workgroup": heads,
        "in_kernel_merge": bool(use_split_kv and counters_ptr is not None),
        "balanced_partitions": bool(use_split_kv and plan.balanced),
        "group_size": group,
        "launch_context": launch_context,
    }
    return output


def paged_gqa_decode_attention_rope_append(
    qkv: Tensor,
    positions: Tensor,
    cos_table: Tensor,
    sin_table: Tensor,
    key_cache: Tensor,
    value_cache: Tensor,
    append_pages: Tensor,
    append_offsets: Tensor,
    active_mask: Tensor,
    block_tables: Tensor,
    context_lengths: Tensor,
    *,
    query_heads: int,
    max_context_length: int,
    output: Tensor,
    workspace: PagedAttentionWorkspace,
    scale: float | None = None,
) -> Tensor:
    """The decode step's RoPE, KV append and attention in one launch.

    ``qkv [batch, (query_heads + 2 * kv_heads) * head_dim]`` holds the
    unrotated projections (rows may be strided).  Each attention workgroup
    rotates its query group at ``positions`` and writes the row's rotated
    key and its value into slot (``append_pages``, ``append_offsets``) when
    ``active_mask`` is set, then attends over ``context_lengths`` tokens
    (which count the new one).  The same results as
    :func:`tensorforge_amd.kernels.rope_paged_kv_append` followed by
    :func:`paged_gqa_decode_attention` (the rotation is computed by the same
    arithmetic); the plan (one pass or split-KV) is chosen as there.
    Replaces the decode step's RoPE (model/layers.py:57-69), cache write and
    attention call (runtime/decode_bucket.py:448-469).
    """

    if not _native.is_available():
        raise RuntimeError(
            "the gfx950 attention library is unavailable; build it with "
            "`python -m tensorforge_amd.build`"
        )
    tensors = (qkv, positions, cos_table, sin_table, key_cache, value_cache, append_pages,
               append_offsets, active_mask, block_tables, context_lengths, output)
    if any(not tensor.is_cuda for tensor in tensors):
        raise ValueError("paged GQA attention requires CUDA tensors")
    if qkv.ndim != 2 or qkv.stride(1) != 1:
        raise ValueError("qkv must be [batch, (q + 2 kv heads) * head_dim] with contiguous rows")
    if key_cache.ndim != 4 or value_cache.shape != key_cache.shape:
        raise ValueError("key/value cache must share [blocks, block_size, kv_heads, head_dim]")
    num_blocks, block_size, kv_heads, head_dim = key_cache.shape
    batch = qkv.shape[0]
    if qkv.shape[1] != (query_heads + 2 * kv_heads) * head_dim or query_heads % kv_heads:
        raise ValueError("qkv rows must hold query_heads + 2 * kv_heads heads of head_dim")
    if qkv.dtype not in (torch.float16, torch.bfloat16) or any(
            t.dtype != qkv.dtype for t in (key_cache, value_cache, cos_table, sin_table, output)):
        raise TypeError("fused RoPE attention takes fp16/bf16 qkv, tables, caches and output")
    if positions.dtype != torch.int64 or positions.shape != (batch,):
        raise ValueError("positions must be int64 [batch]")
    if cos_table.shape != sin_table.shape or cos_table.ndim != 2 or cos_table.shape[1] != head_dim:
        raise ValueError("cos/sin tables must be [positions, head_dim]")
    for name, tensor in (("append_pages", append_pages), ("append_offsets", append_offsets),
                         ("active_mask", active_mask), ("context_lengths", context_lengths)):
        if tensor.dtype != torch.int32 or tensor.shape != (batch,):
            raise ValueError(f"{name} must be int32 [batch]")
    if block_tables.dtype != torch.int32 or block_tables.ndim != 2 or block_tables.shape[0] != batch:
        raise ValueError("block_tables must be int32 with one row per query")
    if output.shape != (batch, query_heads, head_dim) or not output.is_contiguous():
        raise ValueError("output must be a contiguous [batch, query_heads, head_dim] tensor")
    table_width = block_tables.shape[1]
    context_capacity = table_width * block_size
    if max_context_length <= 0 or max_context_length > context_capacity:
        raise ValueError("max_context_length must be positive and within table capacity")
    capacity = min(workspace.partial_max.numel(), workspace.partial_sum.numel(),
                   workspace.partial_accumulator.shape[0])
    plan = attention_plan(max_context_length, batch, kv_heads, context_capacity,
                          slot_limit=capacity // max(batch * query_heads, 1), head_dim=head_dim,
                          element_bytes=qkv.element_size())
    head_bucket = _next_power_of_2(head_dim)
    partial_programs = batch * query_heads * plan.num_splits
    if not plan.one_pass and (capacity < partial_programs
                              or workspace.partial_accumulator.shape[1] != head_bucket):
        raise ValueError("split-KV workspace has insufficient or incompatible capacity")
    _native.check(
        _native.library().tf_paged_gqa_decode_rope_append(
            qkv.data_ptr(), qkv.stride(0), positions.data_ptr(), cos_table.data_ptr(),
            sin_table.data_ptr(), cos_table.shape[0], key_cache.data_ptr(),
            value_cache.data_ptr(), append_pages.data_ptr(), append_offsets.data_ptr(),
            active_mask.data_ptr(), block_tables.data_ptr(), context_lengths.data_ptr(),
            output.data_ptr(), workspace.partial_max.data_ptr(), workspace.partial_sum.data_ptr(),
            workspace.partial_accumulator.data_ptr(), None, capacity, head_bucket, batch,
            query_heads, kv_heads, head_dim, num_blocks, block_size, table_width,
            plan.split_size, plan.num_splits, head_dim**-0.5 if scale is None else scale,
            _native.dtype_code(qkv.dtype), plan.flags, _native.current_stream(qkv.device),
        ),
        "paged_gqa_decode_attention_rope_append",
    )
    return output


def selected_attention_autotune_config() -> dict[str, Any] | None:
    """Dispatch record of the last call (reference: triton_attention.py:521-522)."""

    return _LAST_ATTENTION_CONFIG


def selected_attention_launch() -> dict[str, Any] | None:
    """Launch details of the last call (no reference counterpart): the
    kernel family ("mfma" or "generic"), ``waves_per_head`` (wavefronts per
    kv head), ``heads_per_workgroup`` (kv heads one workgroup serves),
    ``grid`` (workgroups as (x, y)), ``balanced_partitions`` (partition
    size set on the device), ``in_kernel_merge``, ``group_size`` and
    ``launch_context``."""

    return _LAST_ATTENTION_LAUNCH
