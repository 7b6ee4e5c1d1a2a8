"""Address-level emulation, on the CPU, of the fused RoPE + append + attention
launch's load schedule (csrc/tf_paged_attention.hip, paged_decode_mfma_kernel
with ROPE): which cache lines each wavefront's K/V loads touch, chunk by
chunk, against the lines of the token rows the launch appends.

The fused launch is correct only if no compute unit holds a line of an
appended token row in its L1 from before that row's store reached L2.  Its
argument: every wavefront of a row writes the whole appended row and waits
for its own stores before its first K/V load, and nothing else reads a line
of an appended row before that.  The restatement below follows the kernel's
indexing (grid, chunk deal, whole-row loads, stand-in rows) and checks that
argument for the geometries the GPU test runs, including the head_dim-32
case where two kv heads share a cache line.

It also checks a variant that was tried and is not shipped: issuing each
wavefront's first two chunks before the append when neither holds the new
token.  The emulation shows that those early loads touch no appended line in
any of these geometries, so an address overlap does not explain the
differing results that variant gave.  (The same last-bit symptom came back
with another change of the launch's prologue and went away when the
wavefronts' combine was written with explicit fused multiply-adds: the
compiler had fused a different product of `x * a + y * c` in the fused and
the plain kernel; see the note in the kernel source.)
"""

from __future__ import annotations

import math

import pytest
import torch

from tensorforge_amd.kernels.attention import attention_plan
from tensorforge_amd.workloads import make_decode_attention_case

LINE = 128          # bytes per cache line (gfx950 L1 and L2)
CHUNK = 32          # tokens per wavefront step: two 16-token tiles
SEGMENT_TILES = 64  # tiles per page window (1024 tokens)


def _wide_lengths(hq: int, hkv: int, d: int) -> list[int]:
    """The "wide" lengths of tests/test_gpu_rope_attention.py."""

    generator = torch.Generator().manual_seed(hq + d)
    count = max(48, -(-192 // hkv))
    lengths = [int(x) for x in torch.randint(1, 700, (count,), generator=generator)]
    lengths[3] = 0
    lengths[7] = 1
    return lengths


def _schedule(ctx: int, waves_per_head: int, tokens_per_wave: int, sub: int) -> list[int]:
    """Chunk indices (segment-relative, one segment here) that wavefront
    `sub` of a (row, kv head) streams, in order: sub + i * active."""

    active = waves_per_head
    if tokens_per_wave > 0:
        active = min(max(-(-ctx // tokens_per_wave), 1), waves_per_head)
    chunks = -(-ctx // CHUNK)
    if sub >= active or chunks <= sub:
        return []
    mine = (chunks - sub + active - 1) // active
    return [sub + i * active for i in range(mine)]


def _chunk_lines(chunk: int, ctx: int, table: list[int], block_size: int, kv_heads: int,
                 head_dim: int, elem: int, kvh: int) -> set[int]:
    """Cache lines of the key cache read by one chunk of one wavefront in
    the whole-row load form: for tile j, lane piece p of token tt reads 16
    bytes at token tt (absent tokens of a present tile read the tile's
    first token); absent tiles read the row's QKV input (not a cache page,
    so no line of the key cache)."""

    token_bytes = kv_heads * head_dim * elem
    head_bytes = kvh * head_dim * elem
    lines: set[int] = set()
    for j in range(2):
        t0 = chunk * CHUNK + 16 * j
        page = table[t0 // block_size] if t0 < ctx else -1
        if t0 >= ctx or page < 0:
            continue
        ntok = min(16, ctx - t0)
        in_page = t0 % block_size
        base = (page * block_size + in_page) * token_bytes + head_bytes
        for tt in range(16):
            offset = (tt if tt < ntok else 0) * token_bytes
            for piece in range(head_dim * elem // 16):
                address = base + offset + 16 * piece
                lines.add(address // LINE)
    return lines


def _appended_lines(ctx: int, table: list[int], block_size: int, kv_heads: int, head_dim: int,
                    elem: int) -> set[int]:
    token_bytes = kv_heads * head_dim * elem
    position = ctx - 1
    start = (table[position // block_size] * block_size + position % block_size) * token_bytes
    return set(range(start // LINE, (start + token_bytes - 1) // LINE + 1))


GEOMETRIES = [(32, 4, 64, torch.bfloat16), (8, 2, 32, torch.float16),
              (32, 8, 128, torch.bfloat16), (16, 1, 64, torch.float16)]


@pytest.mark.parametrize(("hq", "hkv", "d", "dtype"), GEOMETRIES)
def test_no_load_reads_an_appended_line_before_its_own_wavefront_wrote_it(hq, hkv, d, dtype):
    lengths = _wide_lengths(hq, hkv, d)
    case = make_decode_attention_case(lengths, query_heads=hq, kv_heads=hkv, head_dim=d,
                                      block_size=16, dtype=dtype, seed=len(lengths) + d,
                                      extra_pages=4)
    plan = attention_plan(max(lengths), len(lengths), hkv, max(lengths))
    assert plan.one_pass and plan.waves_per_head > 1  # the wide plan: whole-row loads
    elem = torch.empty((), dtype=dtype).element_size()
    tables = case.block_tables.tolist()
    appended = {}
    for row, ctx in enumerate(lengths):
        if ctx > 0:
            appended[row] = _appended_lines(ctx, tables[row], 16, hkv, d, elem)
    all_appended = set().union(*appended.values())
    # Appended rows of different rows never share a line (tables are disjoint).
    assert sum(len(v) for v in appended.values()) == len(all_appended)
    early_hits = 0
    for row, ctx in enumerate(lengths):
        if ctx == 0:
            continue
        new_chunk = (ctx - 1) // CHUNK
        covered: list[int] = []
        for kvh in range(hkv):
            for sub in range(plan.waves_per_head):
                chunks = _schedule(ctx, plan.waves_per_head, plan.tokens_per_wave, sub)
                if kvh == 0:
                    covered += chunks
                for index, chunk in enumerate(chunks):
                    lines = _chunk_lines(chunk, ctx, tables[row], 16, hkv, d, elem, kvh)
                    # Shipped order: every load follows this wavefront's own
                    # whole-row store and wait, so the only appended lines it
                    # may read are its own row's, in the chunk of the new token.
                    foreign = (lines & all_appended) - appended[row]
                    assert not foreign, (row, kvh, sub, chunk)
                    if lines & appended[row]:
                        assert chunk == new_chunk, (row, kvh, sub, chunk)
                    # The tried variant: chunks 0 and 1 of the schedule issued
                    # before the store when neither is the new token's chunk.
                    early = chunks[:2]
                    if index < 2 and new_chunk not in early:
                        early_hits += len(lines & all_appended)
        # The chunk deal covers every chunk of the row exactly once.
        assert sorted(covered) == list(range(math.ceil(ctx / CHUNK))), row
    assert early_hits == 0
