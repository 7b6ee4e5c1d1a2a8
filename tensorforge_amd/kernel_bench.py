"""Per-kernel timing of the decode hot path on one GPU.

``python -m tensorforge_amd.kernel_bench`` prints one JSON line per case:

* config 4 -- residual+RMSNorm and RMSNorm at T in {1, 8, 64, 256} tokens x
  H in {2048, 4096} (eps 1e-5, weight N(1, 0.1)), SwiGLU at T x F in
  {5632, 14336}, and the paged KV append of T tokens x 4 kv heads x 64
  through ``PagedKVCache.write_layer`` starting mid-page, all bf16;
* config 3 -- paged GQA decode attention at Llama-3-8B geometry (4 rows of
  8k/16k/24k/32k, 32/8 heads, head_dim 128), split size chosen per call;
* decode steps -- one whole graph-captured decode step of the config-1
  model (4 layers, d_model 256, fp16) at batch {1, 4, 8} x context
  {32, 128, 512, 2048}, the grid of the reference's decode-step report
  (results/reference/phase7a-rtx3080ti-wsl/execution.md); device time per
  step from HIP events, and host-inclusive time per step of the pipelined
  launch/collect loop;
* ceiling -- what bounds the config-2 attention call: the graph launch gap,
  a fit of time against bytes over uniform-length batches (fixed cost per
  call and marginal rate), config 2 on random and on contiguous pages, one
  compute unit's rate with 1..8 wavefronts per kv head and with the read
  probe alone, and the page-gather probe over config 2's own pages;
* valu (only with ``--only valu``) -- the attention kernel's products on
  MFMA against its VALU form, at config 2's lengths with group 8 and 4;
* step_projections (only with ``--only step_projections``) -- the four
  projections of a 64-row decode step in the forms the executor launches
  (norm and residual epilogues, gate|up + SwiGLU), for their rates and
  their HBM counters;
* projections -- the decode step's projections at TinyLlama shapes and 1 /
  16 / 64 rows (weights rotated through HBM): hipBLASLt against the paths
  the decode bucket takes (linear_kstream for qkv, linear_stream partials
  for o / down, the K-split gate|up + SwiGLU, linear_stream for the LM
  head), plus the attention plans of narrow calls against one wavefront per
  256-token partition.

Each case is captured as ``--calls`` launches in one HIP graph and timed by
HIP events around one replay (a ctypes call costs the host longer than these
kernels take).  Rates use the algorithmic byte models of
``tensorforge_amd.workloads`` (the reference's models,
benchmark/kernel_benchmark.py:144-158 and attention_benchmark.py:148-161).
At decode token counts the fused ops are launch-bound: their time is
dominated by the launch and the kernel's fixed start-up, not by HBM.
"""

from __future__ import annotations

import argparse
import json
from typing import Callable

import torch

from tensorforge_amd import workloads
from tensorforge_amd.cache import PagedKVCache, PagedKVCacheConfig
from tensorforge_amd.decode import (
    BucketedDecodeExecutor,
    DecoderWeights,
    small_config,
    tinyllama_config,
)
from tensorforge_amd.kernels import (
    PagedAttentionWorkspace,
    linear_kstream,
    linear_rows,
    linear_stream,
    linear_swiglu,
    paged_gqa_decode_attention,
    residual_rms_norm,
    rms_norm,
    selected_attention_autotune_config,
    selected_attention_launch,
    set_attention_split_size,
    swiglu,
    swiglu_gate_up,
)
from tensorforge_amd.kernels.linear import default_splits

HBM_PEAK_GBS = 8000.0


def graph_time_us(run: Callable[[int], None], calls: int, device: torch.device) -> float:
    """Average time per call of `calls` captured calls, replayed once."""

    stream = torch.cuda.Stream(device)
    stream.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(stream):
        for i in range(3):
            run(i)
    torch.cuda.current_stream(device).wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(calls):
            run(i)
    graph.replay()
    torch.cuda.synchronize()
    begin = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    begin.record()
    graph.replay()
    end.record()
    torch.cuda.synchronize()
    return begin.elapsed_time(end) * 1e3 / calls


def report(case: str, us: float, nbytes: int, **extra) -> dict:
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"case": case, "us_per_call": round(us, 3), "algorithmic_bytes": nbytes,
            "GB/s": round(gbs, 1), "hbm_fraction": round(gbs / HBM_PEAK_GBS, 4), **extra}


def config4(device: torch.device, calls: int) -> list[dict]:
    """Config 4 cases, each a dict with its shape under "shape"."""

    results = []
    generator = torch.Generator().manual_seed(0)
    dtype = torch.bfloat16

    def randn(*shape, mean=0.0, std=1.0):
        return (torch.randn(*shape, generator=generator) * std + mean).to(dtype).to(device)

    for hidden in (2048, 4096):
        weight = randn(hidden, mean=1.0, std=0.1)
        for tokens in (1, 8, 64, 256):
            x, r = randn(tokens, hidden), randn(tokens, hidden)
            res_out, norm_out = torch.empty_like(x), torch.empty_like(x)
            us = graph_time_us(lambda i: residual_rms_norm(
                x, r, weight, 1e-5, residual_output=res_out, norm_output=norm_out), calls, device)
            results.append(report(f"residual_rms_norm T={tokens} H={hidden}", us,
                                  workloads.rms_norm_bytes(tokens, hidden, 2, residual=True),
                                  shape={"op": "residual_rms_norm", "tokens": tokens,
                                         "hidden": hidden}))
            out = torch.empty_like(x)
            us = graph_time_us(lambda i: rms_norm(x, weight, 1e-5, output=out), calls, device)
            results.append(report(f"rms_norm T={tokens} H={hidden}", us,
                                  workloads.rms_norm_bytes(tokens, hidden, 2, residual=False),
                                  shape={"op": "rms_norm", "tokens": tokens, "hidden": hidden}))
    for ffn in (5632, 14336):
        for tokens in (1, 8, 64, 256):
            gate, up = randn(tokens, ffn), randn(tokens, ffn)
            out = torch.empty_like(gate)
            us = graph_time_us(lambda i: swiglu(gate, up, output=out), calls, device)
            results.append(report(f"swiglu T={tokens} F={ffn}", us,
                                  workloads.swiglu_bytes(tokens * ffn, 2),
                                  shape={"op": "swiglu", "tokens": tokens, "ffn": ffn}))
    for tokens in (1, 8, 64, 256):
        config = PagedKVCacheConfig(num_layers=1, num_blocks=64, block_size=16, num_kv_heads=4,
                                    head_dim=64, max_sequences=1, max_sequence_length=1024,
                                    dtype=dtype, device=device)
        cache = PagedKVCache(config)
        cache.create_sequence("s")
        head = cache.begin_append("s", 5)  # the timed append starts mid-page
        cache.record_layer_write(head, 0)
        cache.commit(head)
        reservation = cache.begin_append("s", tokens)
        keys, values = randn(tokens, 4, 64), randn(tokens, 4, 64)
        us = graph_time_us(lambda i: cache.write_layer(reservation, 0, keys, values), calls,
                           device)
        results.append(report(f"kv_append T={tokens} (4 x 64, 16-token pages, straddling)", us,
                              workloads.kv_append_bytes(tokens, 4, 64, 2),
                              shape={"op": "kv_append", "tokens": tokens}))
    return results


def config3(device: torch.device, calls: int) -> list[dict]:
    """Config 3 (4 rows of 8k..32k at Llama-3-8B geometry) six ways: the
    entry point's plan (balanced partitions sized on the device from the
    rows' lengths, two wavefronts each, merge launch); the BASELINE's form,
    512-token partitions and a separate log-sum-exp merge launch (the entry
    point with the partition size fixed at 512, as the reference's
    split_size argument fixes it, two wavefronts per partition), the same
    partitions with one wavefront each, and with the in-kernel merge (the
    C ABI with the workspace's arrival counters: the last partition of each
    (row, kv head) merges); and fixed 4096-token
    partitions with four wavefronts each (the plan before the balanced
    partitions) with the merge launch and with the in-kernel merge."""

    from tensorforge_amd import _native

    case = workloads.llama3_long_context_case(seed=0)
    pools = [case.to(device) for _ in range(2)]  # 2 x 671 MB: the MALL cannot hold them
    batch, query_heads, head_dim = case.query.shape
    num_blocks, block_size, kv_heads, _ = case.key_cache.shape
    width = case.block_tables.shape[1]
    workspace = PagedAttentionWorkspace.allocate(
        batch_capacity=batch, query_heads=query_heads, head_dim=head_dim,
        max_context_length=32768, device=device)
    output = torch.empty_like(pools[0].query)
    nbytes = workloads.decode_attention_bytes(case.lengths, query_heads, kv_heads, head_dim,
                                              block_size, 2)
    name = "paged_gqa_decode cfg3 (4 x 8k..32k, 32/8 heads, D128, bf16)"
    results = []

    def entry(i: int) -> None:
        gpu = pools[i % 2]
        paged_gqa_decode_attention(gpu.query, gpu.key_cache, gpu.value_cache, gpu.block_tables,
                                   gpu.context_lengths, scale=case.scale,
                                   max_context_length=32768, output=output, workspace=workspace)

    us = graph_time_us(entry, calls, device)
    tuned = dict(selected_attention_autotune_config() or {})
    launch = selected_attention_launch() or {}
    results.append(report(f"{name}, entry point plan (balanced partitions, "
                          f"{launch.get('heads_per_workgroup')} kv heads per workgroup, "
                          f"{launch.get('waves_per_head')} wavefronts each), merge launch", us,
                          nbytes, record=tuned))

    previous = set_attention_split_size(512)
    try:
        us = graph_time_us(entry, calls, device)
        launch = selected_attention_launch() or {}
        results.append(report(f"{name}, 512-token partitions ({launch.get('heads_per_workgroup')} "
                              f"kv heads per workgroup, {launch.get('waves_per_head')} "
                              f"wavefronts each), merge launch (BASELINE form)", us,
                              nbytes, record=dict(selected_attention_autotune_config() or {})))
    finally:
        set_attention_split_size(previous)

    capacity = workspace.partial_max.numel()
    fixed_flags = ((1 << _native.TF_ATTENTION_HEADS_PER_WG_SHIFT)
                   | (4 << _native.TF_ATTENTION_WAVES_PER_CU_SHIFT)
                   | (1 << _native.TF_ATTENTION_TOKENS_PER_WAVE_SHIFT))
    two_waves = ((1 << _native.TF_ATTENTION_HEADS_PER_WG_SHIFT)
                 | (2 << _native.TF_ATTENTION_WAVES_PER_CU_SHIFT))
    for split, flags, in_kernel, label in (
            (512, 0, False, "512-token partitions, 1 wavefront each, merge launch"),
            (512, two_waves, True, "512-token partitions, 2 wavefronts each, in-kernel merge"),
            (4096, fixed_flags, False, "fixed 4096-token partitions, 4 wavefronts each, "
                                       "merge launch"),
            (4096, fixed_flags, True, "fixed 4096-token partitions, 4 wavefronts each, "
                                      "in-kernel merge")):
        splits = -(-32768 // split)
        counters = workspace.split_counters.data_ptr() if in_kernel else None

        def raw(i: int, split=split, splits=splits, flags=flags, counters=counters) -> None:
            gpu = pools[i % 2]
            _native.check(_native.library().tf_paged_gqa_decode(
                gpu.query.data_ptr(), gpu.key_cache.data_ptr(), gpu.value_cache.data_ptr(),
                gpu.block_tables.data_ptr(), gpu.context_lengths.data_ptr(), output.data_ptr(),
                workspace.partial_max.data_ptr(), workspace.partial_sum.data_ptr(),
                workspace.partial_accumulator.data_ptr(), counters,
                capacity, workspace.partial_accumulator.shape[1], batch, query_heads, kv_heads,
                head_dim, num_blocks, block_size, width, split, splits, case.scale,
                _native.dtype_code(case.query.dtype), flags, _native.current_stream(device)),
                "tf_paged_gqa_decode")

        us = graph_time_us(raw, calls, device)
        results.append(report(f"{name}, {label}", us, nbytes))
    return results


def attention_ceiling(device: torch.device, calls: int) -> list[dict]:
    """What bounds the config-2 attention call: the fixed cost of a call, the
    marginal streaming rate, the cost of ragged lengths, and one compute
    unit's ceiling.

    * the graph launch gap of a one-element kernel;
    * the public entry point (one pass) at TinyLlama geometry over 64 rows
      of uniform length L in {16, 512, 1024, 1210, 2048} plus 8 empty rows:
      a least-squares line through time vs algorithmic bytes gives the
      fixed microseconds per call and the marginal GB/s; 1210 tokens is the
      config-2 byte count spread evenly, so it is the time config 2 would
      take with no length imbalance;
    * config 2 itself with its random pages and with the same rows on
      contiguous pages (page locality);
    * 16 rows x 2048 (64 compute units busy) with 1..8 wavefronts per kv
      head through the C ABI: one compute unit's ceiling at low load;
    * the read probe with one workgroup (one compute unit alone) at 4..16
      wavefronts and 4 or 8 loads in flight per lane: a compute unit's read
      rate against the bytes it keeps in flight;
    * the page-gather probe over config 2's own pages (every byte of each
      K and V page, no compute) at several launch shapes: the attainable
      rate of the call's scattered-page reads.
    Every case rotates 6 copies of its page pool (the MALL cannot hold them).
    """

    from tensorforge_amd import _native

    results = []
    tiny = torch.zeros(1, device=device)
    launch_us = graph_time_us(lambda i: tiny.add_(1.0), 200, device)
    results.append({"case": "graph launch gap (one-element add_ kernel)",
                    "us_per_call": round(launch_us, 3)})

    def attention_case(name: str, case: workloads.DecodeAttentionCase,
                       flags: int | None = None) -> dict:
        gpu = case.to(device)
        pools = [(gpu.key_cache, gpu.value_cache)] + [
            (gpu.key_cache.clone(), gpu.value_cache.clone()) for _ in range(5)]
        output = torch.empty_like(gpu.query)
        batch, query_heads, head_dim = gpu.query.shape
        num_blocks, block_size, kv_heads, _ = gpu.key_cache.shape
        width = gpu.block_tables.shape[1]
        lib = _native.library()

        def run(i: int) -> None:
            key_cache, value_cache = pools[i % len(pools)]
            if flags is None:
                paged_gqa_decode_attention(query=gpu.query, key_cache=key_cache,
                                           value_cache=value_cache,
                                           block_tables=gpu.block_tables,
                                           context_lengths=gpu.context_lengths,
                                           scale=case.scale,
                                           max_context_length=min(2048, width * block_size),
                                           output=output)
                return
            _native.check(lib.tf_paged_gqa_decode(
                gpu.query.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(),
                gpu.block_tables.data_ptr(), gpu.context_lengths.data_ptr(),
                output.data_ptr(), None, None, None, None, 0, head_dim, batch, query_heads,
                kv_heads, head_dim, num_blocks, block_size, width,
                (width * block_size + 31) // 32 * 32, 1, case.scale,
                _native.dtype_code(gpu.query.dtype), flags,
                _native.current_stream(device)), "tf_paged_gqa_decode")

        us = graph_time_us(run, calls, device)
        nbytes = workloads.decode_attention_bytes(case.lengths, query_heads, kv_heads,
                                                  head_dim, block_size, 2)
        return report(name, us, nbytes)

    def rows(lengths: list[int]) -> workloads.DecodeAttentionCase:
        return workloads.make_decode_attention_case(
            lengths, query_heads=32, kv_heads=4, head_dim=64, block_size=16,
            dtype=torch.bfloat16, seed=0)

    uniform = []
    for length in (16, 512, 1024, 1210, 2048):
        result = attention_case(f"one pass, 64 rows x {length} + 8 empty", rows([length] * 64 + [0] * 8))
        uniform.append(result)
        results.append(result)
    xs = [r["algorithmic_bytes"] / 1e6 for r in uniform]
    ys = [r["us_per_call"] for r in uniform]
    mean_x, mean_y = sum(xs) / len(xs), sum(ys) / len(ys)
    slope = (sum((x - mean_x) * (y - mean_y) for x, y in zip(xs, ys))
             / sum((x - mean_x) ** 2 for x in xs))
    fixed_us = mean_y - slope * mean_x
    results.append({"case": "fit over the uniform rows: time = fixed + bytes / rate",
                    "fixed_us": round(fixed_us, 2), "marginal_GB/s": round(1e3 / slope, 1)})

    config2 = workloads.tinyllama_decode_case(seed=0, dtype=torch.bfloat16)
    results.append(attention_case("config 2 (random pages)", config2))
    contiguous = rows(config2.lengths)
    tables = contiguous.block_tables.clone()
    cursor = 0
    for row, ctx in enumerate(config2.lengths):
        pages = (ctx + 15) // 16
        tables[row, :pages] = torch.arange(cursor, cursor + pages, dtype=torch.int32)
        cursor += pages
    contiguous.block_tables = tables
    results.append(attention_case("config 2 rows on contiguous pages", contiguous))

    few = rows([2048] * 16)
    for waves in (1, 2, 3, 4, 6, 8):
        flags = ((1 << _native.TF_ATTENTION_HEADS_PER_WG_SHIFT)
                 | (waves << _native.TF_ATTENTION_WAVES_PER_CU_SHIFT)
                 | ((256 // 64) << _native.TF_ATTENTION_TOKENS_PER_WAVE_SHIFT))
        result = attention_case(f"16 rows x 2048, {waves} wavefronts per kv head", few, flags)
        # 64 (row, kv head) workgroups, one compute unit each
        result["GB/s_per_compute_unit_beyond_fixed"] = round(
            result["algorithmic_bytes"] / 64 / (result["us_per_call"] - fixed_us) / 1e3, 1)
        results.append(result)

    lib = _native.library()
    sink = torch.zeros(1, dtype=torch.int32, device=device)
    region = 8 << 20
    regions = 40  # 320 MiB rotated: no region is served from the MALL
    buffer = torch.ones(regions * region // 4, dtype=torch.int32, device=device)
    for waves, loads in ((4, 4), (8, 4), (8, 8), (16, 4), (16, 8)):
        def read_one_unit(i: int, waves=waves, loads=loads) -> None:
            _native.check(lib.tf_hbm_read_probe(
                buffer.data_ptr() + (i % regions) * region, region, 1, waves, loads,
                sink.data_ptr(), _native.current_stream(device)), "read probe")

        us = graph_time_us(read_one_unit, 20, device)
        results.append({"case": f"read probe, one compute unit, {waves} wavefronts x {loads} "
                                f"loads ({waves * loads} KB in flight)",
                        "us_per_call": round(us, 2), "GB/s": round(region / us / 1e3, 1)})
    del buffer
    torch.cuda.empty_cache()

    gpu = config2.to(device)
    pools = [(gpu.key_cache, gpu.value_cache)] + [
        (gpu.key_cache.clone(), gpu.value_cache.clone()) for _ in range(5)]
    page_list = []
    for row, ctx in enumerate(config2.lengths):
        page_list.extend(int(p) for p in config2.block_tables[row, : (ctx + 15) // 16])
    pages = torch.tensor(page_list, dtype=torch.int32, device=device)
    page_bytes = gpu.key_cache[0].numel() * gpu.key_cache.element_size()
    nbytes2 = workloads.decode_attention_bytes(config2.lengths, 32, 4, 64, 16, 2)
    for workgroups, waves in ((256, 4), (256, 8), (512, 8), (1024, 8), (2048, 4)):
        def gather(i: int, workgroups=workgroups, waves=waves) -> None:
            key_cache, value_cache = pools[i % len(pools)]
            _native.check(lib.tf_hbm_page_gather_probe(
                key_cache.data_ptr(), value_cache.data_ptr(), pages.data_ptr(), pages.numel(),
                page_bytes, gpu.key_cache.shape[0], workgroups, waves, sink.data_ptr(),
                _native.current_stream(device)), "page gather probe")

        us = graph_time_us(gather, calls, device)
        results.append({"case": f"page gather of config 2's {pages.numel()} pages, "
                                f"{workgroups} x {waves} wavefronts",
                        "us_per_call": round(us, 3),
                        "call_bytes_GB/s": round(nbytes2 / us / 1e3, 1)})
    return results


def valu_comparison(device: torch.device, calls: int) -> list[dict]:
    """The attention products on MFMA against the VALU form of the same grid
    kernel (TF_ATTENTION_FLAG_VALU: packed bf16 dot products for the scores,
    fp32 FMAs for P.V; same loads, LDS staging, softmax and epilogue), at
    config 2's lengths with group 8 (32/4 heads) and group 4 (16/4 heads,
    the same K/V bytes), bf16, through the C ABI with the entry point's
    one-pass plan (4 wavefronts per kv head, 576 tokens each) and with one
    wavefront per (row, kv head).  6 rotated page pools."""

    from tensorforge_amd import _native

    lib = _native.library()
    results = []
    config2 = workloads.tinyllama_decode_case(seed=0, dtype=torch.bfloat16)
    plans = {
        "one pass, 4 wavefronts per kv head": (
            (1 << _native.TF_ATTENTION_HEADS_PER_WG_SHIFT)
            | (4 << _native.TF_ATTENTION_WAVES_PER_CU_SHIFT)
            | ((576 // 64) << _native.TF_ATTENTION_TOKENS_PER_WAVE_SHIFT)),
        "one pass, 1 wavefront per kv head": 0,
    }
    for query_heads in (32, 16):
        case = workloads.make_decode_attention_case(
            config2.lengths, query_heads=query_heads, kv_heads=4, head_dim=64, block_size=16,
            dtype=torch.bfloat16, seed=0)
        gpu = case.to(device)
        pools = [(gpu.key_cache, gpu.value_cache)] + [
            (gpu.key_cache.clone(), gpu.value_cache.clone()) for _ in range(5)]
        output = torch.empty_like(gpu.query)
        batch = gpu.query.shape[0]
        num_blocks, block_size, kv_heads, head_dim = gpu.key_cache.shape
        width = gpu.block_tables.shape[1]
        nbytes = workloads.decode_attention_bytes(case.lengths, query_heads, kv_heads, head_dim,
                                                  block_size, 2)
        for plan, plan_flags in plans.items():
            row = {"case": f"group {query_heads // kv_heads}, {plan}"}
            for form, form_flags in (("mfma", 0), ("valu", _native.TF_ATTENTION_FLAG_VALU)):
                def run(i: int, flags=plan_flags | form_flags) -> None:
                    key_cache, value_cache = pools[i % len(pools)]
                    _native.check(lib.tf_paged_gqa_decode(
                        gpu.query.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(),
                        gpu.block_tables.data_ptr(), gpu.context_lengths.data_ptr(),
                        output.data_ptr(), None, None, None, None, 0, head_dim, batch,
                        query_heads, kv_heads, head_dim, num_blocks, block_size, width,
                        (width * block_size + 31) // 32 * 32, 1, case.scale,
                        _native.dtype_code(gpu.query.dtype), flags,
                        _native.current_stream(device)), "tf_paged_gqa_decode")

                us = graph_time_us(run, calls, device)
                row[f"{form}_us"] = round(us, 3)
                row[f"{form}_GB/s"] = round(nbytes / us / 1e3, 1)
            row["valu_over_mfma"] = round(row["valu_us"] / row["mfma_us"], 3)
            results.append(row)
    return results


def measure_decode_step(weights: DecoderWeights, batch: int, context: int, *,
                        steps: int = 64, seed: int = 0,
                        prompt_lengths: list[int] | None = None) -> dict:
    """One graph-captured decode step of ``weights`` at ``batch`` requests in
    the context bucket ``context`` (prompts of about context - 40 tokens, or
    ``prompt_lengths``, prefilled first): device p50/p95 per step from HIP
    events and the host-inclusive time per step of the pipelined
    launch/collect loop."""

    import time

    config = weights.config
    device = weights.embedding.device
    dtype = weights.embedding.dtype
    generator = torch.Generator().manual_seed(seed)
    if prompt_lengths is None:
        prompt_lengths = [context - steps // 2 - 8 if context > steps else context // 2] * batch
    if len(prompt_lengths) != batch or max(prompt_lengths) >= context:
        raise ValueError("one prompt length per request, each below the context bucket")
    prompt_length = max(prompt_lengths)
    cache = PagedKVCache(PagedKVCacheConfig(
        num_layers=config.num_hidden_layers, num_blocks=batch * (context // 16 + 2),
        block_size=16, num_kv_heads=config.num_key_value_heads,
        head_dim=config.head_dim, max_sequences=batch, max_sequence_length=context,
        dtype=dtype, device=device))
    executor = BucketedDecodeExecutor(weights, cache, batch_buckets=(batch,),
                                      context_buckets=(context,))
    rids = [f"s{i}" for i in range(batch)]
    for rid in rids:
        executor.create_request(rid)
    prompts = {rid: torch.randint(0, config.vocab_size, (n,), generator=generator).tolist()
               for rid, n in zip(rids, prompt_lengths)}
    tokens, errors = executor.prefill_tokens(prompts)
    if errors:
        raise RuntimeError(f"prefill failed: {errors}")
    budget = context - prompt_length
    warm = min(4, budget // 4)
    timed = min(steps, budget - warm - 2)
    pending = executor.launch(rids, tokens)
    for _ in range(warm):
        ticket = executor.launch(rids)
        executor.collect(pending)
        pending = ticket
    # The clock starts when a step has just been collected, with the next
    # one already queued, and stops when the timed-th step after it has been
    # collected: exactly `timed` step completions with the pipeline full.
    # (Starting it with a step in flight would count that step's remainder
    # too: about one step more than `timed`.)
    executor.step_records.clear()
    begin = time.perf_counter()
    for _ in range(timed):
        ticket = executor.launch(rids)
        executor.collect(pending)
        pending = ticket
    host_ms = (time.perf_counter() - begin) * 1e3 / timed
    executor.collect(pending)
    times = sorted(r.device_ms for r in executor.step_records[1:])
    p50 = times[len(times) // 2]
    return {
        "steps": timed, "prompt_tokens": sum(prompt_lengths),
        # Contexts of the timed steps, on average (new token included).
        "sum_context_mean": sum(prompt_lengths) + batch * (warm + (timed + 1) // 2),
        "device_ms_p50": round(p50, 4),
        "device_ms_p95": round(times[int(0.95 * (len(times) - 1))], 4),
        "host_inclusive_ms_per_step": round(host_ms, 4),
        "tokens_per_second": round(batch / (max(host_ms, p50) / 1e3), 1),
    }


def decode_steps(device: torch.device, model: str = "cfg1", steps: int = 64) -> None:
    import dataclasses

    if model == "cfg1":
        config = dataclasses.replace(small_config(), max_position_embeddings=4096)
        dtype, grid = torch.float16, [(c, b) for c in (32, 128, 512, 2048) for b in (1, 4, 8)]
    else:
        config = tinyllama_config()
        dtype, grid = torch.bfloat16, [(1024, b) for b in (1, 8, 64)]
    weights = DecoderWeights.random(config, seed=0, dtype=dtype, device=device)
    for context, batch in grid:
        result = measure_decode_step(weights, batch, context, steps=steps)
        print(json.dumps({"case": f"decode_step {model}-model b{batch}-c{context}", **result}),
              flush=True)


def projections(device: torch.device, calls: int) -> list[dict]:
    """The decode step's projections and narrow attention plans (see the
    module docstring); times in microseconds per call."""

    results = []
    shapes = {"qkv": (2560, 2048), "o": (2048, 2048), "down": (2048, 5632),
              "gate_up+swiglu": (11264, 2048), "lm_head": (32000, 2048)}
    for name, (n, k) in shapes.items():
        copies = max(2, int(600e6 // (n * k * 2)))
        weights = [torch.randn(n, k, device=device, dtype=torch.bfloat16) * 0.02
                   for _ in range(copies)]
        for m in (1, 16, 64):
            x = torch.randn(m, k, device=device, dtype=torch.bfloat16)
            y = torch.empty(m, n, device=device, dtype=torch.bfloat16)
            row = {"case": f"projection {name} [{m}x{k}]x[{k}x{n}]", "weight_MB": round(n * k * 2e-6, 1)}

            def timed(fn) -> float:
                return round(graph_time_us(lambda i: fn(weights[i % copies]), calls, device), 2)

            if name == "gate_up+swiglu":
                act = torch.empty(m, n // 2, device=device, dtype=torch.bfloat16)
                row["hipblaslt+swiglu_us"] = timed(
                    lambda w: swiglu_gate_up(torch.mm(x, w.t(), out=y), output=act))
                row["linear_rows+swiglu_us"] = timed(
                    lambda w: swiglu_gate_up(linear_rows(x, w, output=y), output=act))
                row["k_split_swiglu_us"] = timed(
                    lambda w: linear_swiglu(x, w, output=act, k_split=True))
            else:
                row["hipblaslt_us"] = timed(lambda w: torch.mm(x, w.t(), out=y))
                row["linear_rows_us"] = timed(lambda w: linear_rows(x, w, output=y))
                if name == "qkv":
                    row["linear_kstream_us"] = timed(lambda w: linear_kstream(x, w, output=y))
                elif name in ("o", "down"):
                    splits = default_splits(n, k)
                    part = torch.empty(splits, m, n, device=device)
                    row[f"linear_stream_{splits}_slices_us"] = timed(
                        lambda w: linear_stream(x, w, splits=splits, partials=part))
                else:
                    row["linear_stream_us"] = timed(lambda w: linear_stream(x, w, output=y))
            results.append(row)
        del weights
        torch.cuda.empty_cache()

    for batch, context in ((1, 1000), (8, 1000), (1, 4000), (8, 4000), (64, 512), (64, 1000)):
        case = workloads.make_decode_attention_case(
            [context] * batch, query_heads=32, kv_heads=4, head_dim=64, block_size=16,
            dtype=torch.bfloat16, seed=batch + context)
        gpu = case.to(device)
        width = gpu.block_tables.shape[1]
        # Partials for one partition per 128 tokens, as the decode executor sizes them.
        workspace = PagedAttentionWorkspace.allocate(
            batch_capacity=batch, query_heads=32, head_dim=64, max_context_length=2 * width * 16,
            device=device)
        output = torch.empty_like(gpu.query)

        def run(i: int) -> None:
            paged_gqa_decode_attention(gpu.query, gpu.key_cache, gpu.value_cache,
                                       gpu.block_tables, gpu.context_lengths, scale=case.scale,
                                       max_context_length=width * 16, output=output,
                                       workspace=workspace)

        planned = graph_time_us(run, calls, device)
        record = selected_attention_autotune_config()
        launch = selected_attention_launch()
        previous = set_attention_split_size(256)
        try:
            fixed = graph_time_us(run, calls, device)
        finally:
            set_attention_split_size(previous)
        results.append({"case": f"attention {batch} rows x {context} (TinyLlama geometry)",
                        "plan_us": round(planned, 2), "plan": record,
                        "waves_per_head": launch["waves_per_head"],
                        "heads_per_workgroup": launch["heads_per_workgroup"],
                        "fixed_256_partitions_us": round(fixed, 2)})
    return results


def step_projections(device: torch.device, calls: int) -> list[dict]:
    """The four projections of a 64-row TinyLlama decode step in the forms
    the executor's default chain launches (decode._forward): qkv with the
    input RMSNorm, o and down added to the residual stream, gate|up with the
    post-attention RMSNorm and SwiGLU.  Weights rotated through enough
    copies (>= 600 MB) that each call reads its weight from HBM; bytes are
    the weight, x and the output (and the residual) once."""

    from tensorforge_amd.kernels import linear_swiglu

    m, h, f, eps = 64, 2048, 5632, 1e-5
    generator = torch.Generator().manual_seed(0)

    def randn(*shape: int, scale: float = 1.0) -> torch.Tensor:
        return (torch.randn(*shape, generator=generator) * scale).to(torch.bfloat16).to(device)

    x_h, residual, attn, act = randn(m, h), randn(m, h), randn(m, h), randn(m, f)
    y_qkv = torch.empty(m, 2560, dtype=torch.bfloat16, device=device)
    y_h = torch.empty(m, h, dtype=torch.bfloat16, device=device)
    y_act = torch.empty(m, f, dtype=torch.bfloat16, device=device)
    e = 2
    cases = {
        "qkv + input norm (linear_kstream norm)": (
            (2560, h), lambda w: linear_kstream(x_h, w, output=y_qkv, norm_eps=eps),
            (m * h + m * 2560) * e),
        "o + residual (linear_kstream residual)": (
            (h, h), lambda w: linear_kstream(attn, w, output=y_h, residual=residual),
            (2 * m * h + m * h) * e),
        "gate|up + post norm + SwiGLU (linear_swiglu k_split norm)": (
            (2 * f, h), lambda w: linear_swiglu(x_h, w, output=y_act, k_split=True, norm_eps=eps),
            (m * h + m * f) * e),
        "down + residual (linear_kstream residual)": (
            (h, f), lambda w: linear_kstream(act, w, output=y_h, residual=residual),
            (m * f + 2 * m * h) * e),
    }
    results = []
    for name, ((n, k), run, io_bytes) in cases.items():
        copies = max(2, int(600e6 // (n * k * e)))
        weights = [randn(n, k, scale=0.02) for _ in range(copies)]
        us = graph_time_us(lambda i: run(weights[i % copies]), calls, device)
        results.append(report(f"b64 step projection: {name} [{m}x{k}]x[{k}x{n}]", us,
                              n * k * e + io_bytes, weight_bytes=n * k * e,
                              weight_copies=copies))
        del weights
    return results


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--calls", type=int, default=100)
    parser.add_argument("--only", choices=("cfg3", "cfg4", "decode", "decode22", "ceiling", "valu",
                                           "projections", "step_projections"), default=None)
    args = parser.parse_args()
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        return 1
    device = torch.device("cuda", 0)
    if args.only in (None, "cfg4"):
        for result in config4(device, args.calls):
            print(json.dumps(result), flush=True)
    if args.only in (None, "cfg3"):
        for result in config3(device, max(10, args.calls // 4)):
            print(json.dumps(result), flush=True)
    if args.only in (None, "decode"):
        decode_steps(device, "cfg1")
    if args.only in (None, "decode22"):
        decode_steps(device, "tinyllama")
    if args.only == "valu":
        for result in valu_comparison(device, args.calls):
            print(json.dumps(result), flush=True)
    if args.only in (None, "ceiling"):
        for result in attention_ceiling(device, args.calls):
            print(json.dumps(result), flush=True)
    if args.only in (None, "projections"):
        for result in projections(device, args.calls):
            print(json.dumps(result), flush=True)
    if args.only == "step_projections":
        for result in step_projections(device, args.calls):
            print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
