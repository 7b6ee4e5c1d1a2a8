"""Benchmark of the paged GQA decode hot path on one MI355X.

Workload: paged GQA decode attention at TinyLlama
geometry -- 64 rows with context U[128, 2048] plus 8 zero-length rows,
32 query / 4 KV heads, head_dim 64, 16-token pages on a seeded permutation,
bf16, N(0,1) inputs, scale 1/8.  A step is one attention call over one
batch as the Python entry point plans it: at this batch one pass, one
workgroup per (row, kv head) whose wavefronts (up to four, one per 576
tokens of the row) share the row and combine in LDS (no partials, no merge
launch); ``--split-size`` forces the
split-KV form (split stage + log-sum-exp merge launch).  To keep
the 256 MB Infinity Cache from serving the K/V pages, steps rotate over
several independent copies of the page pool (``--pools``), so every step
streams its pages from HBM.

Prints ONE JSON line.  ``value`` is algorithmic GB/s of the whole call
(byte model of benchmark/attention_benchmark.py:148-161: q, K, V, tables,
output of the active rows) over the timed steps.  The K timed steps run as
one HIP-graph replay bracketed by HIP events on the launch stream (a ctypes
call costs the host longer than the kernel takes, so eager steps would
time the host).  ``roofline`` reports the dominant kernel: in one pass the
whole call; in split-KV form the split stage, timed the same way from a
graph of K split-stage launches alone.
``cpu_baseline`` is the CPU oracle on the same rows, on this host's cores.

``decode_step`` is the metric's "decode tokens/s" part: a whole
graph-captured decode step of the 22-layer TinyLlama-geometry model (random
init, bf16) for the same 64 rows, with prompts of the rows' context lengths,
with its own ``roofline`` (the step's algorithmic bytes -- every layer's
weights, the rows' K/V at their contexts, LM head -- over the device step
time), and beside it the oracle's fp32 incremental decode step on all 64
rows on the host cores.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

import torch

REPO_ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO_ROOT))

METRIC = "paged GQA decode HBM GB/s (% peak) + decode tokens/s, TinyLlama-geom b=64"
HBM_PEAK_GBS = 8000.0
TRAFFIC_FILE = REPO_ROOT / "profiles" / "paged_decode_tinyllama_b64_traffic.json"


def parse_args() -> argparse.Namespace:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=200)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--pools", type=int, default=6, help="rotated K/V page pools")
    parser.add_argument("--split-size", type=int, default=0,
                        help="force split-KV with this partition size (multiple of 32); "
                             "0: the Python entry point's plan (one pass at this batch)")
    parser.add_argument("--merge", choices=("fused", "kernel"), default="kernel",
                        help="separate merge launch (the product path) or the in-kernel "
                             "merge enabled by arrival counters")
    parser.add_argument("--cpu-seconds", type=float, default=10.0,
                        help="target CPU time of the oracle baseline sample")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-decode-step", action="store_true",
                        help="skip the 22-layer decode-step tokens/s part of the metric")
    parser.add_argument("--kernels", action="store_true",
                        help="instead of the metric: config 3 and 4 kernels (graph-timed) with "
                             "the CPU oracle timed beside each case; one JSON line")
    parser.add_argument("--copy-calibration-mib", type=int, default=0,
                        help="only run a plain device copy of this many MiB (counter calibration)")
    return parser.parse_args()


def copy_calibration(mib: int) -> int:
    """A plain device-to-device copy of known size: under rocprofv3 --pmc its
    FETCH_SIZE / WRITE_SIZE per dispatch give the counter-to-bytes factor."""

    device = torch.device("cuda", 0)
    src = torch.ones(mib * 1024 * 1024 // 4, dtype=torch.float32, device=device)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_read": src.numel() * 4,
                      "copy_calibration_bytes_written": dst.numel() * 4, "dispatches": 5}))
    return 0


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), for the baseline labels."""

    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def read_ceiling(nbytes: int, gather: dict | None = None) -> dict:
    """What this GPU streams from HBM, measured in this process: the library's
    read probe (contiguous slices, 16-byte nontemporal loads) over 1 GiB and
    over the attention call's own byte count, each rotated over regions the
    256 MB Infinity Cache cannot hold, the best of a few launch shapes (swept
    on MI355X: 512 x 4 waves for 1 GiB, 4096 x 16 waves for ~80 MB); and the
    reference's method, a torch copy_ of 256 MiB counted as read + write
    (benchmark/kernel_benchmark.py:176-192).

    With ``gather`` (``pools``: the rotated (key, value) caches, ``pages``:
    the call's physical pages in row order on the device, ``page_bytes``,
    ``num_blocks``), also the library's page-gather probe over exactly
    those pages -- the call's own scattered-page reads and nothing else,
    best of a few launch shapes -- reported as its time and as the call's
    algorithmic bytes over that time."""

    from tensorforge_amd import _native

    lib = _native.library()
    device = torch.device("cuda", 0)
    buffer = torch.ones(3 << 28, dtype=torch.int32, device=device)  # 3 GiB
    sink = torch.zeros(1, dtype=torch.int32, device=device)
    total = buffer.numel() * 4

    def timed(size: int, shape: tuple[int, int, int]) -> float:
        size -= size % 16
        regions = max(2, min(12, total // size))
        stride = (total // regions) // 256 * 256
        reps = 24 if size < (256 << 20) else 8
        stream = torch.cuda.Stream(device)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(reps):
                _native.check(lib.tf_hbm_read_probe(
                    buffer.data_ptr() + (i % regions) * stride, size, *shape, sink.data_ptr(),
                    stream.cuda_stream), "read probe")
        graph.replay()
        torch.cuda.synchronize()
        best = float("inf")
        for _ in range(3):
            begin = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            begin.record()
            graph.replay()
            end.record()
            end.synchronize()
            best = min(best, begin.elapsed_time(end) / reps)
        return size / (best * 1e-3) / 1e9

    one_gib = max(timed(1 << 30, shape) for shape in ((512, 4, 4), (256, 8, 4), (4096, 4, 8)))
    same = max(timed(nbytes, shape) for shape in ((4096, 16, 4), (8192, 8, 8), (2048, 16, 4)))
    source = buffer[: (256 << 20) // 4]
    destination = torch.empty_like(source)
    for _ in range(3):
        destination.copy_(source)
    torch.cuda.synchronize()
    begin = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    begin.record()
    for _ in range(10):
        destination.copy_(source)
    end.record()
    end.synchronize()
    copy = 2 * source.numel() * 4 / (begin.elapsed_time(end) / 10 * 1e-3) / 1e9
    del buffer, source, destination
    torch.cuda.empty_cache()
    result = {"read_1GiB": round(one_gib, 1), "read_same_bytes": round(same, 1),
              "copy_256MiB": round(copy, 1), "unit": "GB/s",
              "method": "tf_hbm_read_probe graph replays (best launch shape), 1 GiB and the "
                        "call's byte count, regions rotated past the MALL; torch copy_ of 256 MiB "
                        "counted as 2 x bytes (the reference's ceiling)"}
    if gather is not None:
        gather_us = page_gather_us(**gather)
        result["gather_call_pages_us"] = round(gather_us, 3)
        result["gather_call_pages"] = round(nbytes / (gather_us * 1e-6) / 1e9, 1)
        result["gather_method"] = ("tf_hbm_page_gather_probe over the call's own pages (whole "
                                   "pages, rotated pools, best of 3 launch shapes): the call's "
                                   "algorithmic bytes / the probe's time")
    return result


def page_gather_us(pools: list, pages: torch.Tensor, page_bytes: int, num_blocks: int) -> float:
    """Graph-timed microseconds of reading ``pages`` of every pool's K and V
    caches once (one pool per launch, rotated), the best of a few launch
    shapes (swept on MI355X at config 2: 256 x 8 waves best, 13.8 us)."""

    from tensorforge_amd import _native

    lib = _native.library()
    device = pages.device
    sink = torch.zeros(1, dtype=torch.int32, device=device)
    best = float("inf")
    for workgroups, waves in ((256, 8), (512, 8), (1024, 8)):
        reps = 6 * len(pools)
        stream = torch.cuda.Stream(device)
        stream.wait_stream(torch.cuda.current_stream(device))
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(reps):
                key_cache, value_cache = pools[i % len(pools)]
                _native.check(lib.tf_hbm_page_gather_probe(
                    key_cache.data_ptr(), value_cache.data_ptr(), pages.data_ptr(),
                    pages.numel(), page_bytes, num_blocks, workgroups, waves, sink.data_ptr(),
                    stream.cuda_stream), "page gather probe")
        torch.cuda.current_stream(device).wait_stream(stream)
        graph.replay()
        torch.cuda.synchronize()
        for _ in range(3):
            begin = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            begin.record()
            graph.replay()
            end.record()
            end.synchronize()
            best = min(best, begin.elapsed_time(end) * 1e3 / reps)
    return best


def call_pages(block_tables: torch.Tensor, lengths: list[int], block_size: int) -> torch.Tensor:
    """The physical pages an attention call reads, in row order (host side)."""

    pages = []
    for row, ctx in enumerate(lengths):
        pages.extend(int(page) for page in block_tables[row, : (ctx + block_size - 1) // block_size])
    return torch.tensor(pages, dtype=torch.int32)


def cpu_baseline(case, rows: list[int], seconds: float) -> dict:
    """Time the CPU oracle (fp32 torch on the host cores) on ``rows``."""

    from oracle.reference import paged_gqa_decode_reference
    from tensorforge_amd.workloads import decode_attention_bytes

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    cpu = case.to("cpu")
    args = (cpu.query[rows], cpu.key_cache, cpu.value_cache, cpu.block_tables[rows],
            cpu.context_lengths[rows])
    paged_gqa_decode_reference(*args, scale=case.scale)  # warmup
    samples = []
    started = time.perf_counter()
    while len(samples) < 3 or time.perf_counter() - started < seconds:
        t0 = time.perf_counter_ns()
        paged_gqa_decode_reference(*args, scale=case.scale)
        samples.append((time.perf_counter_ns() - t0) / 1e9)
    samples.sort()
    p50 = samples[len(samples) // 2]
    lengths = [case.lengths[r] for r in rows]
    nbytes = decode_attention_bytes(lengths, 32, 4, 64, 16, 2)
    return {
        "value": round(nbytes / p50 / 1e9, 4),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": (
            f"CPU oracle paged_gqa_decode_reference (fp32 torch {torch.__version__}) on "
            f"{len(rows)} of the 64 active rows (sum ctx {sum(lengths)}), p50 of "
            f"{len(samples)} reps = {p50 * 1e3:.2f} ms; {cpu_model()}"
        ),
    }


def decode_step(lengths: list[int], cpu_seconds: float, with_cpu: bool) -> dict:
    """The metric's "decode tokens/s" part: one graph-captured decode step of
    the 22-layer TinyLlama-geometry model (random init, bf16) for the 64
    active rows of this workload, prompts of the workload's context lengths
    (less the steps decoded), context bucket 2048.  The CPU baseline is the
    fp32 incremental decode step of the oracle on the same rows."""

    from tensorforge_amd.decode import DecoderWeights, tinyllama_config
    from tensorforge_amd.kernel_bench import measure_decode_step
    from tensorforge_amd.workloads import decode_step_bytes

    device = torch.device("cuda", 0)
    config = tinyllama_config()
    weights = DecoderWeights.random(config, seed=0, dtype=torch.bfloat16, device=device)
    active = [n for n in lengths if n > 0]
    steps = 40
    prompts = [max(1, min(n, 2048 - steps - 8)) for n in active]
    gpu = measure_decode_step(weights, len(active), 2048, steps=steps, prompt_lengths=prompts)
    step_bytes = decode_step_bytes(config, gpu["sum_context_mean"], len(active), 2)
    rate = step_bytes["total"] / (gpu["device_ms_p50"] * 1e-3) / 1e9
    result = {
        "model": "TinyLlama-1.1B geometry, 22 layers, random init (seed 0), bf16",
        "batch": len(active),
        "tokens_per_second": gpu["tokens_per_second"],
        "ms_per_step_device_p50": gpu["device_ms_p50"],
        "ms_per_step_host_inclusive": gpu["host_inclusive_ms_per_step"],
        "steps": gpu["steps"],
        "timing": "HIP events around each graph replay; host-inclusive = pipelined "
                  "launch/collect loop wall time per step",
        "roofline": {"bound": "hbm", "achieved": round(rate, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(rate / HBM_PEAK_GBS, 4),
                     "algorithmic_bytes_per_step": step_bytes,
                     "sum_context_mean": gpu["sum_context_mean"],
                     "model": "workloads.decode_step_bytes: every layer's weights once, the "
                              "rows' K/V read at their contexts and the new K/V written, LM "
                              "head, embedding rows and logits; over the device p50 step time"},
    }
    if with_cpu:
        result["cpu_baseline"] = decode_step_cpu_baseline(weights, prompts, cpu_seconds)
    return result


def decode_step_cpu_baseline(weights, contexts: list[int], seconds: float) -> dict:
    """The oracle's fp32 incremental decode step (oracle/model.py) on the host
    cores: every row at its context, caches filled with random K/V (one
    K and one V buffer serve all layers: the step's arithmetic and reads
    are the same, at a 22nd of the host memory)."""

    from oracle.model import decode_step_reference
    from tensorforge_amd.decode import DecoderWeights, LayerWeights

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    f32 = lambda t: t.detach().float().cpu()  # noqa: E731
    cpu = DecoderWeights(
        config=weights.config, embedding=f32(weights.embedding),
        layers=[LayerWeights(*(f32(getattr(layer, name)) for name in
                               ("input_norm", "qkv", "o_proj", "post_norm", "gate_up", "down")))
                for layer in weights.layers],
        final_norm=f32(weights.final_norm), lm_head=f32(weights.lm_head),
        rope_cos=f32(weights.rope_cos), rope_sin=f32(weights.rope_sin))
    config = weights.config
    batch, capacity = len(contexts), max(contexts) + 64
    generator = torch.Generator().manual_seed(0)
    key = torch.randn(batch, capacity, config.num_key_value_heads, config.head_dim,
                      generator=generator)
    value = torch.randn_like(key)
    keys, values = [key] * len(cpu.layers), [value] * len(cpu.layers)
    positions = torch.tensor(contexts)
    tokens = torch.randint(0, config.vocab_size, (batch,), generator=generator)
    decode_step_reference(cpu, keys, values, tokens, positions)  # warmup
    samples = []
    started = time.perf_counter()
    while len(samples) < 3 or (time.perf_counter() - started < seconds and len(samples) < 60):
        positions = positions + 1
        t0 = time.perf_counter_ns()
        decode_step_reference(cpu, keys, values, tokens, positions)
        samples.append((time.perf_counter_ns() - t0) / 1e9)
    samples.sort()
    p50 = samples[len(samples) // 2]
    return {
        "value": round(batch / p50, 2),
        "unit": "tokens/s",
        "cores": cores,
        "kind": "port",
        "sample": (
            f"oracle decode_step_reference (fp32 torch {torch.__version__}), 22 layers, "
            f"all {batch} rows (sum of contexts {sum(contexts)}), p50 of {len(samples)} steps = "
            f"{p50 * 1e3:.1f} ms; {cpu_model()}"
        ),
    }


def _cpu_p50(fn, seconds: float, reps: int = 3) -> float:
    fn()  # warmup
    samples = []
    started = time.perf_counter()
    while len(samples) < reps or (time.perf_counter() - started < seconds and len(samples) < 50):
        t0 = time.perf_counter_ns()
        fn()
        samples.append((time.perf_counter_ns() - t0) / 1e9)
    samples.sort()
    return samples[len(samples) // 2]


def kernels_line(calls: int, seconds_per_case: float) -> dict:
    """Config 4 (fused ops and the KV append) and config 3 (long-context
    attention) through the public entry points, graph-timed, each beside the
    CPU oracle of the same op on the same shape (fp32 torch / numpy on the
    host cores)."""

    from oracle.reference import (
        paged_gqa_decode_reference,
        paged_kv_write_slots_reference,
        residual_rms_norm_fused_reference,
        rms_norm_reference,
        swiglu_fused_reference,
    )
    from tensorforge_amd.kernel_bench import config3, config4
    from tensorforge_amd.workloads import llama3_long_context_case

    device = torch.device("cuda", 0)
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    generator = torch.Generator().manual_seed(0)

    def randn(*shape):
        return torch.randn(*shape, generator=generator).to(torch.bfloat16)

    cases = config4(device, calls)
    for case in cases:
        shape = case["shape"]
        tokens = shape["tokens"]
        if shape["op"] in ("rms_norm", "residual_rms_norm"):
            x, r, w = randn(tokens, shape["hidden"]), randn(tokens, shape["hidden"]), randn(
                shape["hidden"])
            fn = ((lambda: rms_norm_reference(x, w, 1e-5)) if shape["op"] == "rms_norm"
                  else (lambda: residual_rms_norm_fused_reference(x, r, w, 1e-5)))
        elif shape["op"] == "swiglu":
            g, u = randn(tokens, shape["ffn"]), randn(tokens, shape["ffn"])
            fn = lambda: swiglu_fused_reference(g, u)  # noqa: E731
        else:
            keys, values = randn(tokens, 4, 64), randn(tokens, 4, 64)
            kc, vc = randn(64, 16, 4, 64), randn(64, 16, 4, 64)
            slots = torch.arange(5, 5 + tokens, dtype=torch.int64)
            fn = lambda: paged_kv_write_slots_reference(keys, values, kc, vc, slots)  # noqa: E731
        p50 = _cpu_p50(fn, seconds_per_case)
        case["cpu_baseline"] = {"GB/s": round(case["algorithmic_bytes"] / p50 / 1e9, 3),
                                "us_per_call": round(p50 * 1e6, 1), "cores": cores,
                                "kind": "port"}
    attention = config3(device, max(10, calls // 4))
    cpu = llama3_long_context_case(seed=0)
    p50 = _cpu_p50(lambda: paged_gqa_decode_reference(
        cpu.query, cpu.key_cache, cpu.value_cache, cpu.block_tables, cpu.context_lengths,
        scale=cpu.scale), seconds_per_case * 4, reps=2)
    for case in attention:  # one oracle time: the same call whatever the GPU plan
        case["cpu_baseline"] = {"GB/s": round(case["algorithmic_bytes"] / p50 / 1e9, 3),
                                "us_per_call": round(p50 * 1e6, 1), "cores": cores,
                                "kind": "port"}
    return {"metric": "config 3 and 4 kernels, graph-timed, CPU oracle beside each",
            "unit": "GB/s", "cases": cases + attention,
            "cpu": cpu_model()}


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(
            json.dumps({
                "error": "this build runs on one GPU; multi-GPU sharding of the decode path "
                         "is design-only (see the sharding section of the design notes)",
                "n_gpus": args.gpus,
            })
        )
        return 2
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        return 1
    if args.copy_calibration_mib > 0:
        return copy_calibration(args.copy_calibration_mib)
    if args.kernels:
        print(json.dumps(kernels_line(100, 0.3)))
        return 0

    from tensorforge_amd import _native
    from tensorforge_amd.kernels import PagedAttentionWorkspace, set_attention_split_size
    from tensorforge_amd.kernels.attention import attention_plan, attention_split_size_for
    from tensorforge_amd.workloads import (
        decode_attention_bytes,
        decode_attention_flops,
        tinyllama_decode_case,
    )

    device = torch.device("cuda", 0)
    lib = _native.library()

    case = tinyllama_decode_case(seed=0, dtype=torch.bfloat16)
    gpu = case.to(device)
    pools = [(gpu.key_cache, gpu.value_cache)]
    for _ in range(args.pools - 1):
        pools.append((gpu.key_cache.clone(), gpu.value_cache.clone()))
    batch, query_heads, head_dim = gpu.query.shape
    num_blocks, block_size, kv_heads, _ = gpu.key_cache.shape
    table_width = gpu.block_tables.shape[1]
    max_context = 2048
    fused = args.merge == "fused"
    if args.split_size or fused:  # split-KV forced: the alternative paths
        split_size = args.split_size or attention_split_size_for(max_context, batch, kv_heads)
        set_attention_split_size(split_size)
        path = "split_kv"
    else:
        path = "auto"
    plan = attention_plan(max_context, batch, kv_heads, table_width * block_size, path,
                          head_dim=head_dim)
    split_size, num_splits, flags = plan.split_size, plan.num_splits, plan.flags
    one_pass = plan.one_pass
    workspace = PagedAttentionWorkspace.allocate(
        batch_capacity=batch, query_heads=query_heads, head_dim=head_dim,
        max_context_length=num_splits * 256, device=device,
    )
    head_bucket = workspace.partial_accumulator.shape[1]
    capacity = workspace.partial_max.numel()
    output = torch.empty_like(gpu.query)
    dtype = _native.dtype_code(gpu.query.dtype)
    stream = torch.cuda.current_stream(device)
    variant = lib.tf_paged_gqa_decode_variant(dtype, head_dim, query_heads // kv_heads, block_size, 0)

    counters = workspace.split_counters

    def attention_call(pool: int, handle: int) -> None:
        # tf_paged_gqa_decode as the plan launches it: one pass (one launch);
        # split-KV without arrival counters (split kernel + merge kernel); or
        # with them one launch whose last wavefront per (row, kv head) merges.
        key_cache, value_cache = pools[pool]
        _native.check(lib.tf_paged_gqa_decode(
            gpu.query.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(),
            gpu.block_tables.data_ptr(), gpu.context_lengths.data_ptr(), output.data_ptr(),
            workspace.partial_max.data_ptr(), workspace.partial_sum.data_ptr(),
            workspace.partial_accumulator.data_ptr(), counters.data_ptr() if fused else None,
            capacity, head_bucket, batch, query_heads, kv_heads, head_dim, num_blocks,
            block_size, table_width, split_size, num_splits, case.scale, dtype, flags, handle),
            "attention")

    def split_stage(pool: int, handle: int) -> None:
        key_cache, value_cache = pools[pool]
        _native.check(lib.tf_paged_gqa_decode_partials(
            gpu.query.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(),
            gpu.block_tables.data_ptr(), gpu.context_lengths.data_ptr(),
            workspace.partial_max.data_ptr(), workspace.partial_sum.data_ptr(),
            workspace.partial_accumulator.data_ptr(), capacity, head_bucket, batch,
            query_heads, kv_heads, head_dim, num_blocks, block_size, table_width, split_size,
            num_splits, case.scale, dtype, 0, handle), "partials")

    def merge_stage(handle: int) -> None:
        _native.check(lib.tf_paged_gqa_decode_merge(
            workspace.partial_max.data_ptr(), workspace.partial_sum.data_ptr(),
            workspace.partial_accumulator.data_ptr(), gpu.context_lengths.data_ptr(),
            output.data_ptr(), capacity, head_bucket, batch, query_heads, head_dim, split_size,
            num_splits, table_width * block_size, dtype, handle), "merge")

    # Gate before timing: the benchmarked raw call must equal the Python entry
    # point (the parity tests check that entry point) -- bit for bit on the
    # product path, up to rounding for the in-kernel merge alternative.
    eager = stream.cuda_stream
    attention_call(0, eager)
    torch.cuda.synchronize()
    from tensorforge_amd.kernels import paged_gqa_decode_attention

    check = paged_gqa_decode_attention(
        gpu.query, gpu.key_cache, gpu.value_cache, gpu.block_tables, gpu.context_lengths,
        scale=case.scale, max_context_length=max_context, workspace=workspace,
        attention_path=path,
    )
    torch.cuda.synchronize()
    if not fused:
        agree = torch.equal(check.view(torch.int16), output.view(torch.int16))
    else:  # a different merge order: equal up to rounding
        agree = float((check.float() - output.float()).abs().max()) < 2e-2
    if not agree:
        print(json.dumps({"error": "raw C-ABI call and the Python entry point disagree"}))
        return 1

    def one_step(step: int, handle: int) -> None:
        if fused or one_pass:
            attention_call(step % args.pools, handle)
        else:
            split_stage(step % args.pools, handle)
            merge_stage(handle)

    for step in range(args.warmup):
        one_step(step, eager)
    torch.cuda.synchronize()

    # Whole-job throughput: the K steps are captured once in a HIP graph and
    # replayed, so the host-side cost of a ctypes call (several microseconds,
    # longer than the kernel) does not throttle the device.  One untimed
    # replay precedes the timed one.
    graph = torch.cuda.CUDAGraph()
    capture_stream = torch.cuda.Stream(device)
    capture_stream.wait_stream(stream)
    with torch.cuda.graph(graph, stream=capture_stream):
        for step in range(args.steps):
            one_step(step, capture_stream.cuda_stream)
    stream.wait_stream(capture_stream)
    graph.replay()
    torch.cuda.synchronize()
    replay_begin = torch.cuda.Event(enable_timing=True)
    replay_end = torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    replay_begin.record(stream)
    graph.replay()
    replay_end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms_per_step = replay_begin.elapsed_time(replay_end) / args.steps

    # Kernel duration for the roofline.  In one pass or with the in-kernel
    # merge a step is exactly one launch, so the graph replay's time per step
    # is the kernel's duration (plus the graph's inter-launch gap).  With the
    # separate merge, K split-stage launches alone are captured in a second
    # graph and timed the same way.
    if fused or one_pass:
        split_ms = ms_per_step
        kernel_timing = "HIP events around the timed graph replay; one launch per step"
    else:
        split_graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(split_graph, stream=capture_stream):
            for step in range(args.steps):
                split_stage(step % args.pools, capture_stream.cuda_stream)
        stream.wait_stream(capture_stream)
        split_graph.replay()
        torch.cuda.synchronize()
        split_begin = torch.cuda.Event(enable_timing=True)
        split_end = torch.cuda.Event(enable_timing=True)
        split_begin.record(stream)
        split_graph.replay()
        split_end.record(stream)
        torch.cuda.synchronize()
        split_ms = split_begin.elapsed_time(split_end) / args.steps
        kernel_timing = ("HIP events around a graph replay of K split-stage launches "
                         "(the merge launch excluded)")

    lengths = case.lengths
    nbytes = decode_attention_bytes(lengths, query_heads, kv_heads, head_dim, block_size, 2)
    value = nbytes / (ms_per_step * 1e-3) / 1e9
    achieved = nbytes / (split_ms * 1e-3) / 1e9
    # Counter traffic is reported only when the committed profile was taken of
    # this very launch (kernel, plan and load form); otherwise null.
    launch_signature = (f"{'mfma' if variant == _native.TF_ATTENTION_MFMA else 'generic'}"
                        f"|{'one_pass' if one_pass else 'split_kv'}|waves={plan.waves_per_head}"
                        f"|tokens_per_wave={plan.tokens_per_wave}|split={split_size}"
                        f"|merge={args.merge}|abi={lib.tf_abi_version()}")
    traffic = None
    if TRAFFIC_FILE.exists():
        profiled = json.loads(TRAFFIC_FILE.read_text())
        if profiled.get("launch") == launch_signature:
            traffic = profiled.get("hbm_bytes_per_launch")
    num_blocks = gpu.key_cache.shape[0]
    page_bytes = gpu.key_cache[0].numel() * gpu.key_cache.element_size()
    ceiling = read_ceiling(nbytes, gather={
        "pools": pools, "pages": call_pages(case.block_tables, lengths, block_size).to(device),
        "page_bytes": page_bytes, "num_blocks": num_blocks})

    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "paged GQA decode attention, TinyLlama geometry (BASELINE config 2)",
            "batch": 64,
            "padded_rows": 8,
            "query_heads": query_heads,
            "kv_heads": kv_heads,
            "head_dim": head_dim,
            "page_size": block_size,
            "context": "U[128,2048], seed 0",
            "sum_context": sum(lengths),
            "kernel": "mfma" if variant == _native.TF_ATTENTION_MFMA else "generic",
            "plan": "one_pass" if one_pass else "split_kv",
            "split_size": split_size,
            "num_splits": num_splits,
            "waves_per_kv_head": plan.waves_per_head,
            "kv_pools_rotated": args.pools,
            "merge": ("none (one pass)" if one_pass
                      else "in-kernel (arrival counters)" if fused else "separate merge launch"),
            "algorithmic_bytes_per_call": nbytes,
            "algorithmic_flops_per_call": decode_attention_flops(lengths, query_heads, head_dim),
        },
        "hbm_fraction": round(value / HBM_PEAK_GBS, 4),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "launch": launch_signature,
            "ceiling": ceiling,
            "frac_of_ceiling": round(achieved / ceiling["read_1GiB"], 4),
            "frac_of_same_size_read": round(achieved / ceiling["read_same_bytes"], 4),
            "frac_of_page_gather": round(achieved / ceiling["gather_call_pages"], 4),
            "kernel": "paged_decode_mfma_kernel"
            + (" (one pass, the whole call)" if one_pass
               else " (split stage with in-kernel merge)" if fused else " (split stage)"),
            "merge_ms": None if (fused or one_pass) else round(ms_per_step - split_ms, 6),
            "timing": kernel_timing,
            "kernel_ms": round(split_ms, 6),
        },
        "timing": "K steps captured in one HIP graph, one timed replay",
        "wall_s_timed_loop": round(wall, 4),
    }
    if not args.no_cpu_baseline:
        active = [row for row, ctx in enumerate(lengths) if ctx > 0]
        result["cpu_baseline"] = cpu_baseline(case, active, args.cpu_seconds)
    if not args.no_decode_step:
        result["decode_step"] = decode_step(lengths, args.cpu_seconds, not args.no_cpu_baseline)
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
