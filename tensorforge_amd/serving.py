"""Continuous batching over the graph-bucketed decode executor.

Drives BASELINE config 5: a TinyLlama-1.1B-geometry decoder (random init,
seed 0, bf16) serving 512 requests that arrive as a Poisson process at
20 req/s, prompt lengths lognormal (median 256, sigma 0.8 -- the spread is
not fixed by the workload, so it is stated here -- clipped to [16, 2048]),
output lengths uniform in [64, 512], token ids uniform over the vocabulary,
at most 64 requests in flight, 16-token pages, greedy sampling.

The request lifecycle restates the reference's continuous policy
(scheduler/continuous.py:230-328, 350-390): arrived requests queue; while
fewer than ``max_batch`` run, the oldest are admitted and prefilled whole
(its parallel-prefill mode, up to ``max_prefill_tokens`` prompt tokens per
iteration); every running request then decodes one token per step until it
has ``max_new_tokens``.  Unlike the reference, which reads every step's
argmax back before the next step (continuous.py:265-279), the loop keeps one
decode step in flight: step n+1 is launched with its tokens fed back on the
device before step n's tokens are read on the host.

Reported (the reference's definitions, metrics/statistics.py:40-98):
output tok/s = generated tokens / (last completion - first arrival),
time to first token, time per output token, request latency; plus
decode-only tok/s = sum of lanes / sum of decode-step device time, and the
per-bucket p50 step time.

``python -m tensorforge_amd.serving [--requests 512] [--rate 20] [--burst]``
prints one JSON line.
"""

from __future__ import annotations

import argparse
import json
import math
import random
import sys
import time
from collections import deque
from dataclasses import dataclass, field

import numpy as np
import torch

from tensorforge_amd.cache import CacheExhaustedError, PagedKVCache, PagedKVCacheConfig
from tensorforge_amd.decode import (
    BucketedDecodeExecutor,
    DecoderConfig,
    DecoderWeights,
    DecodeTicket,
    tinyllama_config,
)


@dataclass(frozen=True, slots=True)
class RequestSpec:
    request_id: str
    prompt: tuple[int, ...]
    max_new_tokens: int
    arrival_s: float


@dataclass(slots=True)
class RequestTrace:
    request_id: str
    prompt_tokens: int
    max_new_tokens: int
    arrival_ns: int
    started_ns: int | None = None
    token_ns: list[int] = field(default_factory=list)
    generated: list[int] = field(default_factory=list)
    completed_ns: int | None = None
    error: str | None = None  # set when the request failed (it still completes)


def synthetic_requests(count: int = 512, *, rate: float = 20.0, vocab_size: int = 32000,
                       median_prompt: int = 256, sigma: float = 0.8,
                       prompt_range: tuple[int, int] = (16, 2048),
                       output_range: tuple[int, int] = (64, 512), burst: bool = False,
                       seed: int = 0) -> list[RequestSpec]:
    """Poisson arrivals (exponential gaps at ``rate`` per second, the first at
    t=0; all at t=0 when ``burst``), lognormal prompt lengths, uniform output
    lengths and token ids."""

    rng = np.random.default_rng(seed)
    gaps = rng.exponential(1.0 / rate, size=count)
    arrivals = np.zeros(count) if burst else np.concatenate(([0.0], np.cumsum(gaps[1:])))
    lengths = np.clip(np.rint(rng.lognormal(math.log(median_prompt), sigma, size=count)),
                      *prompt_range).astype(int)
    outputs = rng.integers(output_range[0], output_range[1] + 1, size=count)
    return [RequestSpec(f"r{i:04d}", tuple(int(t) for t in rng.integers(0, vocab_size, size=n)),
                        int(o), float(a))
            for i, (n, o, a) in enumerate(zip(lengths, outputs, arrivals))]


class ContinuousServer:
    """Admission, prefill and pipelined decode over one executor.

    A request the executor cannot serve -- its prefill or one of its decode
    steps reports an error (an exhausted cache, an invalid token) -- fails
    alone: it is completed with the error recorded and its sequence
    released, and the other requests carry on (the reference fails only
    that request, scheduler/continuous.py:284-299).
    """

    def __init__(self, executor: BucketedDecodeExecutor, *, max_batch: int = 64,
                 max_prefill_tokens: int = 8192, progress_s: float = 5.0,
                 logits: dict[str, list] | None = None,
                 watch: dict[str, list] | None = None) -> None:
        """``logits`` (a dict to fill, for checkers): every step is read back
        before the next is launched and the fp32 logits row behind each
        sampled token is appended per request; the schedule is unchanged.

        ``watch`` (a dict keyed by request id, for checkers of the pipelined
        mode): the logits row behind each token of those requests is copied
        to the host as the steps run (``BucketedDecodeExecutor.watch_logits``)
        and appended to ``watch[request_id]`` in the model dtype; one step
        stays in flight as in serving."""

        self.executor = executor
        self.max_batch = max_batch
        self.max_prefill_tokens = max_prefill_tokens
        self.progress_s = progress_s
        self.logits = logits
        self.watch = watch

    def run(self, requests: list[RequestSpec]) -> list[RequestTrace]:
        executor = self.executor
        clock = time.perf_counter_ns
        t0 = clock()
        arrivals = deque(sorted(requests, key=lambda r: r.arrival_s))
        specs = {r.request_id: r for r in requests}
        traces: dict[str, RequestTrace] = {}
        queue: deque[str] = deque()
        running: list[str] = []      # decode order = lane order
        launched: dict[str, int] = {}  # tokens produced or in flight
        in_flight: DecodeTicket | None = None
        done = 0
        last_report = t0
        watch = self.watch
        if watch is not None:
            executor.watch_logits = set(watch)

        def finish(request_id: str, now: int, error: str | None = None) -> None:
            nonlocal done
            trace = traces[request_id]
            trace.completed_ns = now
            trace.error = error
            if request_id in running:
                running.remove(request_id)
            executor.release_request(request_id)
            done += 1

        while done < len(requests):
            now = clock()
            while arrivals and t0 + int(arrivals[0].arrival_s * 1e9) <= now:
                spec = arrivals.popleft()
                traces[spec.request_id] = RequestTrace(
                    spec.request_id, len(spec.prompt), spec.max_new_tokens,
                    t0 + int(spec.arrival_s * 1e9))
                queue.append(spec.request_id)
            # Admission and whole-prompt prefill.
            admitted: dict[str, list[int]] = {}
            budget = self.max_prefill_tokens
            while queue and len(running) + len(admitted) < self.max_batch:
                spec = specs[queue[0]]
                if admitted and len(spec.prompt) > budget:
                    break
                try:
                    executor.create_request(spec.request_id)
                except CacheExhaustedError:
                    break
                queue.popleft()
                traces[spec.request_id].started_ns = clock()
                admitted[spec.request_id] = list(spec.prompt)
                budget -= len(spec.prompt)
            host_tokens: dict[str, int] = {}
            if admitted:
                if self.logits is None and watch is not None and any(r in watch for r in admitted):
                    result = executor.prefill_prompts(admitted)
                    failed = dict(result.errors)
                    ids = list(result.logits)
                    first = {}
                    if ids:
                        stacked = torch.stack([result.logits[r] for r in ids])
                        first = dict(zip(ids, torch.argmax(stacked, dim=-1).tolist()))
                        for request_id in ids:
                            if request_id in watch:
                                watch[request_id].append(result.logits[request_id].cpu().clone())
                elif self.logits is None:
                    first, failed = executor.prefill_tokens(admitted)
                else:
                    result = executor.prefill_prompts(admitted)
                    failed = dict(result.errors)
                    first = {}
                    for request_id, row in result.logits.items():
                        self.logits[request_id] = [row.float().cpu()]
                        first[request_id] = int(torch.argmax(row))
                stamp = clock()
                for request_id, message in failed.items():
                    finish(request_id, stamp, message)
                for request_id, token in first.items():
                    trace = traces[request_id]
                    trace.generated.append(token)
                    trace.token_ns.append(stamp)
                    launched[request_id] = 1
                    running.append(request_id)
                    host_tokens[request_id] = token
                    if trace.max_new_tokens == 1:
                        finish(request_id, stamp)
            # Launch the next step before reading the previous one.
            order = [rid for rid in running if launched[rid] < specs[rid].max_new_tokens]
            ticket = None
            if order:
                ticket = executor.launch(order, {r: host_tokens[r] for r in order
                                                 if r in host_tokens})
                for request_id in ticket.request_ids:
                    launched[request_id] += 1
                for request_id, message in ticket.errors.items():
                    finish(request_id, clock(), message)
                if ticket.slot < 0:
                    ticket = None
            if self.logits is not None and ticket is not None:
                # Read this step back before the next launch, with its logits.
                if in_flight is not None:
                    raise RuntimeError("a recorded run keeps no step in flight")
                in_flight, ticket = ticket, None
                sampled = executor.collect(in_flight)
                for request_id, row in executor.logits_of(in_flight).items():
                    self.logits[request_id].append(row.float().cpu())
                stamp = clock()
                for request_id, token in zip(in_flight.request_ids, sampled):
                    trace = traces[request_id]
                    trace.generated.append(token)
                    trace.token_ns.append(stamp)
                    if len(trace.generated) >= trace.max_new_tokens:
                        finish(request_id, stamp)
                in_flight = None
            if in_flight is not None:
                sampled = executor.collect(in_flight)
                stamp = clock()
                rows = executor.watched_logits(in_flight) if watch is not None else {}
                for request_id, token in zip(in_flight.request_ids, sampled):
                    if request_id not in running:
                        continue  # failed in the step launched since
                    if request_id in rows:
                        watch[request_id].append(rows[request_id])
                    trace = traces[request_id]
                    trace.generated.append(token)
                    trace.token_ns.append(stamp)
                    if len(trace.generated) >= trace.max_new_tokens:
                        finish(request_id, stamp)
            in_flight = ticket
            if in_flight is None and not running and not queue and arrivals:
                wait = t0 + int(arrivals[0].arrival_s * 1e9) - clock()
                if wait > 0:
                    time.sleep(wait / 1e9)
            if self.progress_s and clock() - last_report > self.progress_s * 1e9:
                last_report = clock()
                print(f"[serve] {done}/{len(requests)} done, {len(running)} running, "
                      f"{len(queue)} queued, t={(last_report - t0) / 1e9:.1f}s",
                      file=sys.stderr, flush=True)
        if watch is not None:
            executor.watch_logits = set()
        return [traces[r.request_id] for r in requests]


def _percentiles(values: list[float]) -> dict[str, float]:
    if not values:
        return {}
    array = np.asarray(values, dtype=np.float64)
    return {f"p{q}": round(float(np.percentile(array, q)), 4) for q in (5, 50, 95)}


def summarize(traces: list[RequestTrace], executor: BucketedDecodeExecutor) -> dict:
    """The reference's serving metrics (metrics/statistics.py:40-98) plus
    the decode-only rate and per-bucket step time."""

    failed = [t for t in traces if t.error is not None]
    served = [t for t in traces if t.error is None]
    generated = sum(len(t.generated) for t in traces)
    first_arrival = min(t.arrival_ns for t in traces)
    last_completion = max(t.completed_ns for t in traces)
    ttft = [(t.token_ns[0] - t.arrival_ns) / 1e6 for t in served if t.token_ns]
    tpot = [(t.completed_ns - t.token_ns[0]) / (len(t.generated) - 1) / 1e6
            for t in served if len(t.generated) > 1]
    latency = [(t.completed_ns - t.arrival_ns) / 1e6 for t in served]
    records = executor.step_records
    lanes = sum(r.lanes for r in records)
    device_ms = sum(r.device_ms for r in records)
    buckets: dict[str, list[float]] = {}
    for record in records:
        buckets.setdefault(f"b{record.bucket[0]}-c{record.bucket[1]}", []).append(record.device_ms)
    return {
        "output_tokens_per_second": round(generated / ((last_completion - first_arrival) / 1e9), 1),
        "decode_tokens_per_second": round(lanes / (device_ms / 1e3), 1) if device_ms else None,
        "generated_tokens": generated,
        "requests": len(traces),
        "failed_requests": len(failed),
        "decode_steps": len(records),
        "mean_lanes_per_step": round(lanes / max(len(records), 1), 2),
        "ttft_ms": _percentiles(ttft),
        "tpot_ms": _percentiles(tpot),
        "request_latency_ms": _percentiles(latency),
        "step_ms_by_bucket": {key: {"steps": len(v), "p50": round(float(np.median(v)), 4)}
                              for key, v in sorted(buckets.items())},
    }


def build_executor(config: DecoderConfig, *, max_batch: int = 64, dtype=torch.bfloat16,
                   device: torch.device | str = "cuda", seed: int = 0,
                   max_sequence_length: int = 4096,
                   pages: int | None = None) -> BucketedDecodeExecutor:
    """Random-init weights and a paged cache whose pool holds ``max_batch``
    requests of 2048 prompt + 512 output tokens, handed out in a seeded
    random page order."""

    device = torch.device(device)
    weights = DecoderWeights.random(config, seed=seed, dtype=dtype, device=device)
    pages = pages or max_batch * ((2048 + 512) // 16)
    order = list(range(pages))
    random.Random(seed).shuffle(order)
    cache = PagedKVCache(
        PagedKVCacheConfig(num_layers=config.num_hidden_layers, num_blocks=pages, block_size=16,
                           num_kv_heads=config.num_key_value_heads, head_dim=config.head_dim,
                           max_sequences=max_batch, max_sequence_length=max_sequence_length,
                           dtype=dtype, device=device),
        page_order=order)
    buckets = tuple(b for b in (1, 2, 4, 8, 16, 32, 64, 128, 256) if b <= max_batch)
    contexts = tuple(c for c in (512, 1024, 2048, 4096) if c <= max_sequence_length)
    return BucketedDecodeExecutor(weights, cache, batch_buckets=buckets, context_buckets=contexts)


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--requests", type=int, default=512)
    parser.add_argument("--rate", type=float, default=20.0)
    parser.add_argument("--burst", action="store_true", help="all requests arrive at t=0")
    parser.add_argument("--max-batch", type=int, default=64)
    parser.add_argument("--seed", type=int, default=0)
    args = parser.parse_args()
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        return 1
    config = tinyllama_config()
    executor = build_executor(config, max_batch=args.max_batch, seed=args.seed)
    requests = synthetic_requests(args.requests, rate=args.rate, vocab_size=config.vocab_size,
                                  burst=args.burst, seed=args.seed)
    # Capture every bucket before the clock starts (the reference reports
    # setup and capture separately from steady state).
    setup_begin = time.perf_counter()
    warm = ContinuousServer(executor, max_batch=args.max_batch, progress_s=0)
    warm.run(synthetic_requests(args.max_batch, vocab_size=config.vocab_size, burst=True,
                                output_range=(2, 2), prompt_range=(16, 16), seed=args.seed + 1))
    executor.capture_all()
    executor.step_records.clear()
    setup_s = time.perf_counter() - setup_begin
    traces = ContinuousServer(executor, max_batch=args.max_batch).run(requests)
    summary = summarize(traces, executor)
    print(json.dumps({
        "workload": "cfg5 TinyLlama-1.1B geometry (22 layers, random init), "
                    + ("burst" if args.burst else f"Poisson {args.rate:g} req/s"),
        "requests": args.requests, "max_batch": args.max_batch, "dtype": "bf16",
        "prompt_lengths": "lognormal median 256 sigma 0.8 clipped [16, 2048]",
        "output_lengths": "uniform [64, 512]", "setup_s": round(setup_s, 2), **summary,
    }), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
