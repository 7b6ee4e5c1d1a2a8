"""The continuous-batching loop's host logic on the CPU, against a stub
executor with the decode executor's contract (launch / collect with tokens
fed back from the previous step, one step in flight).

The request lifecycle follows the reference's continuous policy
(scheduler/continuous.py:230-328): admission in arrival order up to the
batch limit, whole-prompt prefill, one token per running request per step,
completion at max_new_tokens with the cache released.
"""

from __future__ import annotations

from dataclasses import dataclass

import pytest

from tensorforge_amd.decode import DecodeStepRecord, DecodeTicket
from tensorforge_amd.serving import ContinuousServer, RequestSpec, summarize, synthetic_requests

VOCAB = 97


def next_token(token: int) -> int:
    return (token * 31 + 7) % VOCAB


@dataclass
class _Launched:
    tokens: dict[str, int]


class StubExecutor:
    """The executor contract without a GPU: a request that ran in the
    previous launched step continues from that step's sample; any other
    request needs a host token; at most a few steps are in flight."""

    vocab_size = VOCAB

    def __init__(self, fail_prefill: set[str] | None = None,
                 fail_step: dict[str, int] | None = None) -> None:
        # Requests whose prefill reports an error, and requests whose n-th
        # decode launch reports one (the executor's per-request errors).
        self.fail_prefill = set(fail_prefill or ())
        self.fail_step = dict(fail_step or {})
        self.launches: dict[str, int] = {}
        self.live: set[str] = set()
        self.max_live = 0
        self.created: list[str] = []
        self._previous: dict[str, int] = {}
        self._pending: dict[int, _Launched] = {}
        self._next = 0
        self.step_records: list[DecodeStepRecord] = []
        self.steps: list[tuple[str, ...]] = []

    def create_request(self, request_id: str) -> None:
        assert request_id not in self.live
        self.live.add(request_id)
        self.created.append(request_id)
        self.max_live = max(self.max_live, len(self.live))

    def release_request(self, request_id: str) -> None:
        self.live.remove(request_id)
        self._previous.pop(request_id, None)

    def prefill_tokens(self, prompts: dict[str, list[int]]) -> tuple[dict[str, int], dict[str, str]]:
        assert set(prompts) <= self.live
        errors = {rid: "CacheExhaustedError: no pages" for rid in prompts if rid in self.fail_prefill}
        return ({rid: len(prompt) % VOCAB for rid, prompt in prompts.items() if rid not in errors},
                errors)

    def launch(self, request_ids: list[str], tokens: dict[str, int] | None = None) -> DecodeTicket:
        tokens = tokens or {}
        inputs = {}
        errors = {}
        for rid in request_ids:
            assert rid in self.live, f"{rid} launched after release"
            self.launches[rid] = self.launches.get(rid, 0) + 1
            if self.fail_step.get(rid) == self.launches[rid]:
                errors[rid] = "CacheExhaustedError: no pages"
                continue
            if rid in tokens:
                inputs[rid] = tokens[rid]
            else:
                assert rid in self._previous, f"{rid} has no token to continue from"
                inputs[rid] = self._previous[rid]
        if not inputs:
            return DecodeTicket((), (0, 0), -1, errors)
        assert len(self._pending) < 3, "too many steps in flight"
        sampled = {rid: next_token(token) for rid, token in inputs.items()}
        self._previous = dict(sampled)
        slot = self._next
        self._next += 1
        self._pending[slot] = _Launched(sampled)
        staged = tuple(inputs)
        self.steps.append(staged)
        bucket = 1 << max(0, (len(staged) - 1).bit_length())
        self.step_records.append(DecodeStepRecord((bucket, 512), len(staged), 1.0))
        return DecodeTicket(staged, (bucket, 512), slot, errors)

    def collect(self, ticket: DecodeTicket) -> list[int]:
        if ticket.slot < 0:
            return []
        launched = self._pending.pop(ticket.slot)
        return [launched.tokens[rid] for rid in ticket.request_ids]


def _expected(prompt_length: int, count: int) -> list[int]:
    tokens = [prompt_length % VOCAB]
    while len(tokens) < count:
        tokens.append(next_token(tokens[-1]))
    return tokens


def _requests(lengths: list[int], outputs: list[int], gap_s: float = 0.0) -> list[RequestSpec]:
    return [RequestSpec(f"r{i}", tuple(range(n)), o, i * gap_s)
            for i, (n, o) in enumerate(zip(lengths, outputs))]


def test_burst_respects_the_batch_limit_and_generates_every_token() -> None:
    executor = StubExecutor()
    requests = _requests([5, 9, 3, 12, 7, 2, 30, 4, 8, 11], [6, 1, 9, 3, 4, 12, 2, 7, 5, 8])
    traces = ContinuousServer(executor, max_batch=4, progress_s=0).run(requests)
    assert executor.max_live <= 4
    assert executor.created == [r.request_id for r in requests]  # arrival order
    assert not executor.live  # every cache released
    for spec, trace in zip(requests, traces):
        assert trace.generated == _expected(len(spec.prompt), spec.max_new_tokens)
        assert trace.completed_ns is not None and trace.completed_ns >= trace.arrival_ns
        assert len(trace.token_ns) == spec.max_new_tokens
    # A request decodes max_new_tokens - 1 steps (the first token is prefill's).
    counts: dict[str, int] = {}
    for step in executor.steps:
        for rid in step:
            counts[rid] = counts.get(rid, 0) + 1
    assert counts == {r.request_id: r.max_new_tokens - 1 for r in requests
                      if r.max_new_tokens > 1}


def test_prefill_budget_limits_admission_per_iteration() -> None:
    executor = StubExecutor()
    calls: list[int] = []
    original = executor.prefill_tokens

    def counting(prompts):
        calls.append(len(prompts))
        return original(prompts)

    executor.prefill_tokens = counting
    requests = _requests([100, 100, 100, 40, 40], [3, 3, 3, 3, 3])
    ContinuousServer(executor, max_batch=8, max_prefill_tokens=150, progress_s=0).run(requests)
    # 100 alone (a second 100 exceeds the rest of the budget), then 100,
    # then 100 + 40 (within 150), then 40.
    assert calls == [1, 1, 2, 1]


def test_arrivals_follow_the_clock() -> None:
    executor = StubExecutor()
    requests = _requests([3, 3, 3], [2, 2, 2], gap_s=0.02)
    traces = ContinuousServer(executor, max_batch=4, progress_s=0).run(requests)
    starts = [t.started_ns for t in traces]
    assert starts == sorted(starts)
    assert all(t.started_ns >= t.arrival_ns for t in traces)
    assert (traces[2].arrival_ns - traces[0].arrival_ns) == pytest.approx(0.04e9, rel=1e-6)
    summary = summarize(traces, executor)
    assert summary["generated_tokens"] == 6 and summary["requests"] == 3
    assert summary["output_tokens_per_second"] > 0


def test_synthetic_requests_match_the_workload() -> None:
    requests = synthetic_requests(512, rate=20.0, vocab_size=32000, seed=0)
    lengths = [len(r.prompt) for r in requests]
    outputs = [r.max_new_tokens for r in requests]
    arrivals = [r.arrival_s for r in requests]
    assert min(lengths) >= 16 and max(lengths) <= 2048
    assert 200 <= sorted(lengths)[256] <= 320  # median near 256
    assert min(outputs) >= 64 and max(outputs) <= 512
    assert arrivals[0] == 0.0 and arrivals == sorted(arrivals)
    assert 20.0 < arrivals[-1] < 32.0  # 511 gaps of mean 50 ms
    assert all(0 <= t < 32000 for r in requests[:20] for t in r.prompt)
    burst = synthetic_requests(8, burst=True)
    assert all(r.arrival_s == 0.0 for r in burst)


def test_a_failed_decode_step_fails_only_its_request() -> None:
    """An executor error for one request mid-run (an exhausted cache at its
    third decode launch) completes that request with the error and releases
    it; every other request still gets all of its tokens
    (scheduler/continuous.py:284-299)."""

    executor = StubExecutor(fail_step={"r2": 3})
    requests = _requests([5, 9, 3, 12, 7], [6, 6, 6, 6, 6])
    traces = ContinuousServer(executor, max_batch=8, progress_s=0).run(requests)
    assert not executor.live  # every sequence released, the failed one too
    for spec, trace in zip(requests, traces):
        if spec.request_id == "r2":
            assert trace.error is not None and "CacheExhausted" in trace.error
            # prefill's token and the first two decode steps' samples, at most
            assert 1 <= len(trace.generated) <= 3
            assert trace.generated == _expected(3, len(trace.generated))
        else:
            assert trace.error is None
            assert trace.generated == _expected(len(spec.prompt), spec.max_new_tokens)
    summary = summarize(traces, executor)
    assert summary["failed_requests"] == 1 and summary["requests"] == 5


def test_a_failed_prefill_fails_only_its_request() -> None:
    executor = StubExecutor(fail_prefill={"r1"})
    requests = _requests([5, 9, 3], [4, 4, 4])
    traces = ContinuousServer(executor, max_batch=8, progress_s=0).run(requests)
    assert not executor.live
    assert traces[1].error is not None and traces[1].generated == []
    assert traces[0].generated == _expected(5, 4) and traces[2].generated == _expected(3, 4)
    assert "r1" not in {rid for step in executor.steps for rid in step}
