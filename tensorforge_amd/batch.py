"""Batch execution contract between the decode executor and a scheduler
(reference: tensorforge/runtime/batch.py:11-31).

An executor step takes a token (or a whole prompt) per request and returns
the last position's logits of every request that ran, plus an error
message for every request that could not run: an input token outside the
vocabulary, a cache reservation that could not be made, or a failed
launch.  A failure is confined to its request; the others run.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Protocol

from torch import Tensor


@dataclass(frozen=True, slots=True)
class BatchExecutionResult:
    logits: dict[str, Tensor]
    errors: dict[str, str]


class BatchTokenExecutor(Protocol):
    @property
    def vocab_size(self) -> int: ...

    def create_request(self, request_id: str) -> None: ...

    def release_request(self, request_id: str) -> None: ...

    def append_tokens(self, tokens: dict[str, int]) -> BatchExecutionResult: ...


class BatchPrefillExecutor(Protocol):
    def prefill_prompts(self, prompts: dict[str, tuple[int, ...]]) -> BatchExecutionResult: ...
