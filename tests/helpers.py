"""Comparison helpers shared by the parity tests."""

from __future__ import annotations

import torch
from torch import Tensor

# Tolerances of the reference's own kernel tests
# (tests/test_decode_attention.py:103, tests/test_triton_kernels.py:21-26).
REFERENCE_TOLERANCE = {torch.float32: 1e-5, torch.float16: 3e-3, torch.bfloat16: 3e-2}
# Bar of this build for bf16/fp16 outputs with fp32 accumulation:
# |actual - expected| <= 2e-2 + 1e-2 * |expected|.
NORTH_STAR_ATOL = 2e-2
NORTH_STAR_RTOL = 1e-2


def assert_close(actual: Tensor, expected: Tensor, atol: float, rtol: float, what: str = "") -> None:
    actual = actual.detach().cpu().float()
    expected = expected.detach().cpu().float()
    assert actual.shape == expected.shape, f"{what}: shape {actual.shape} != {expected.shape}"
    diff = (actual - expected).abs()
    bound = atol + rtol * expected.abs()
    bad = diff > bound
    if bool(bad.any()) or not bool(torch.isfinite(actual).all()):
        index = int(torch.argmax((diff - bound).flatten()))
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {bad.numel()} elements out of tolerance "
            f"(atol {atol}, rtol {rtol}); max abs diff {float(diff.max()):.3e}; "
            f"worst flat index {index}: actual {float(actual.flatten()[index]):.6f} "
            f"expected {float(expected.flatten()[index]):.6f}"
        )


def assert_bit_exact(actual: Tensor, expected: Tensor, what: str = "") -> None:
    actual = actual.detach().cpu().contiguous()
    expected = expected.detach().cpu().contiguous()
    assert actual.shape == expected.shape and actual.dtype == expected.dtype, what
    width = {1: torch.int8, 2: torch.int16, 4: torch.int32, 8: torch.int64}[actual.element_size()]
    mismatch = actual.view(width) != expected.view(width)
    assert not bool(mismatch.any()), f"{what}: {int(mismatch.sum())} elements differ bitwise"


class GreedyParity:
    """Greedy tokens of a decode run against a teacher-forced oracle.

    For each request the oracle runs one full-prefix forward over the prompt
    and the run's own tokens (but the last), so position i's logits are the
    ones the run's token i was sampled from.  A token that is not the
    oracle's argmax is a flip; ``margin`` is the oracle's logit gap between
    its argmax and the flipped token.

    If |device logit - oracle logit| <= e for every entry of a row, a flip
    there needs margin <= 2e.  So with the run's logits recorded, the
    measured e is checked against the stated bound and a flip at a larger
    margin fails (it would mean the sampled token is not the argmax of the
    device's own logits).  Without recorded logits the stated bound stands
    in for e.  Flips are counted and printed either way (``pytest -rP``
    shows them).
    """

    def __init__(self, weights, *, bound: float, device="cpu", dtype=torch.float32,
                 name: str = "") -> None:
        self.weights = weights
        self.bound = bound
        self.device = device
        self.dtype = dtype
        self.name = name
        self.flips: list[tuple] = []
        self.tokens = 0
        self.max_dlogit = 0.0
        self.min_margin = float("inf")

    def check(self, request_id, prompt, generated, logits=None) -> None:
        from oracle.model import decoder_forward

        tokens = torch.tensor(list(prompt) + list(generated[:-1]), dtype=torch.long)
        expected = decoder_forward(self.weights, tokens, device=self.device, dtype=self.dtype)
        rows = expected[len(prompt) - 1:]
        assert rows.shape[0] == len(generated)
        if logits is not None:
            got = torch.stack([row.float().cpu() for row in logits])
            assert got.shape == rows.shape
            self.max_dlogit = max(self.max_dlogit, float((got - rows).abs().max()))
        for step, token in enumerate(generated):
            row = rows[step]
            top = torch.topk(row, 2).values
            self.min_margin = min(self.min_margin, float(top[0] - top[1]))
            best = int(torch.argmax(row))
            self.tokens += 1
            if token != best:
                self.flips.append((request_id, step, int(token), best, float(row[best] - row[token])))

    def finish(self) -> None:
        measured = self.max_dlogit if self.max_dlogit > 0 else None
        e = measured if measured is not None else self.bound
        print(f"[greedy parity] {self.name}: {self.tokens} tokens, {len(self.flips)} flips "
              f"{[(r, s, round(m, 5)) for r, s, _, _, m in self.flips]}, max |dlogit| "
              f"{measured if measured is None else round(measured, 5)} (stated bound "
              f"{self.bound}), smallest oracle top-two margin {self.min_margin:.5f}")
        if measured is not None:
            assert measured <= self.bound, (
                f"{self.name}: max |dlogit| {measured:.4e} exceeds the stated bound {self.bound}")
        wide = [f for f in self.flips if f[4] > 2 * e]
        assert not wide, f"{self.name}: flips at margins above 2 x {e:.4e}: {wide}"
