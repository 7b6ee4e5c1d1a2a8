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
    in for e.  ``max_flip_rate`` caps the share of flipped tokens (0 makes
    the check one of identity).  Flips are counted and printed either way
    (``pytest -rP`` shows them), and every failure message carries the
    counts.
    """

    def __init__(self, weights, *, bound: float | None = None, device="cpu",
                 dtype=torch.float32, name: str = "", max_flip_rate: float | None = None,
                 tolerance: tuple[float, float] | None = None) -> None:
        """``bound``: the stated largest |device logit - oracle logit|; or
        ``tolerance=(atol, rtol)``: the bound is ``atol + rtol * L`` with L
        the largest |oracle logit| of the checked rows (a reference-style
        tolerance at the run's own logit magnitude)."""

        if (bound is None) == (tolerance is None):
            raise ValueError("give either bound or tolerance")
        self.weights = weights
        self._bound = bound
        self.tolerance = tolerance
        self.max_logit = 0.0
        self.device = device
        self.dtype = dtype
        self.name = name
        # Flip budget: at most this fraction of the checked tokens may
        # differ from the oracle's argmax (None: no budget beyond the margin
        # rule; 0: identity).
        self.max_flip_rate = max_flip_rate
        self.flips: list[tuple] = []
        self.tokens = 0
        self.max_dlogit = 0.0
        self.min_margin = float("inf")
        self.margins: list[float] = []  # the oracle's top-two margin at every token

    def check(self, request_id, prompt, generated, logits=None) -> None:
        from oracle.model import decoder_forward

        tokens = torch.tensor(list(prompt) + list(generated[:-1]), dtype=torch.long)
        expected = decoder_forward(self.weights, tokens, device=self.device, dtype=self.dtype)
        rows = expected[len(prompt) - 1:]
        assert rows.shape[0] == len(generated)
        self.max_logit = max(self.max_logit, float(rows.abs().max()))
        if logits is not None:
            got = torch.stack([row.float().cpu() for row in logits])
            assert got.shape == rows.shape
            self.max_dlogit = max(self.max_dlogit, float((got - rows).abs().max()))
        for step, token in enumerate(generated):
            row = rows[step]
            top = torch.topk(row, 2).values
            self.min_margin = min(self.min_margin, float(top[0] - top[1]))
            self.margins.append(float(top[0] - top[1]))
            best = int(torch.argmax(row))
            self.tokens += 1
            if token != best:
                self.flips.append((request_id, step, int(token), best, float(row[best] - row[token])))

    @property
    def bound(self) -> float:
        if self._bound is not None:
            return self._bound
        atol, rtol = self.tolerance
        return atol + rtol * self.max_logit

    def summary(self) -> dict:
        """Counts of the run so far: tokens, flips, the flip rate, the
        largest flip margin, the measured logit deviation, and how many
        tokens had an oracle margin within twice it (the only places a flip
        is allowed)."""

        measured = self.max_dlogit if self.max_dlogit > 0 else None
        e = measured if measured is not None else self.bound
        return {
            "tokens": self.tokens,
            "flips": len(self.flips),
            "flip_rate": round(len(self.flips) / max(self.tokens, 1), 5),
            "largest_flip_margin": round(max((f[4] for f in self.flips), default=0.0), 5),
            "max_dlogit": None if measured is None else round(measured, 5),
            "near_ties": sum(1 for m in self.margins if m <= 2 * e),
            "smallest_margin": round(self.min_margin, 6),
            "max_abs_oracle_logit": round(self.max_logit, 4),
            "logit_bound": round(self.bound, 5),
        }

    def finish(self) -> dict:
        measured = self.max_dlogit if self.max_dlogit > 0 else None
        e = measured if measured is not None else self.bound
        summary = self.summary()
        text = (f"[greedy parity] {self.name}: {summary} (stated logit bound {self.bound}, "
                f"flip budget {self.max_flip_rate}); flips (request, step, margin): "
                f"{[(r, s, round(m, 5)) for r, s, _, _, m in self.flips][:40]}")
        print(text)
        if measured is not None:
            assert measured <= self.bound, (
                f"max |dlogit| {measured:.4e} exceeds the stated bound {self.bound}: {text}")
        wide = [f for f in self.flips if f[4] > 2 * e]
        assert not wide, f"flips at margins above 2 x {e:.4e}: {wide}: {text}"
        if self.max_flip_rate is not None:
            assert len(self.flips) <= self.max_flip_rate * self.tokens, (
                f"flip rate above the budget {self.max_flip_rate}: {text}")
        return summary
