"""Seeded sweep of the decode-shaped linear layers over drawn shapes.

Each case draws fp16 or bf16, 1-64 rows, 1-3000 output columns (any
remainder of the 16- and 64-column tiles), K a multiple of 32 from 32 to
6144 (chunk remainders, K quarters that leave wavefronts idle), and
column-sliced x and output buffers.  It runs ``linear_rows``,
``linear_stream`` (rounded output, and split-K partials summed on the
host), ``linear_kstream`` with each epilogue (plain, the RMSNorm of x's rows,
the residual add) and ``linear_swiglu`` in both forms (with and without the
norm for the K-split one) against fp32 torch on the same inputs.

Tolerance: the reference's elementwise bars (tests/test_triton_kernels.py
:21-26 of the reference: fp16 3e-3, bf16 3e-2) relative to the largest
magnitude of the fp32 result, plus one rounding of the intermediate the
kernel rounds (the residual sum's product, the SwiGLU's gate and up).
"""

from __future__ import annotations

import random

import pytest
import torch

from tensorforge_amd.kernels import (
    linear_kstream,
    linear_rows,
    linear_stream,
    linear_swiglu,
)

CASES = 32
TOLERANCE = {torch.float16: 3e-3, torch.bfloat16: 3e-2}


def draw(seed: int) -> dict:
    """One case of the sweep, a function of the seed only."""

    rng = random.Random(104729 * seed + 3)
    return {
        "dtype": rng.choice([torch.bfloat16, torch.float16]),
        "rows": rng.choice([1, 2, 7, 16, 17, 31, 33, 48, 63, 64, rng.randint(1, 64)]),
        "n": rng.choice([16, 48, 100, 257, 1000, 2048, 2560, rng.randint(1, 3000)]),
        "k": 32 * rng.choice([1, 3, 8, 31, 64, 65, 100, 176, rng.randint(1, 192)]),
        "x_pad": 8 * rng.randint(0, 4),
        "y_pad": rng.randint(0, 9),
        "splits": rng.choice([2, 3, 5, 8]),
    }


def _slices(k: int, wanted: int) -> int:
    """The most K slices up to ``wanted`` that cut K's 32-wide steps into
    non-empty slices of equal whole steps (the last one shorter)."""

    steps = k // 32
    for splits in range(min(wanted, steps), 0, -1):
        per = -(-steps // splits)
        if -(-steps // per) == splits:
            return splits
    return 1


def test_the_sweep_reaches_the_tile_and_chunk_remainders():
    """The drawn shapes cover what the sweep is for (host only)."""

    cases = [draw(seed) for seed in range(CASES)]
    assert {c["dtype"] for c in cases} == {torch.bfloat16, torch.float16}
    assert any(c["n"] % 16 for c in cases) and any(c["n"] % 64 for c in cases)
    assert any((c["k"] // 32) % 4 for c in cases)   # K quarters of unequal length
    assert any(c["k"] < 128 for c in cases) and any(c["k"] > 4096 for c in cases)
    assert any(c["rows"] > 32 for c in cases) and any(c["rows"] == 1 for c in cases)
    assert all(_slices(c["k"], c["splits"]) >= 1 for c in cases)
    assert any(_slices(c["k"], c["splits"]) > 1 for c in cases)


def _close(actual, expected, dtype, what, extra=0.0):
    tol = TOLERANCE[dtype]
    scale = max(float(expected.abs().max()), 1e-6)
    torch.testing.assert_close(actual.float().cpu(), expected, rtol=tol,
                               atol=tol * scale + extra, msg=lambda m: f"{what}: {m}")


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(CASES))
def test_drawn_shape_matches_fp32(device, seed):
    spec = draw(seed)
    dtype, m, n, k = spec["dtype"], spec["rows"], spec["n"], spec["k"]
    what = f"seed {seed}: {dtype} [{m}x{k}]x[{k}x{n}]"
    generator = torch.Generator().manual_seed(seed)
    x_wide = torch.randn(m, k + spec["x_pad"], generator=generator).to(dtype)
    x_cpu = x_wide[:, spec["x_pad"]:]
    w_cpu = (torch.randn(n, k, generator=generator) * 0.02).to(dtype)
    r_cpu = torch.randn(m, n, generator=generator).to(dtype)
    x = x_wide.to(device)[:, spec["x_pad"]:]
    w = w_cpu.to(device)
    xf, wf = x_cpu.float(), w_cpu.float()
    expected = xf @ wf.T

    def out_buffer(cols):
        wide = torch.full((m, cols + spec["y_pad"]), float("nan"), dtype=dtype, device=device)
        return wide, wide[:, :cols]

    wide, out = out_buffer(n)
    linear_rows(x, w, output=out)
    _close(out, expected, dtype, f"{what} linear_rows")
    assert bool(wide[:, n:].isnan().all()), what

    wide, out = out_buffer(n)
    linear_stream(x, w, output=out)
    _close(out, expected, dtype, f"{what} linear_stream")
    assert bool(wide[:, n:].isnan().all()), what
    splits = _slices(k, spec["splits"])
    partials = torch.empty(splits, m, n, dtype=torch.float32, device=device)
    linear_stream(x, w, splits=splits, partials=partials)
    _close(partials.sum(0), expected, torch.float16, f"{what} linear_stream {splits} slices")

    wide, out = out_buffer(n)
    linear_kstream(x, w, output=out)
    _close(out, expected, dtype, f"{what} linear_kstream")
    assert bool(wide[:, n:].isnan().all()), what

    eps = 1e-5
    inv = torch.rsqrt(xf.square().mean(dim=-1, keepdim=True) + eps)
    wide, out = out_buffer(n)
    linear_kstream(x, w, output=out, norm_eps=eps)
    _close(out, (xf * inv) @ wf.T, dtype, f"{what} linear_kstream norm")

    wide, out = out_buffer(n)
    linear_kstream(x, w, output=out, residual=r_cpu.to(device))
    rounded = expected.to(dtype).float()
    _close(out, rounded + r_cpu.float(), dtype, f"{what} linear_kstream residual",
           extra=TOLERANCE[dtype] * float(r_cpu.float().abs().max()))

    # SwiGLU over a stacked [2I, K] weight (I = n rounded down to even).
    inter = max(n // 2, 1)
    gu_cpu = w_cpu[: 2 * inter] if 2 * inter <= n else torch.cat([w_cpu, w_cpu])[: 2 * inter]
    gu = gu_cpu.contiguous().to(device)
    for k_split, norm in ((False, False), (True, False), (True, True)):
        xin = xf * inv if norm else xf
        g_u = (xin @ gu_cpu.float().T).to(dtype).float()
        g, u = g_u[:, :inter], g_u[:, inter:]
        want = g * torch.sigmoid(g) * u
        wide, out = out_buffer(inter)
        linear_swiglu(x, gu, output=out, k_split=k_split, norm_eps=eps if norm else None)
        _close(out, want, dtype, f"{what} linear_swiglu k_split={k_split} norm={norm}",
               extra=TOLERANCE[dtype] * float(want.abs().max()))
        assert bool(wide[:, inter:].isnan().all()), what
