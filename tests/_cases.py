"""Seeded input sets and enumerated neighbours shared by the CPU and GPU tests.

The inputs restate the reference's own test inputs: the cast-check cases
(benchmarks/cast_checks.py:10-67), the minifloat boundary sets
(tests/test_minifloat.py:16-52) and the dyadic optimizer gradients
(tests/test_rng_streams.py:33-38).  ``bf16_bracket`` and
``oracle_neighbors`` find the neighbours of FP32 inputs by enumerating the
target format, independently of any rounding formula.
"""

from __future__ import annotations

import torch


def all_values(dtype: torch.dtype) -> torch.Tensor:
    """Every encoding of a 16- or 8-bit format, as that dtype."""
    if dtype in (torch.float16, torch.bfloat16):
        return torch.arange(65536, dtype=torch.int32).to(torch.int16).view(dtype)
    return torch.arange(256, dtype=torch.int32).to(torch.uint8).view(dtype)


def positive_grid(dtype: torch.dtype) -> torch.Tensor:
    """Sorted finite non-negative values of a format, as FP32."""
    values = all_values(dtype).float()
    return values[torch.isfinite(values) & ~torch.signbit(values)].sort().values


def boundary_inputs(dtype: torch.dtype) -> torch.Tensor:
    """Grid points, midpoints and their FP32 neighbours, extremes, specials (+/-)."""
    grid = positive_grid(dtype)
    mid = (grid[:-1] + grid[1:]) * 0.5
    up = torch.nextafter(mid, torch.full_like(mid, float("inf")))
    down = torch.nextafter(mid, torch.zeros_like(mid))
    maximum = float(torch.finfo(dtype).max)
    extra = torch.tensor(
        [maximum, maximum + 16, 2.0**-149, 2.0**-126, 1e-30, 1e30, float("inf"), float("nan")]
    )
    positive = torch.cat((grid, mid, up, down, extra))
    return torch.cat((positive, -positive))


def random_words(n: int, seed: int) -> torch.Tensor:
    """n uniformly random FP32 bit patterns (NaNs and Infs included)."""
    generator = torch.Generator().manual_seed(seed)
    bits = torch.randint(0, 2**32, (n,), generator=generator, dtype=torch.int64)
    return bits.to(torch.int32).view(torch.float32)


def cast_cases():
    """(x, seed, offset) triples of benchmarks/cast_checks.py:10-35."""
    generator = torch.Generator().manual_seed(91)
    for n in (0, 1, 127, 128, 129, 255, 257, 513, 4097, 100_003):
        bits = torch.randint(0, 2**32, (n,), generator=generator, dtype=torch.int64)
        yield bits.to(torch.int32).view(torch.float32), 7, 2**32 - 13
    exact = (torch.arange(65536, dtype=torch.int64) << 16).to(torch.int32)
    yield exact.view(torch.float32).reshape(256, 256), 0, 0
    boundaries = torch.tensor(
        [0, 1, 0x7FFF, 0x8000, 0xFFFF, 0x10000, 0x7FFFFF, 0x800000, 0x3F807FFF, 0x3F808000,
         0x3F808001, 0x7F7FFFFF, 0x7F800000, 0x7F800001, 0x7FC00000],
        dtype=torch.int64,
    )
    bits = torch.cat((boundaries, boundaries | 0x80000000)).to(torch.int32)
    for seed, offset in ((2**32 + 9, -17), (991, 2**32 - 31)):
        yield bits.view(torch.float32).repeat(19), seed, offset


def rn_midpoint_words() -> torch.Tensor:
    """Both sides of every positive finite BF16 midpoint, and their negatives."""
    high = torch.arange(0x7F80, dtype=torch.int64) << 16
    bits = (high[:, None] + torch.tensor([0x7FFF, 0x8000, 0x8001])).flatten()
    return torch.cat((bits, bits | 0x80000000)).to(torch.int32).view(torch.float32)


def dyadic_gradient(n: int = 1031) -> torch.Tensor:
    """1 + i/2048: FP32 AdamW/SGDM proposals from it are exact."""
    return 1.0 + torch.arange(n, dtype=torch.float32) / 2048


def bf16_bracket(x: torch.Tensor):
    """Independent BF16 neighbours of finite FP32 x by enumeration around RN(x)."""
    rn = x.to(torch.bfloat16).view(torch.int16).to(torch.int32)
    candidates = torch.stack([rn - 1, rn, rn + 1]).to(torch.int16).view(torch.bfloat16).float()
    xf = x[None, :]
    below = torch.where(candidates <= xf, candidates, torch.full_like(candidates, -float("inf")))
    above = torch.where(candidates >= xf, candidates, torch.full_like(candidates, float("inf")))
    # Across zero the integer neighbours of RN(x) are on the far side: sign-aware fix.
    return below.max(0).values, above.min(0).values


def oracle_neighbors(x, dtype):
    """Enumerated-grid neighbours after saturation (tests/test_minifloat.py:55-74)."""
    grid = positive_grid(dtype)
    a = x.abs()
    saturate = dtype != torch.float16
    if saturate:
        a = a.clamp_max(grid[-1].item())
    index = torch.searchsorted(grid, a)
    upper = grid[index.clamp_max(grid.numel() - 1)]
    exact = upper == a
    lower = torch.where(exact, upper, grid[(index - 1).clamp(0, grid.numel() - 1)])
    if not saturate:
        upper = torch.where(a > grid[-1], float("inf"), upper)
        lower = torch.where(torch.isinf(a), float("inf"), lower)
    lo = torch.copysign(torch.where(torch.signbit(x), upper, lower), x)
    hi = torch.copysign(torch.where(torch.signbit(x), lower, upper), x)
    lo = torch.where(torch.isnan(x), x, lo)
    hi = torch.where(torch.isnan(x), x, hi)
    return torch.minimum(lo, hi), torch.maximum(lo, hi)
