"""Pinning the encoder oracles with closed forms (CPU).

Each check is independent of the restated formula: neighbours come from an
enumeration of the target format, probabilities from exact rational
arithmetic or brute force over every random word, nearest rounding from
torch's own conversions, and the two oracles (torch restatement and C
restatement, different formulations) must agree bit for bit.
Mirrors tests/test_sr_edge_cases.py, tests/test_minifloat.py,
tests/test_seed_reproducibility.py and benchmarks/cast_checks.py.
"""

from __future__ import annotations

from fractions import Fraction

import pytest
import torch
from _cases import (
    all_values,
    bf16_bracket,
    boundary_inputs,
    cast_cases,
    oracle_neighbors,
    positive_grid,
    random_words,
    rn_midpoint_words,
)
from conftest import RULES, STATE_DTYPES, assert_bits_or_nan

from oracle import c_oracle, sr_oracle

MINIFLOATS = (torch.float8_e4m3fn, torch.float8_e5m2, torch.float16)


# ---------------------------------------------------------------------------
# The two oracles agree everywhere we can look.
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", STATE_DTYPES)
@pytest.mark.parametrize("rounding", RULES)
def test_c_and_torch_oracles_agree(dtype, rounding):
    parts = [random_words(200_003, 17), torch.randn(50_000, generator=torch.Generator().manual_seed(3)) * 1e3]
    if dtype in MINIFLOATS:
        parts.append(boundary_inputs(dtype))
    x = torch.cat(parts)
    for seed, offset in ((0, 0), (2**32 + 9, 2**32 - 17), (-5, 123456789)):
        options = {"dtype": dtype, "rounding": rounding, "seed": seed, "offset": offset}
        assert_bits_or_nan(c_oracle.cast(x, **options), sr_oracle.cast(x, **options), str(options))


# ---------------------------------------------------------------------------
# BF16 stochastic rounding (sr_states/_bf16.py:37-74)
# ---------------------------------------------------------------------------
def test_bf16_sr_output_is_a_neighbour_and_exact_values_are_fixed():
    gen = torch.Generator().manual_seed(123)
    x = torch.cat([torch.randn(20_000, generator=gen) * 100, torch.randn(20_000, generator=gen) * 1e-30])
    out = sr_oracle.stochastic_round_bf16(x, seed=7).float()
    lo, hi = bf16_bracket(x)
    ok = (out == lo) | (out == hi) | ((x.abs() < 1e-38) & (out.abs() <= hi.abs().clamp_min(lo.abs())))
    assert torch.all(ok)
    exact = (torch.arange(65536, dtype=torch.int64) << 16).to(torch.int32).view(torch.float32)
    assert_bits_or_nan(sr_oracle.stochastic_round_bf16(exact, seed=999), exact.to(torch.bfloat16))
    assert_bits_or_nan(c_oracle.cast(exact, dtype=torch.bfloat16, seed=999), exact.to(torch.bfloat16))


def test_bf16_sr_probability_is_exact_over_every_random_word(monkeypatch):
    """With the hash replaced by the identity, word r = index: brute force all 2^16 words.

    Unbiased rounding means exactly low16(bits) of the 65536 words round away
    from zero, and they are the largest words (a threshold rule).
    """
    monkeypatch.setattr(sr_oracle, "u32_hash", lambda indices, seed: indices & 0xFFFFFFFF)
    for word in (0x3F800001, 0x3F807FFF, 0x3F808000, 0x3F80FFFF, 0xBF812345, 0x00000001, 0x7F7FFFFF):
        x = torch.tensor([word], dtype=torch.int64).to(torch.int32).view(torch.float32).repeat(65536)
        out = sr_oracle.stochastic_round_bf16(x, seed=0).view(torch.int16).to(torch.int32) & 0xFFFF
        truncated = (word >> 16) & 0xFFFF
        up = out != truncated
        low = word & 0xFFFF
        assert int(up.sum()) == low
        assert torch.equal(up, torch.arange(65536) >= 65536 - low)


def test_bf16_specials_and_payload_nan():
    values = torch.tensor([0.0, -0.0, 1.5, -2.0, float("inf"), -float("inf"), float("nan")])
    for fn in (lambda t: sr_oracle.stochastic_round_bf16(t, seed=999),
               lambda t: c_oracle.cast(t, dtype=torch.bfloat16, seed=999)):
        out = fn(values)
        assert torch.equal(out[:6], values[:6].to(torch.bfloat16))
        assert torch.signbit(out[1]) and torch.isnan(out[6])
        low_payload = torch.tensor([0x7F800001, 0xFF800001], dtype=torch.int64).to(torch.int32).view(torch.float32)
        assert torch.isnan(fn(low_payload)).all()


def test_bf16_cast_check_cases_and_rn_midpoints():
    """benchmarks/cast_checks.py cases: both oracles agree; RN equals torch's conversion."""
    for x, seed, offset in cast_cases():
        assert_bits_or_nan(
            c_oracle.cast(x.reshape(-1), dtype=torch.bfloat16, seed=seed, offset=offset),
            sr_oracle.stochastic_round_bf16(x, seed=seed, offset=offset).reshape(-1),
        )
    x = rn_midpoint_words()
    for fn in (sr_oracle.cast, c_oracle.cast):
        assert_bits_or_nan(fn(x, dtype=torch.bfloat16, rounding="nearest"), x.to(torch.bfloat16))


def test_partition_and_seed_periodicity():
    """tests/test_seed_reproducibility.py:13-36."""
    x = torch.linspace(-3, 7, 10_003)
    whole = sr_oracle.stochastic_round_bf16(x, seed=99, offset=1000)
    split = 4096
    parts = torch.cat([sr_oracle.stochastic_round_bf16(x[:split], seed=99, offset=1000),
                       sr_oracle.stochastic_round_bf16(x[split:], seed=99, offset=1000 + split)])
    assert torch.equal(whole, parts)
    for periods in (-(2**60), -1, 1, 2**60):
        shifted = sr_oracle.stochastic_round_bf16(x, seed=99 + periods * 2**32, offset=1000 + periods * 2**32)
        assert torch.equal(shifted, whole)
    y = torch.full((4096,), 1.0 + 2.0**-9)
    assert not torch.equal(sr_oracle.stochastic_round_bf16(y, seed=1), sr_oracle.stochastic_round_bf16(y, seed=2))


@pytest.mark.statistical
def test_bf16_sr_is_unbiased_statistically():
    n, lower, ulp, p_up = 200_000, 1.0, 2.0**-7, 0.25
    x = torch.full((n,), lower + p_up * ulp)
    out = sr_oracle.stochastic_round_bf16(x, seed=2026).float()
    freq = (out > lower).float().mean().item()
    assert abs(freq - p_up) < 6 * (p_up * (1 - p_up) / n) ** 0.5


# ---------------------------------------------------------------------------
# Minifloats (sr_states/_minifloat.py:10-70)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", MINIFLOATS)
@pytest.mark.parametrize("rounding", RULES)
def test_every_finite_encoding_is_fixed(dtype, rounding):
    values = all_values(dtype).float()
    values = values[torch.isfinite(values)]
    for fn in (sr_oracle.cast, c_oracle.cast):
        got = fn(values, dtype=dtype, rounding=rounding, seed=913, offset=2**32 - 17)
        assert_bits_or_nan(got, values.to(dtype))


@pytest.mark.parametrize("dtype", MINIFLOATS)
def test_sr_brackets_and_rn_matches_torch_conversion(dtype):
    x = torch.cat((boundary_inputs(dtype), random_words(10_003, 71)))
    lo, hi = oracle_neighbors(x, dtype)
    result = sr_oracle.cast(x, dtype=dtype, seed=2**32 + 9).float()
    finite = ~torch.isnan(x)
    assert torch.all((result[finite] == lo[finite]) | (result[finite] == hi[finite]))
    assert torch.equal(torch.signbit(result[finite]), torch.signbit(x[finite]))
    assert torch.equal(torch.isnan(result), torch.isnan(x))
    maximum = torch.finfo(dtype).max
    expected = x.to(dtype) if dtype == torch.float16 else x.clamp(-maximum, maximum).to(dtype)
    for fn in (sr_oracle.cast, c_oracle.cast):
        assert_bits_or_nan(fn(x, dtype=dtype, rounding="nearest"), expected)
    grid = positive_grid(dtype)
    mid = (grid[:-1] + grid[1:]) * 0.5
    even = torch.where(torch.arange(mid.numel()) % 2 == 0, grid[:-1], grid[1:])
    for fn in (sr_oracle.cast, c_oracle.cast):
        assert_bits_or_nan(fn(mid, dtype=dtype, rounding="nearest"), even.to(dtype))


@pytest.mark.parametrize("dtype", MINIFLOATS)
def test_sr_matches_exact_rational_thresholds(dtype):
    """tests/test_minifloat.py:226-251: up iff (hash >> 8) < floor(frac * 2^24), exactly."""
    gen = torch.Generator().manual_seed(904)
    x = torch.randint(0, 2**31 - 1, (2003,), dtype=torch.int32, generator=gen).view(torch.float32)
    x = x[torch.isfinite(x) & (x <= torch.finfo(dtype).max)]
    lower, upper = oracle_neighbors(x, dtype)
    threshold = [
        0 if lo == hi else int((Fraction(v) - Fraction(lo)) / (Fraction(hi) - Fraction(lo)) * 2**24)
        for v, lo, hi in zip(x.tolist(), lower.tolist(), upper.tolist())
    ]
    seed, offset = 71, 2**32 - 91
    k = sr_oracle.u32_hash(torch.arange(x.numel(), dtype=torch.int64) + offset, seed) >> 8
    expected = torch.where(k < torch.tensor(threshold), upper, lower)
    for sign in (1.0, -1.0):
        for fn in (sr_oracle.cast, c_oracle.cast):
            got = fn(x * sign, dtype=dtype, seed=seed, offset=offset)
            assert_bits_or_nan(got, (expected * sign).to(dtype))


@pytest.mark.parametrize("dtype", MINIFLOATS)
def test_probability_resolution_and_strict_threshold(dtype, monkeypatch):
    """tests/test_minifloat.py:178-192: words k = 0..3 with R = 0..3 round up iff k < R."""
    step = positive_grid(dtype)[1].item()
    monkeypatch.setattr(sr_oracle, "u32_hash", lambda indices, seed: torch.arange(4, dtype=torch.int64) << 8)
    for r in (0, 1, 2, 3):
        x = torch.full((4,), step * (r + 0.5) * 2**-24)
        result = sr_oracle.cast(x, dtype=dtype).float()
        assert torch.equal(result == step, torch.arange(4) < r)


@pytest.mark.parametrize("dtype", MINIFLOATS)
@pytest.mark.parametrize("rounding", RULES)
def test_exceptional_values_and_signed_zero(dtype, rounding):
    """tests/test_minifloat.py:128-150."""
    maximum = torch.finfo(dtype).max
    tiny = positive_grid(dtype)[1].item() * 2**-25
    x = torch.tensor([0.0, -0.0, tiny, -tiny, maximum * 2, -maximum * 2, float("inf"), -float("inf"), float("nan")])
    for fn in (sr_oracle.cast, c_oracle.cast):
        result = fn(x, dtype=dtype, rounding=rounding).float()
        assert torch.equal(result[:4].view(torch.int32), x[:4].mul(0).view(torch.int32))
        expected = float("inf") if dtype == torch.float16 else maximum
        assert torch.equal(result[4:8], torch.tensor([expected, -expected, expected, -expected]))
        assert torch.isnan(result[-1])


@pytest.mark.parametrize("dtype", MINIFLOATS)
def test_decode_matches_torch_for_every_encoding(dtype):
    raw = all_values(dtype)
    words = raw.view(torch.uint8 if dtype != torch.float16 else torch.int16).to(torch.int64) & 0xFFFF
    code = c_oracle.CODES[dtype]
    decoded = torch.tensor([c_oracle.lib().oc_decode(int(w), code) for w in words.tolist()])
    assert_bits_or_nan(decoded, raw.float())


@pytest.mark.statistical
@pytest.mark.parametrize("dtype", MINIFLOATS)
def test_round_up_probability(dtype):
    grid = positive_grid(dtype)
    lo, hi = 1.0, grid[torch.searchsorted(grid, torch.tensor(1.0)) + 1].item()
    value = torch.tensor(lo + (hi - lo) * 0.3).item()
    p = int(Fraction(value - lo) / Fraction(hi - lo) * 2**24) / 2**24
    count = 200_003
    result = sr_oracle.cast(torch.full((count,), value), dtype=dtype, seed=93, offset=2**32 - 41).float()
    freq = (result == hi).double().mean().item()
    assert abs(freq - p) < 6 * (p * (1 - p) / count) ** 0.5


def test_oracle_bf16_neighbors_match_enumeration():
    """sr_oracle.bf16_neighbors (sr_states/_bf16.py:77-101) against enumeration."""
    gen = torch.Generator().manual_seed(5)
    words = random_words(50_000, 6)
    boundary = torch.tensor([0x00000001, 0x00008000, 0x0000FFFF, 0x00010000, 0x3F807FFF, 0x3F808000,
                             0x3F808001, 0x7F7F7FFF, 0x7F7F8000, 0x7F7FFFFF], dtype=torch.int64)
    boundary = torch.cat((boundary, boundary | 0x80000000)).to(torch.int32).view(torch.float32)
    x = torch.cat([torch.randn(20_000, generator=gen) * 100, torch.randn(20_000, generator=gen) * 1e-39,
                   torch.tensor([1.5, -2.0, 0.0, -0.0]), boundary, words[torch.isfinite(words)]])
    lower, upper = sr_oracle.bf16_neighbors(x)
    lo, hi = bf16_bracket(x)
    assert torch.equal(lower.float(), lo) and torch.equal(upper.float(), hi)
    assert torch.equal(torch.signbit(lower.float()), torch.signbit(x))
    assert torch.equal(torch.signbit(upper.float()), torch.signbit(x))
    special = torch.tensor([float("inf"), -float("inf"), float("nan")])
    lower, upper = sr_oracle.bf16_neighbors(special)
    assert_bits_or_nan(lower, special.to(torch.bfloat16))
    assert_bits_or_nan(upper, special.to(torch.bfloat16))


@pytest.mark.parametrize("dtype", MINIFLOATS)
def test_oracle_minifloat_neighbors_match_enumerated_grid(dtype):
    """sr_oracle.minifloat_neighbors (sr_states/_minifloat.py:73-99), tests/test_minifloat.py:94-100."""
    x = boundary_inputs(dtype)
    lower, upper = sr_oracle.minifloat_neighbors(x, dtype=dtype)
    expected_lower, expected_upper = oracle_neighbors(x, dtype)
    assert_bits_or_nan(lower, expected_lower.to(dtype))
    assert_bits_or_nan(upper, expected_upper.to(dtype))
