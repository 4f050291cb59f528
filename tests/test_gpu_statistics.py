"""Stochastic rounding on the device is unbiased: Monte-Carlo checks with 6-sigma bounds.

Mirrors tests/test_sr_statistics.py (empirical round-up probability and mean
at a quarter ulp above 1.0; aggregate unbiasedness over 41 binades) for every
stochastic storage format, on the HIP cast with 2^22 draws instead of 2e5,
and extends it to the fused optimizers: one step from zero states stores
each SR moment as one of the two neighbours of its FP32 value, with the
round-up frequency that makes the stored mean equal the FP32 value.

The random stream is a hash of the element index, so "draws" are the
elements of one tensor; the bounds are the binomial ones of the reference's
tests.
"""

from __future__ import annotations

import math

import pytest
import torch
from conftest import raw_bits

pytestmark = [pytest.mark.gpu, pytest.mark.statistical]

N = 1 << 22
# Spacing of each format just above 1.0.
ULP_AT_ONE = {torch.bfloat16: 2.0**-7, torch.float16: 2.0**-10, torch.float8_e4m3fn: 2.0**-3,
              torch.float8_e5m2: 2.0**-2}
# Normal binades whose whole [2^e, 2^(e+1)) range stays below each format's
# largest finite value.
BINADES = {torch.bfloat16: range(-20, 21), torch.float16: range(-14, 15), torch.float8_e4m3fn: range(-6, 8),
           torch.float8_e5m2: range(-14, 15)}


@pytest.mark.parametrize("dtype", list(ULP_AT_ONE))
def test_empirical_up_probability_and_mean(cuda, dtype):
    """tests/test_sr_statistics.py:9-25, per stochastic format."""
    import sr_states

    ulp, p_up = ULP_AT_ONE[dtype], 0.25
    x_value = 1.0 + p_up * ulp
    x = torch.full((N,), x_value, device=cuda)
    out = sr_states.cast(x, dtype=dtype, seed=2026).float().cpu()
    assert set(torch.unique(out).tolist()) == {1.0, 1.0 + ulp}
    empirical = (out > 1.0).double().mean().item()
    standard_error = math.sqrt(p_up * (1 - p_up) / N)
    assert abs(empirical - p_up) < 6 * standard_error
    assert abs(out.double().mean().item() - x_value) < 6 * standard_error * ulp


@pytest.mark.parametrize("dtype", list(BINADES))
def test_distribution_stress_is_unbiased_in_aggregate(cuda, dtype):
    """tests/test_sr_statistics.py:28-36, per stochastic format, with a self-normalised bound."""
    import sr_states

    exponents = torch.tensor(list(BINADES[dtype]), dtype=torch.float64)
    base = torch.pow(2.0, exponents)
    inputs = (base[:, None] * (1.0 + torch.linspace(0.01, 0.99, 1024, dtype=torch.float64)[None, :])).flatten()
    inputs = inputs.float()
    rounded = sr_states.cast(inputs.to(cuda), dtype=dtype, seed=91).float().double().cpu()
    normalized_error = (rounded - inputs.double()) / inputs.double().abs()
    mean, std = normalized_error.mean().item(), normalized_error.std().item()
    assert std > 0
    assert abs(mean) < 6 * std / math.sqrt(normalized_error.numel())
    if dtype == torch.bfloat16:
        assert abs(mean) < 1e-4  # the reference's own bound


def _neighbours(stored: torch.Tensor, exact: float):
    """The two stored values, checked to be adjacent encodings around `exact`."""
    values = torch.unique(stored.float().cpu())
    assert values.numel() == 2, values
    lo, hi = values.tolist()
    assert lo < exact < hi
    words = raw_bits(torch.tensor([lo, hi]).to(stored.dtype)).to(torch.int64)
    assert int(words[1] - words[0]) == 1, "stored values are not adjacent encodings"
    return lo, hi


def _assert_unbiased(stored: torch.Tensor, exact: float):
    lo, hi = _neighbours(stored, exact)
    p_up = (exact - lo) / (hi - lo)
    standard_error = math.sqrt(p_up * (1 - p_up) / stored.numel())
    empirical = (stored.float() == hi).double().mean().item()
    assert abs(empirical - p_up) < 6 * standard_error
    assert abs(stored.float().double().mean().item() - exact) < 6 * standard_error * (hi - lo)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float8_e4m3fn, torch.float8_e5m2])
def test_adamw_moments_are_unbiased(cuda, dtype):
    """One step from zero moments: m' = (1-b1) g and v' = (1-b2) g g in FP32, stored by SR.

    The stored moments take the two neighbours of those FP32 values with the
    frequencies that make their mean the FP32 value.
    """
    import sr_states

    g_value = 0.37
    p = torch.nn.Parameter(torch.zeros(N, device=cuda))
    p.grad = torch.full((N,), g_value, device=cuda)
    opt = sr_states.AdamWHip([p], lr=1e-3, weight_decay=0.0, state_dtype=dtype, seed=5)
    opt.step()
    g32 = torch.tensor(g_value, dtype=torch.float32)
    m32 = (g32 * torch.tensor(1 - 0.9, dtype=torch.float32)).item()
    v32 = ((torch.tensor(1 - 0.999, dtype=torch.float32) * g32) * g32).item()
    _assert_unbiased(opt.state[p]["exp_avg"].cpu(), m32)
    _assert_unbiased(opt.state[p]["exp_avg_sq"].cpu(), v32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float8_e4m3fn, torch.float8_e5m2])
def test_sgdm_momentum_is_unbiased(cuda, dtype):
    """One step from a zero momentum stores u' = g by SR: unbiased around the FP32 gradient."""
    import sr_states

    g_value = 0.3
    p = torch.nn.Parameter(torch.zeros(N, device=cuda))
    p.grad = torch.full((N,), g_value, device=cuda)
    opt = sr_states.SGDMHip([p], lr=1e-3, momentum=0.9, state_dtype=dtype, seed=6)
    opt.step()
    _assert_unbiased(opt.state[p]["momentum_buffer"].cpu(), torch.tensor(g_value, dtype=torch.float32).item())
