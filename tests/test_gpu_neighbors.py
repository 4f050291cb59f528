"""The HIP neighbour kernel behind ``bf16_neighbors``/``minifloat_neighbors``.

For each FP32 input the two storage values that stochastic rounding chooses
between (sr_states/_bf16.py:77-101, sr_states/_minifloat.py:73-99).  Checked

- over every FP32 bit pattern, against the definition itself: lower <= x <=
  upper (x clamped to the maximum for E4M3/E5M2), both with x's sign,
  adjacent encodings, and equal exactly when x is representable; NaN gives
  NaN.  Those properties leave one possible pair per input;
- against the torch oracle and the enumerated-grid neighbours on the
  reference's boundary sets and random words, bit for bit;
- as the reference's tests use them (tests/test_sr_edge_cases.py:9-54,
  tests/test_minifloat.py:94-100): the HIP casts' stochastic outputs are
  always one of the two.
"""

from __future__ import annotations

import pytest
import torch
from _cases import bf16_bracket, boundary_inputs, oracle_neighbors, random_words
from conftest import assert_bits_or_nan

from oracle import sr_oracle
from sr_states import cast
from sr_states.reference import bf16_neighbors, minifloat_neighbors, stochastic_round_bf16

pytestmark = pytest.mark.gpu

FORMATS = (torch.bfloat16, torch.float16, torch.float8_e4m3fn, torch.float8_e5m2)
MINIFLOATS = FORMATS[1:]
IDS = ["bf16", "fp16", "e4m3", "e5m2"]


def _neighbors(x, dtype):
    return bf16_neighbors(x) if dtype == torch.bfloat16 else minifloat_neighbors(x, dtype=dtype)


def _oracle(x, dtype):
    if dtype == torch.bfloat16:
        return sr_oracle.bf16_neighbors(x)
    return sr_oracle.minifloat_neighbors(x, dtype=dtype)


def _magnitude_code(t):
    if t.element_size() == 2:
        return t.view(torch.int16).to(torch.int32) & 0x7FFF
    return t.view(torch.uint8).to(torch.int32) & 0x7F


@pytest.mark.parametrize("dtype", FORMATS, ids=IDS)
def test_every_fp32_input_gets_its_bracketing_pair(cuda, dtype):
    """All 2^32 inputs, in chunks of 2^27, against the definition of the pair."""
    saturate = dtype in (torch.float8_e4m3fn, torch.float8_e5m2)
    maximum = torch.finfo(dtype).max
    chunk = 1 << 27
    failures = 0
    for start in range(-(1 << 31), 1 << 31, chunk):
        x = torch.arange(start, start + chunk, dtype=torch.int64, device=cuda).to(torch.int32).view(torch.float32)
        lower, upper = _neighbors(x, dtype)
        lo, hi = lower.float(), upper.float()
        nan = torch.isnan(x)
        clamped = x.clamp(-maximum, maximum) if saturate else x
        step = _magnitude_code(lower) - _magnitude_code(upper)
        step = torch.where(torch.signbit(x), step, -step)
        sign = torch.signbit(x)
        good = torch.where(
            nan,
            torch.isnan(lo) & torch.isnan(hi),
            (lo <= clamped) & (clamped <= hi)
            & (torch.signbit(lo) == sign) & (torch.signbit(hi) == sign)
            & ((step == 0) | (step == 1))
            & ((step == 0) == (lo == clamped)),
        )
        failures += int((~good).sum())
        del x, lower, upper, lo, hi, nan, clamped, step, sign, good
    assert failures == 0


@pytest.mark.parametrize("dtype", FORMATS, ids=IDS)
def test_neighbors_equal_the_oracle_and_the_enumeration(cuda, dtype):
    words = random_words(1 << 18, 17)
    x = torch.cat((boundary_inputs(dtype), words, torch.tensor([0.0, -0.0, 2.0**-149, -(2.0**-149)])))
    lower, upper = _neighbors(x.to(cuda), dtype)
    want_lower, want_upper = _oracle(x, dtype)
    assert_bits_or_nan(lower.cpu(), want_lower, "lower")
    assert_bits_or_nan(upper.cpu(), want_upper, "upper")
    finite = torch.isfinite(x)
    if dtype == torch.bfloat16:
        lo, hi = bf16_bracket(x[finite])
    else:
        lo, hi = oracle_neighbors(x, dtype)
        lo, hi = lo[finite], hi[finite]
    assert torch.equal(lower.cpu()[finite].float(), lo)
    assert torch.equal(upper.cpu()[finite].float(), hi)


def test_output_is_one_of_the_two_bf16_neighbors(cuda):
    """tests/test_sr_edge_cases.py:9-14."""
    generator = torch.Generator().manual_seed(123)
    x = (torch.randn(20_000, generator=generator, dtype=torch.float32) * 100).to(cuda)
    output = stochastic_round_bf16(x, seed=7)
    lower, upper = bf16_neighbors(x)
    assert torch.all((output == lower) | (output == upper))


def test_fp32_subnormals_and_bf16_midpoint_boundaries(cuda):
    """tests/test_sr_edge_cases.py:32-54."""
    tiny = torch.nextafter(torch.tensor(0.0), torch.tensor(1.0)).reshape(1).to(cuda)
    output = stochastic_round_bf16(tiny, seed=3)
    lower, upper = bf16_neighbors(tiny)
    assert torch.all((output == lower) | (output == upper))
    words = torch.tensor([0x00000001, 0x00008000, 0x0000FFFF, 0x00010000, 0x3F807FFF, 0x3F808000, 0x3F808001],
                         dtype=torch.int32, device=cuda)
    values = words.view(torch.float32)
    output = stochastic_round_bf16(values, seed=867)
    lower, upper = bf16_neighbors(values)
    assert torch.all((output == lower) | (output == upper))


@pytest.mark.parametrize("dtype", MINIFLOATS, ids=IDS[1:])
def test_stochastic_casts_land_on_a_neighbor(cuda, dtype):
    """tests/test_minifloat.py:103-114 with the HIP cast and the HIP neighbours."""
    x = torch.cat((boundary_inputs(dtype), random_words(10_003, 71))).to(cuda)
    lower, upper = minifloat_neighbors(x, dtype=dtype)
    for seed in (2**32 + 9, 5):
        result = cast(x, dtype=dtype, seed=seed).float()
        finite = ~torch.isnan(x)
        hit = (result == lower.float()) | (result == upper.float())
        assert torch.all(hit[finite])
        assert torch.equal(torch.isnan(result), torch.isnan(x))


def test_shapes_layouts_and_errors(cuda):
    x = torch.randn(37, 53, generator=torch.Generator().manual_seed(3)).to(cuda)
    view = x.t()
    lower, upper = bf16_neighbors(view)
    assert lower.shape == view.shape and lower.dtype == torch.bfloat16
    want_lower, want_upper = sr_oracle.bf16_neighbors(view.cpu().contiguous())
    assert torch.equal(lower.cpu(), want_lower) and torch.equal(upper.cpu(), want_upper)
    lower, upper = minifloat_neighbors(torch.empty(0, 3, device=cuda), dtype=torch.float8_e4m3fn)
    assert lower.shape == (0, 3) and upper.dtype == torch.float8_e4m3fn
    with pytest.raises(TypeError, match="float32"):
        bf16_neighbors(x.double())
    with pytest.raises(TypeError, match="float32"):
        minifloat_neighbors(x.half(), dtype=torch.float8_e4m3fn)
    with pytest.raises(ValueError, match="E4M3, E5M2, and FP16"):
        minifloat_neighbors(x, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU"):
        bf16_neighbors(x.cpu())
