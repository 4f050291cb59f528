"""The AdamW update's square root and division are IEEE correctly rounded on every input.

The reference divides by sqrt(1 - beta2^t) and by the denominator, and takes
the square root of the second moment, each correctly rounded in FP32
(sr_states/reference/adamw.py:86-96).  The kernels compute the square root
from the hardware reciprocal square root with one Newton step on the exact
residual (sr::sqrt_rn), the division by sqrt(1 - beta2^t), a constant of the
launch, as a multiply by its correctly rounded reciprocal plus one remainder
correction (sr::div_by_constant), and the division by the denominator the
same way from a reciprocal made exact by one Newton step, where its first
quotient is in range (sr::div_short; the library division elsewhere).
tests/native/divsqrt_check.hip compares them with the correctly rounded
operations on the device:

- the square root on every FP32 input;
- each division on every pair of significands (2^46 pairs), which stands
  for every dividend and divisor of the function's domain, because scaling
  by powers of two scales every intermediate exactly there;
- for div_by_constant, zero, infinite and NaN dividends and both ends of
  the exponent ranges; for div_short, the reciprocal on every float of
  [2^-126, 2^126), hashed cases across its whole domain, and special
  dividends and divisors, which it must refuse.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

LIBRARY = Path(__file__).resolve().parent / "native" / "libdivsqrt_check.so"
COUNTERS = ctypes.c_ulonglong * 2


def _library():
    import torch  # noqa: F401  (load the HIP runtime first)

    assert LIBRARY.exists(), f"{LIBRARY} is not built (tests/native/build_checks.py)"
    lib = ctypes.CDLL(str(LIBRARY))
    for name in ("sr_check_sqrt", "sr_check_div_edges"):
        getattr(lib, name).restype = ctypes.c_int
        getattr(lib, name).argtypes = [ctypes.POINTER(ctypes.c_ulonglong)]
    for name in ("sr_check_div_by_constant", "sr_check_div_short"):
        getattr(lib, name).restype = ctypes.c_int
        getattr(lib, name).argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.POINTER(ctypes.c_ulonglong)]
    for name in ("sr_check_rcp_rn", "sr_check_div_short_domain"):
        getattr(lib, name).restype = ctypes.c_int
        getattr(lib, name).argtypes = [ctypes.POINTER(ctypes.c_ulonglong)]
    return lib


def test_square_root_is_correctly_rounded_on_every_input(cuda):
    counters = COUNTERS()
    assert _library().sr_check_sqrt(counters) == 0
    assert counters[1] == 2**32
    assert counters[0] == 0, f"{counters[0]} of 2^32 square roots differ from sqrtf"


def test_division_by_the_bias_correction_edges(cuda):
    counters = COUNTERS()
    assert _library().sr_check_div_edges(counters) == 0
    assert counters[1] == 2**14 * 2 * (2**9 * 4 + 2 * 2**23)
    assert counters[0] == 0, f"{counters[0]} of {counters[1]} quotients differ from x / c"


def test_division_by_the_bias_correction_on_every_significand_pair(cuda):
    lib, chunk = _library(), 1 << 15
    mismatches = comparisons = 0
    for first in range(0, 1 << 23, chunk):
        counters = COUNTERS()
        assert lib.sr_check_div_by_constant(first, chunk, counters) == 0, first
        mismatches += counters[0]
        comparisons += counters[1]
        assert mismatches == 0, f"divisor significands from {first:#x}: {mismatches} quotients differ"
    assert comparisons == 2**46


def test_short_division_reciprocal_is_correctly_rounded_on_every_normal_divisor(cuda):
    counters = COUNTERS()
    assert _library().sr_check_rcp_rn(counters) == 0
    assert counters[1] == 0x7E000000
    assert counters[0] == 0, f"{counters[0]} reciprocals differ from 1 / b"


def test_short_division_on_every_significand_pair(cuda):
    lib, chunk = _library(), 1 << 15
    mismatches = comparisons = 0
    for first in range(0, 1 << 23, chunk):
        counters = COUNTERS()
        assert lib.sr_check_div_short(first, chunk, counters) == 0, first
        mismatches += counters[0]
        comparisons += counters[1]
        assert mismatches == 0, f"divisor significands from {first:#x}: {mismatches} quotients differ or refused"
    assert comparisons == 2**46


def test_short_division_across_its_domain_and_refusals(cuda):
    counters = (ctypes.c_ulonglong * 3)()
    assert _library().sr_check_div_short_domain(counters) == 0
    assert counters[1] == 2**16 * 512 * 3
    assert counters[0] == 0, f"{counters[0]} wrong quotients accepted or special cases not refused"
    # A good share of the random cases (half of them with dividends of every
    # exponent, so quotients far outside the range) is accepted.
    assert counters[2] > 2**16 * 512 // 4
