"""The device minifloat encoders and decoders equal the integer forms on every input.

The kernels encode FP16, E4M3 and E5M2 states with sr::minifloat_bits_fast
(bit arithmetic on the FP32 pattern finished by a hardware convert of an
exactly representable value) and decode them with one hardware convert
(sr::minifloat_decode).  The reference rule (sr_states/_minifloat.py:
17-70) is restated as sr::minifloat_bits, which the CPU suite pins against
the oracles.  tests/native/minifloat_check.hip compares the two on the device
bit for bit over every FP32 input, nearest rounding once and stochastic
rounding at the random values where the input's decision flips and at the
extremes (both round up exactly when the random value's upper 24 bits are
below a threshold of the input); and every encoding through both decoders
(equal bits, or NaN for NaN).
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

LIBRARY = Path(__file__).resolve().parent / "native" / "libminifloat_check.so"


@pytest.mark.parametrize("name,code,width", [("float16", 0, 16), ("float8_e4m3fn", 1, 8), ("float8_e5m2", 2, 8)])
def test_device_minifloat_codecs_match_the_integer_forms_exhaustively(cuda, name, code, width):
    import torch  # noqa: F401  (load the HIP runtime first)

    assert LIBRARY.exists(), f"{LIBRARY} is not built (tests/native/build_checks.py)"
    check = ctypes.CDLL(str(LIBRARY))
    check.sr_check_minifloat.restype = ctypes.c_int
    check.sr_check_minifloat.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_ulonglong)]
    counters = (ctypes.c_ulonglong * 2)()
    assert check.sr_check_minifloat(code, counters) == 0
    mismatches, comparisons = counters[0], counters[1]
    assert comparisons == 7 * 2**32 + 2**width
    assert mismatches == 0, f"{name}: {mismatches} of {comparisons} comparisons differ"


@pytest.mark.parametrize("name,code,width", [("float16", 0, 16), ("float8_e4m3fn", 1, 8), ("float8_e5m2", 2, 8)])
def test_device_group_codecs_match_the_integer_forms_in_every_position(cuda, name, code, width):
    """The four-element forms of the kernels' vector paths (two elements per paired convert).

    Every FP32 input at each position of a group, beside finite companions and
    beside a NaN companion, nearest and stochastic at its six random values;
    every encoding at each position through the group decoder.
    """
    import torch  # noqa: F401  (load the HIP runtime first)

    assert LIBRARY.exists(), f"{LIBRARY} is not built (tests/native/build_checks.py)"
    check = ctypes.CDLL(str(LIBRARY))
    check.sr_check_minifloat_groups.restype = ctypes.c_int
    check.sr_check_minifloat_groups.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_ulonglong)]
    counters = (ctypes.c_ulonglong * 2)()
    assert check.sr_check_minifloat_groups(code, counters) == 0
    mismatches, comparisons = counters[0], counters[1]
    assert comparisons == 144 * 2**32 + 16 * 2**width
    assert mismatches == 0, f"{name}: {mismatches} of {comparisons} comparisons differ"
