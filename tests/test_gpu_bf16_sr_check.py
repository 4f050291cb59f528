"""The device BF16 stochastic-rounding encoder equals the reference rule on every input.

The kernels round BF16 states with gfx950's v_cvt_sr_bf16_f32; the reference
rule (sr_states/_bf16.py:37-74) is restated as sr::bf16_sr_bits, which the
CPU suite pins against the oracles.  tests/native/bf16_sr_check.hip compares
the two on the device bit for bit, NaN payloads included: every FP32 input
at its decision boundaries, 0, 0xFFFF and a hashed random value, and every
(low half, random value) pair for twelve upper halves.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

LIBRARY = Path(__file__).resolve().parent / "native" / "libbf16_sr_check.so"


def test_hardware_sr_convert_matches_the_reference_rule_exhaustively(cuda):
    import torch  # noqa: F401  (load the HIP runtime first)

    assert LIBRARY.exists(), f"{LIBRARY} is not built (tests/native/build_checks.py)"
    check = ctypes.CDLL(str(LIBRARY))
    check.sr_check_bf16_sr.restype = ctypes.c_int
    check.sr_check_bf16_sr.argtypes = [ctypes.POINTER(ctypes.c_ulonglong)]
    counters = (ctypes.c_ulonglong * 2)()
    assert check.sr_check_bf16_sr(counters) == 0
    mismatches, comparisons = counters[0], counters[1]
    assert comparisons == 5 * 2**32 + 12 * 2**32
    assert mismatches == 0


def test_hardware_nearest_convert_matches_the_reference_rule_on_every_input(cuda):
    """sr::bf16_rn (v_cvt_pk_bf16_f32, NaN as 0x7FC0) against the integer nearest-even form."""
    import torch  # noqa: F401  (load the HIP runtime first)

    assert LIBRARY.exists(), f"{LIBRARY} is not built (tests/native/build_checks.py)"
    check = ctypes.CDLL(str(LIBRARY))
    check.sr_check_bf16_rn.restype = ctypes.c_int
    check.sr_check_bf16_rn.argtypes = [ctypes.POINTER(ctypes.c_ulonglong)]
    counters = (ctypes.c_ulonglong * 2)()
    assert check.sr_check_bf16_rn(counters) == 0
    assert counters[1] == 2**32
    assert counters[0] == 0, f"{counters[0]} of 2^32 inputs differ"


def test_group_converts_match_the_reference_rules_in_every_position(cuda):
    """The four-element BF16 forms of the kernels' vector paths (two elements per convert).

    Every FP32 input at each position of a group, stochastic at its five random
    values and nearest (in the optimizers' form and in the casts' form, which
    takes loaded values without the barrier against FMA fusion); the twelve
    upper halves' (low half, random) pairs at each position.
    """
    import torch  # noqa: F401  (load the HIP runtime first)

    assert LIBRARY.exists(), f"{LIBRARY} is not built (tests/native/build_checks.py)"
    check = ctypes.CDLL(str(LIBRARY))
    check.sr_check_bf16_groups.restype = ctypes.c_int
    check.sr_check_bf16_groups.argtypes = [ctypes.POINTER(ctypes.c_ulonglong)]
    counters = (ctypes.c_ulonglong * 2)()
    assert check.sr_check_bf16_groups(counters) == 0
    mismatches, comparisons = counters[0], counters[1]
    assert comparisons == 112 * 2**32 + 12 * 2**31 * 32
    assert mismatches == 0, f"{mismatches} of {comparisons} comparisons differ"
