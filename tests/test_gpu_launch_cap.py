"""The resident-workgroup cap of large optimizer launches pays for itself.

Large FP32-parameter launches reserve LDS they never use so that only
sr::resident_cap workgroups stay resident per CU: about 80 KiB of tiles in
flight per CU, where 16 workgroups fit.  tests/native/stream_ceiling.hip's
sr_launch_cap_sweep times the library's fused AdamW kernel (FP32 parameter
and gradient, BF16 stochastic moments) on one tensor of 2^28 elements
(5.4 GB) with the rule's cap and with none, interleaved over three rounds:
the occupancy calculator must report the rule's 8 workgroups per CU, and
the capped kernel must be at least as fast as the uncapped one (on MI355X
it is 3-4% faster at this footprint).
"""

from __future__ import annotations

import ctypes
import statistics
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

LIBRARY = Path(__file__).resolve().parent / "native" / "libstream_ceiling.so"
N = 1 << 28


def test_capped_fused_kernel_is_at_least_as_fast_as_uncapped(cuda):
    assert LIBRARY.exists(), f"{LIBRARY} is not built (tests/native/build_checks.py)"
    lib = ctypes.CDLL(str(LIBRARY))
    lib.sr_launch_cap_sweep.restype = ctypes.c_int
    lib.sr_launch_cap_sweep.argtypes = [ctypes.c_uint64, ctypes.c_int, ctypes.POINTER(ctypes.c_int), ctypes.c_int,
                                        ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_float),
                                        ctypes.POINTER(ctypes.c_int)]
    caps = (ctypes.c_int * 2)(-1, 0)
    capped, uncapped = [], []
    for _ in range(3):
        trivial, fused, resident = (ctypes.c_float * 2)(), (ctypes.c_float * 2)(), (ctypes.c_int * 2)()
        assert lib.sr_launch_cap_sweep(N, 40, caps, 2, trivial, fused, resident) == 0
        assert resident[0] == 8 and resident[1] == 16, list(resident)
        capped.append(fused[0])
        uncapped.append(fused[1])
    rate = lambda ms: 20 * N / ms / 1e6  # noqa: E731  (GB/s)
    capped_ms, uncapped_ms = statistics.median(capped), statistics.median(uncapped)
    assert capped_ms <= uncapped_ms, (
        f"capped {rate(capped_ms):.0f} GB/s against uncapped {rate(uncapped_ms):.0f} GB/s")
