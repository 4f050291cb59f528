"""bench.py's contract on the CPU: workloads, byte accounting and the one-GPU rule.

The timed run needs a GPU (the round-end driver runs it); here the
workload table, the algorithmic bytes per element (the reference's traffic
model, benchmarks/bench_states.py:65-70, extended to mixed widths) and the
refusal of more than one GPU are checked without one.
"""

from __future__ import annotations

import math
import subprocess
import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
import bench  # noqa: E402


@pytest.mark.parametrize(
    "name,expected",
    [("north_star", 20), ("c1_cast_bf16", 6), ("c2_single_2e26", 20), ("c3_gpt2", 18), ("c4_fp8_mixed", 18),
     ("c5_sgdm_fp16", 16), ("bf16_params_bf16sr", 14), ("bf16_params_e4m3_bf16sr", 12),
     ("bf16_params_fp16sr", 14), ("cast_2e26_e4m3", 5), ("cast_2e26_fp16", 6)],
)
def test_bytes_per_element_follow_the_traffic_model(name, expected):
    assert bench.bytes_per_element(bench.WORKLOADS[name]) == expected


def test_north_star_is_the_default_and_has_the_stated_size():
    spec = bench.WORKLOADS["north_star"]
    assert sum(math.prod(s) for s in spec["shapes"]) == 1_547_698_176
    assert len(spec["shapes"]) == 50
    assert spec["p_dtype"] == spec["g_dtype"] == torch.float32
    assert spec.get("warmup", 25) == 25 and spec.get("steps", 100) == 100


def test_short_launches_warm_up_for_the_clock_ramp():
    """Each cast or sub-millisecond workload's default warmup spans at least ~0.3 s of GPU work."""
    rough_ms = {"c1_cast_bf16": 0.0165, "c2_single_2e26": 0.208, "c3_gpt2": 0.353, "cast_2e26_bf16": 0.061}
    for name, ms in rough_ms.items():
        assert bench.WORKLOADS[name]["warmup"] * ms >= 300, name


def test_more_than_one_gpu_is_refused_with_a_reason():
    result = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True,
                            text=True, timeout=300)
    assert result.returncode != 0
    assert "one GPU" in result.stderr or "one GPU" in result.stdout


@pytest.mark.parametrize("value", ["float8_e4m3fn/sideways", "float9/stochastic", "bfloat16"])
def test_state_format_override_is_validated_before_anything_runs(value):
    result = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--state-format", value],
                            capture_output=True, text=True, timeout=300)
    assert result.returncode != 0 and "--state-format" in result.stderr


def test_ceiling_helpers_refuse_bad_arguments_before_any_device_work():
    """The placement sweep and the pattern ceiling check their arguments first (no GPU here)."""
    import ctypes

    lib = ctypes.CDLL(str(bench.CEILING_LIBRARY))
    lib.sr_stream_placements.restype = ctypes.c_int
    lib.sr_stream_placements.argtypes = [ctypes.c_uint64, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_int, ctypes.POINTER(ctypes.c_uint64), ctypes.c_int,
                                         ctypes.POINTER(ctypes.c_float)]
    lib.sr_stream_ceiling_p.restype = ctypes.c_int
    lib.sr_stream_ceiling_p.argtypes = [ctypes.c_uint64, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                        ctypes.c_int, ctypes.POINTER(ctypes.c_float)]
    ms = (ctypes.c_float * 4)()

    def placements(n, widths, gaps, reps=1):
        array = (ctypes.c_uint64 * max(len(gaps), 1))(*gaps)
        return lib.sr_stream_placements(n, *widths, reps, array, len(gaps), ms)

    n = 512 * 1000
    assert placements(n, (4, 4, 2, 2), [100]) == 1  # not a multiple of 256
    assert placements(n, (4, 4, 2, 2), [(16 << 20) + 256]) == 1  # above 16 MiB
    assert placements(n, (4, 4, 2, 2), []) == 1
    assert placements(n + 1, (4, 4, 2, 2), [0]) == 1  # not whole tiles
    assert placements(n, (4, 4, 3, 2), [0]) == 1  # no such pattern
    assert placements(n, (4, 4, 2, 2), [0], reps=0) == 1
    assert lib.sr_stream_ceiling_p(n, 2, 4, 2, 2, 1, ms) == 1
    assert lib.sr_stream_ceiling_p(0, 4, 4, 2, 2, 1, ms) == 1
    assert bench.PLACEMENT_GAPS[0] == 0 and all(g % 256 == 0 and g <= 16 << 20 for g in bench.PLACEMENT_GAPS)
