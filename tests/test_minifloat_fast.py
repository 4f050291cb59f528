"""The device minifloat encoder's bit arithmetic equals the integer form (CPU).

tests/native/minifloat_fast.cpp compiles csrc/sr_math.h for the host, where
sr::minifloat_bits_fast finishes with the integer nearest form instead of a
hardware convert, and compares it with sr::minifloat_bits on every 257th
FP32 input: nearest once, stochastic at the random values where the input's
decision flips and at the extremes.  It also checks sr::fp8_sr_grid_bits,
the kernels' single-form FP8 stochastic rounding, the same way.  The exhaustive comparison including the
hardware converts runs on the device (tests/test_gpu_minifloat_check.py).
"""

from __future__ import annotations

import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_minifloat_fast_bit_arithmetic_matches_the_integer_form(tmp_path):
    binary = tmp_path / "minifloat_fast"
    subprocess.run(["g++", "-O2", "-std=c++17", "-I", str(ROOT / "stochastic-rounding-pytorch_amd" / "csrc"),
                    str(ROOT / "tests" / "native" / "minifloat_fast.cpp"), "-o", str(binary)], check=True)
    result = subprocess.run([str(binary)], capture_output=True, text=True, timeout=300)
    assert result.returncode == 0, result.stdout + result.stderr
    lines = result.stdout.strip().splitlines()
    assert len(lines) == 5 and all(" 0 mismatches of " in line for line in lines), result.stdout
    assert all(" 0 mismatches of 116" in line for line in lines[:3]), result.stdout
