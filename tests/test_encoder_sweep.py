"""The product's encoders against the C oracle over FP32 bit patterns (CPU).

tests/native/encoder_sweep.cpp compiles the kernels' element header
(csrc/sr_math.h) for the host and compares every encoder with the C
oracle's independent float-grid formulation.  The suite uses a stride of
1021 (4.2 M inputs per encoder); ``encoder_sweep 1`` covers all 2^32 inputs
(done for this build: no mismatch).
"""

from __future__ import annotations

import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_product_encoders_match_the_c_oracle(tmp_path):
    objects = tmp_path / "sr_oracle.o"
    subprocess.run(["gcc", "-O2", "-std=c11", "-ffp-contract=off", "-c", str(ROOT / "oracle" / "sr_oracle.c"),
                    "-o", str(objects)], check=True)
    binary = tmp_path / "encoder_sweep"
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off",
                    "-I", str(ROOT / "stochastic-rounding-pytorch_amd" / "csrc"),
                    str(ROOT / "tests" / "native" / "encoder_sweep.cpp"), str(objects), "-o", str(binary),
                    "-lpthread", "-lm"], check=True)
    result = subprocess.run([str(binary), "1021"], capture_output=True, text=True, timeout=300)
    assert result.returncode == 0, result.stdout + result.stderr
    assert result.stdout.count(" 0 mismatches") == 12, result.stdout
