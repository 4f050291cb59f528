"""The kernels' workgroup-to-tile order is a permutation of every launch (CPU).

tests/native/tile_order.cpp compiles csrc/sr_tile_order.h for the host and
walks every workgroup of launches of 1..5000 tiles and of the configs' tile
counts: each tile is covered exactly once, padding workgroups map past the
last tile, and each XCD walks whole chunks of consecutive tiles.  It also
checks the resident-workgroup cap of large optimizer launches (resident_cap).
"""

from __future__ import annotations

import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_tile_order_is_a_permutation(tmp_path):
    binary = tmp_path / "tile_order"
    subprocess.run(["g++", "-O2", "-std=c++17", "-I", str(ROOT / "stochastic-rounding-pytorch_amd" / "csrc"),
                    str(ROOT / "tests" / "native" / "tile_order.cpp"), "-o", str(binary)], check=True)
    result = subprocess.run([str(binary)], capture_output=True, text=True, timeout=120)
    assert result.returncode == 0, result.stdout + result.stderr
    assert result.stdout.strip().endswith(", 0 failures"), result.stdout
