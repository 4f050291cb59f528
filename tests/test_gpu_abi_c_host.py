"""The C ABI driven from plain C: no Python, no torch in the process.

tests/native/abi_c_host.c allocates device memory with the HIP runtime,
calls sr_cast, sr_adamw_step, sr_sgdm_step and sr_adamw_multi (with the row
table and tile map it builds) as a C, Go (cgo) or Rust host would, and compares every output byte with the C oracle linked into it;
it checks sr_neighbors' BF16 pairs against their definition, and that a bad argument comes back as
SR_ERR_ARGUMENT with a message.
"""

from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

BINARY = Path(__file__).resolve().parent / "native" / "abi_c_host"


def test_plain_c_host_matches_the_c_oracle(cuda):
    assert BINARY.exists(), f"{BINARY} is not built (tests/native/build_checks.py)"
    result = subprocess.run([str(BINARY)], capture_output=True, text=True, timeout=120)
    assert result.returncode == 0, result.stdout + result.stderr
    lines = result.stdout.splitlines()
    assert lines[-1] == "abi_c_host ok"
    assert sum(line.startswith("ok ") for line in lines) == 13, result.stdout
