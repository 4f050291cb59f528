"""Compile the device-side checks under tests/native for gfx950.

``build()`` writes tests/native/libbf16_sr_check.so (the exhaustive BF16
stochastic-rounding check of bf16_sr_check.hip) with the library's own HIP
flags.  __graft_entry__.build() calls it; tests/conftest.py calls it on a
CPU checkout where it is missing.  GPU runs use the prebuilt file.
"""

from __future__ import annotations

import importlib.util
import os
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
CHECK_LIBRARY = HERE / "libbf16_sr_check.so"


def _package_build():
    spec = importlib.util.spec_from_file_location(
        "sr_states_build", ROOT / "stochastic-rounding-pytorch_amd" / "build.py"
    )
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


def build() -> Path:
    package = _package_build()
    tmp = CHECK_LIBRARY.with_name(CHECK_LIBRARY.name + ".tmp")
    cmd = [package.HIPCC, *package.HIP_FLAGS, "-shared", str(HERE / "bf16_sr_check.hip"), "-o", str(tmp)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"command failed ({result.returncode}): {' '.join(cmd)}\n{result.stderr}")
    os.replace(tmp, CHECK_LIBRARY)
    return CHECK_LIBRARY


if __name__ == "__main__":
    print(build())
