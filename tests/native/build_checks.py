"""Compile the device-side checks under tests/native for gfx950.

``build()`` writes, with the library's own HIP flags:

- tests/native/libbf16_sr_check.so, the exhaustive BF16 stochastic-rounding
  check of bf16_sr_check.hip;
- tests/native/libminifloat_check.so, the exhaustive check of the device
  minifloat encoders of minifloat_check.hip;
- tests/native/libdivsqrt_check.so, the exhaustive check of the AdamW
  update's square root and constant-divisor division of divsqrt_check.hip;
- tests/native/libstream_ceiling.so, the trivial-math kernel of
  stream_ceiling.hip that measures the bandwidth ceiling of the fused
  update's access pattern (bench.py and tests/test_gpu_stream_ceiling.py).

__graft_entry__.build() calls it; tests/conftest.py calls it on a CPU
checkout where a library is missing.  GPU runs use the prebuilt files.
"""

from __future__ import annotations

import importlib.util
import os
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
CHECK_LIBRARY = HERE / "libbf16_sr_check.so"
CEILING_LIBRARY = HERE / "libstream_ceiling.so"
MINIFLOAT_LIBRARY = HERE / "libminifloat_check.so"
DIVSQRT_LIBRARY = HERE / "libdivsqrt_check.so"
LIBRARIES = {CHECK_LIBRARY: HERE / "bf16_sr_check.hip", CEILING_LIBRARY: HERE / "stream_ceiling.hip",
             MINIFLOAT_LIBRARY: HERE / "minifloat_check.hip", DIVSQRT_LIBRARY: HERE / "divsqrt_check.hip"}


def _package_build():
    spec = importlib.util.spec_from_file_location(
        "sr_states_build", ROOT / "stochastic-rounding-pytorch_amd" / "build.py"
    )
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


def build() -> list[Path]:
    package = _package_build()
    for library, source in LIBRARIES.items():
        tmp = library.with_name(library.name + ".tmp")
        cmd = [package.HIPCC, *package.HIP_FLAGS, "-shared", str(source), "-o", str(tmp)]
        result = subprocess.run(cmd, capture_output=True, text=True)
        if result.returncode != 0:
            raise RuntimeError(f"command failed ({result.returncode}): {' '.join(cmd)}\n{result.stderr}")
        os.replace(tmp, library)
    return list(LIBRARIES)


if __name__ == "__main__":
    print(build())
