"""Compile the device-side checks under tests/native for gfx950.

``build()`` writes, with the library's own HIP flags:

- tests/native/libbf16_sr_check.so, the exhaustive BF16 stochastic-rounding
  check of bf16_sr_check.hip;
- tests/native/libminifloat_check.so, the exhaustive check of the device
  minifloat encoders of minifloat_check.hip;
- tests/native/libdivsqrt_check.so, the exhaustive check of the AdamW
  update's square root and constant-divisor division of divsqrt_check.hip;
- tests/native/abi_c_host, a plain C program that drives the C ABI and
  checks it against the C oracle (when the package library is built);
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


# A plain C host of the C ABI (abi_c_host.c), linked against the product
# library and the C oracle as its checker; needs the package built first.
C_HOST = HERE / "abi_c_host"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))


def _run(cmd):
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"command failed ({result.returncode}): {' '.join(cmd)}\n{result.stderr}")


def build_c_host() -> Path:
    package_lib = ROOT / "stochastic-rounding-pytorch_amd" / "sr_states"
    tmp = C_HOST.with_name(C_HOST.name + ".tmp")
    _run(["gcc", "-O2", "-std=gnu11", "-ffp-contract=off", "-fno-fast-math", "-Wall", "-I", str(ROCM / "include"),
          str(HERE / "abi_c_host.c"), str(ROOT / "oracle" / "sr_oracle.c"), "-o", str(tmp),
          "-L", str(package_lib), "-lsr_states_hip", "-Wl,-rpath,$ORIGIN/../../stochastic-rounding-pytorch_amd/sr_states",
          "-L", str(ROCM / "lib"), "-lamdhip64", f"-Wl,-rpath,{ROCM / 'lib'}", "-lm"])
    os.replace(tmp, C_HOST)
    return C_HOST


def build() -> list[Path]:
    package = _package_build()
    for library, source in LIBRARIES.items():
        tmp = library.with_name(library.name + ".tmp")
        _run([package.HIPCC, *package.HIP_FLAGS, "-shared", str(source), "-o", str(tmp)])
        os.replace(tmp, library)
    built = list(LIBRARIES)
    if (ROOT / "stochastic-rounding-pytorch_amd" / "sr_states" / "libsr_states_hip.so").exists():
        built.append(build_c_host())
    return built


if __name__ == "__main__":
    print(build())
