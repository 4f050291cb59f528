"""Compile the gfx950 kernels and the C ABI into sr_states/libsr_states_hip.so.

Run ``python build.py`` from anywhere.  The AdamW instantiations are split
into nine translation units (one per first-moment encoding) that compile in
parallel; the shared library is linked in place next to the Python package,
so it travels with the source tree.  Two CPython extensions over torch's
tensor type are built alongside it: the host-side group walk
(csrc/group_walk.cpp -> sr_states/_group_walk<EXT_SUFFIX>) and the native
entries of the single-tensor launches (csrc/launch.cpp ->
sr_states/_launch<EXT_SUFFIX>).
"""

from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

ROOT = Path(__file__).resolve().parent
CSRC = ROOT / "csrc"
BUILD = ROOT / "_build"
OUTPUT = ROOT / "sr_states" / "libsr_states_hip.so"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")
WALK_OUTPUT = ROOT / "sr_states" / f"_group_walk{sysconfig.get_config_var('EXT_SUFFIX')}"
LAUNCH_OUTPUT = ROOT / "sr_states" / f"_launch{sysconfig.get_config_var('EXT_SUFFIX')}"

# -ffp-contract=off: only the explicit fmaf() calls may fuse, matching the
# eager CPU reference.  Division and sqrt stay IEEE correctly rounded.
# Packed FP32 instructions are disabled on this platform.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-mcode-object-version=5",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def units() -> list[tuple[Path, list[str], Path]]:
    jobs = [(CSRC / "sr_abi.hip", [], BUILD / "sr_abi.o")]
    jobs.append((CSRC / "sr_sgdm_cast.hip", [], BUILD / "sr_sgdm_cast.o"))
    for enc in range(9):
        jobs.append((CSRC / "sr_adamw.hip", [f"-DSR_M_ENC={enc}"], BUILD / f"sr_adamw_m{enc}.o"))
    return jobs


def walk_command(output: Path, source: Path = CSRC / "group_walk.cpp") -> list[str]:
    """g++ line for a CPython extension against the running torch (the group walk by default)."""
    import torch.utils.cpp_extension as ext

    torch_lib = ext.library_paths()[0]
    return [
        CXX,
        "-O2",
        "-std=c++17",
        "-shared",
        "-fPIC",
        "-Wall",
        f"-D_GLIBCXX_USE_CXX11_ABI={int(__import__('torch')._C._GLIBCXX_USE_CXX11_ABI)}",
        f"-I{sysconfig.get_paths()['include']}",
        *(f"-I{path}" for path in ext.include_paths()),
        str(source),
        "-o",
        str(output),
        f"-L{torch_lib}",
        "-lc10",
        "-ltorch",
        "-ltorch_cpu",
        "-ltorch_python",
        f"-Wl,-rpath,{torch_lib}",
    ]


def _run(cmd: list[str]) -> None:
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"command failed ({result.returncode}): {' '.join(cmd)}\n{result.stderr}")
    noise = "not a recognized feature for this target"
    for line in result.stderr.splitlines():
        if line.strip() and noise not in line:
            print(line, file=sys.stderr)


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    """Compile every unit and link the shared library; returns its path."""
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    BUILD.mkdir(exist_ok=True)
    commands = [
        [HIPCC, *HIP_FLAGS, *defines, "-c", str(src), "-o", str(obj)]
        for src, defines, obj in units()
    ]
    walk_tmp = WALK_OUTPUT.with_name(WALK_OUTPUT.name + ".tmp")
    commands.append(walk_command(walk_tmp))
    launch_tmp = LAUNCH_OUTPUT.with_name(LAUNCH_OUTPUT.name + ".tmp")
    commands.append(walk_command(launch_tmp, CSRC / "launch.cpp"))
    workers = jobs or min(len(commands), max(1, min(16, os.cpu_count() or 1)))
    with ThreadPoolExecutor(workers) as pool:
        for cmd, _ in zip(commands, pool.map(_run, commands)):
            if verbose:
                print(" ".join(cmd))
    tmp = OUTPUT.with_suffix(".so.tmp")
    link = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp)]
    link += [str(obj) for _, _, obj in units()]
    _run(link)
    os.replace(tmp, OUTPUT)
    os.replace(walk_tmp, WALK_OUTPUT)
    os.replace(launch_tmp, LAUNCH_OUTPUT)
    return OUTPUT


def main() -> None:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("-j", "--jobs", type=int, default=None)
    parser.add_argument("-v", "--verbose", action="store_true")
    args = parser.parse_args()
    path = build(args.jobs, args.verbose)
    print(path)


if __name__ == "__main__":
    main()
