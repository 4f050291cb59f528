"""The C ABI library loads, exports every declared symbol, and validates arguments (CPU).

No call here reaches the GPU: the argument checks of each entry point run
before any HIP call, so invalid arguments return an error code on a machine
without a GPU.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

HEADER = Path(__file__).resolve().parents[1] / "include" / "sr_states_hip.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(sr_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_expected_surface():
    assert declared_functions() == sorted(
        [
            "sr_abi_version",
            "sr_last_error",
            "sr_lane_elements",
            "sr_update_key",
            "sr_state_key",
            "sr_cast",
            "sr_neighbors",
            "sr_adamw_step",
            "sr_adamw_multi",
            "sr_adamw_multi_noalloc",
            "sr_sgdm_step",
            "sr_sgdm_multi",
        ]
    )


def test_library_exports_every_declared_symbol():
    from sr_states import _lib

    handle = _lib.library()
    for name in declared_functions():
        assert hasattr(handle, name), name
    assert set(_lib.SIGNATURES) == set(declared_functions())
    assert handle.sr_abi_version() == _lib.ABI_VERSION


def test_header_constants_match_the_binding():
    from sr_states import _lib

    text = HEADER.read_text()
    assert f"#define SR_ABI_VERSION {_lib.ABI_VERSION}" in text
    assert f"#define SR_LANE_ELEMENTS {_lib.LANE_ELEMENTS}" in text
    assert f"#define SR_LANE_ELEMENTS_NARROW {_lib.LANE_ELEMENTS_NARROW}" in text
    assert "#define SR_ROW_VECTOR 1u" in text and _lib.ROW_VECTOR == 1
    assert "#define SR_ROW_KEYED 2u" in text and _lib.ROW_KEYED == 2
    assert _lib.ROW_DTYPE.itemsize == 64
    assert ctypes.sizeof(_lib.AdamWHparams) == 32 and ctypes.sizeof(_lib.SgdmHparams) == 8


def test_invalid_arguments_fail_before_any_device_work():
    from sr_states import _lib

    lib = _lib.library()
    assert lib.sr_cast(None, None, 16, 9, 0, 0, 0, 256, None) == 1
    assert b"unsupported cast dtype" in lib.sr_last_error()
    assert lib.sr_cast(None, None, 16, 1, 1, 0, 0, 100, None) == 1
    assert b"block size" in lib.sr_last_error()
    assert lib.sr_cast(None, None, 0, 1, 1, 0, 0, 256, None) == 0  # empty: nothing to do
    assert lib.sr_neighbors(None, None, None, 16, 0, None) == 1  # FP32 has no neighbours
    assert b"neighbors support" in lib.sr_last_error()
    assert lib.sr_neighbors(None, None, None, 16, 3, None) == 1
    assert b"null pointer" in lib.sr_last_error()
    assert lib.sr_neighbors(None, None, None, -1, 3, None) == 1
    assert lib.sr_neighbors(None, None, None, 0, 3, None) == 0  # empty: nothing to do
    hp = _lib.AdamWHparams()
    assert lib.sr_adamw_step(None, None, None, None, 8, 2, 0, 1, 1, 1, 1, ctypes.byref(hp), 0, 0, 256, None) == 1
    assert b"FP32 or BF16" in lib.sr_last_error()
    assert lib.sr_adamw_multi(None, None, None, 1, 1, 0, 0, 1, 1, 1, 1, ctypes.byref(hp), 0, 0, 256, None) == 1
    assert b"null argument" in lib.sr_last_error()
    # The division by sqrt(1 - beta2^t) is exact for values in [2^-27, 1],
    # which every 0 <= beta2 < 1 and step >= 1 give; zero (hp's default),
    # NaN and values above 1 are refused.
    for correction in (0.0, 2.0**-28, 1.0000001, float("nan")):
        hp.correction2_sqrt = correction
        for call in (
            lambda: lib.sr_adamw_step(None, None, None, None, 8, 0, 0, 1, 1, 1, 1, ctypes.byref(hp), 0, 0, 256, None),
            lambda: lib.sr_adamw_multi(1, 1, None, 1, 1, 0, 0, 1, 1, 1, 1, ctypes.byref(hp), 0, 0, 256, None),
        ):
            assert call() == 1
            assert b"correction2_sqrt" in lib.sr_last_error()
    sp = _lib.SgdmHparams()
    assert lib.sr_sgdm_multi(None, None, 0, 1, 0, 0, 7, 1, ctypes.byref(sp), 0, 0, 256, None) == 1
    assert b"unsupported state" in lib.sr_last_error()


def test_noalloc_checks_its_host_tables_before_any_device_work():
    """sr_adamw_multi_noalloc reads its tables on the host; bad ones never reach the GPU.

    The pointers are fake addresses: nothing is dereferenced before the checks.
    """
    import numpy as np

    from sr_states import _lib
    from sr_states.hip._multi_tensor import build_records

    lib = _lib.library()
    hp = _lib.AdamWHparams(beta1=0.9, beta2=0.999, one_minus_beta1=0.1, one_minus_beta2=0.001,
                           neg_step_size=-1e-3, correction2_sqrt=0.5, decay=1.0, eps=1e-8)
    tile = 128 * _lib.LANE_ELEMENTS
    pointers = [(0x10000, 0x20000, 0x30000, 0x40000), (0x50000, 0x60000, 0x70000, 0x80000)]
    records = build_records([(4099, 0, 0), (600, 1, 0)], pointers, tile)
    total = int(records["tile_end"][-1])

    def status(table=records, nrows=2, tiles=total, scalars=None, block=128):
        return lib.sr_adamw_multi_noalloc(table.ctypes.data, None if scalars is None else scalars.ctypes.data,
                                          nrows, tiles, 0, 0, 1, 1, 1, 1, ctypes.byref(hp), 0, 0, block, None)

    cases = [
        (dict(nrows=_lib.NOALLOC_MAX_ROWS + 1), b"row count"),
        (dict(tiles=_lib.NOALLOC_MAX_TILES + 1), b"tiles outside"),
        (dict(tiles=0), b"tiles outside"),
        (dict(tiles=total - 1), b"rows cover"),
        (dict(block=256), b"tiles for"),
        (dict(scalars=np.array([-1.0, 0.5, -1.0, 2.0], dtype=np.float32)), b"correction2_sqrt"),
    ]
    for kwargs, message in cases:
        assert status(**kwargs) == 1, kwargs
        assert message in lib.sr_last_error(), (kwargs, lib.sr_last_error())
    negative = records.copy()
    negative["numel"][0] = 0
    assert status(negative) == 1 and b"numel 0 below 1" in lib.sr_last_error()
    flagged = records.copy()
    flagged["flags"][1] = 8
    assert status(flagged) == 1 and b"unknown flags" in lib.sr_last_error()
    assert lib.sr_adamw_multi_noalloc(None, None, 2, total, 0, 0, 1, 1, 1, 1, ctypes.byref(hp), 0, 0, 128,
                                      None) == 1
    assert b"null argument" in lib.sr_last_error()


def test_call_raises_with_the_library_message():
    from sr_states import _lib

    with pytest.raises(RuntimeError, match="unsupported cast dtype"):
        _lib.call("sr_cast", None, None, 16, 9, 0, 0, 0, 256, None)


def test_lane_width_of_every_optimizer_launch():
    """Every dtype combination currently moves SR_LANE_ELEMENTS per lane; unknown dtypes give 0."""
    import itertools

    import torch

    from sr_states import _lib

    lib = _lib.library()
    states = (_lib.SR_F32, _lib.SR_BF16, _lib.SR_F16, _lib.SR_E4M3, _lib.SR_E5M2)
    for p, g in itertools.product((_lib.SR_F32, _lib.SR_BF16), repeat=2):
        for a, b in itertools.product(states, repeat=2):
            assert lib.sr_lane_elements(p, g, a, b) == _lib.LANE_ELEMENTS, (p, g, a, b)
    assert lib.sr_lane_elements(0, 0, 5, 0) == 0 and lib.sr_lane_elements(-1, 0, 0, 0) == 0
    assert _lib.lane_elements(torch.float32, torch.float32, torch.float8_e4m3fn, torch.bfloat16) == 4


@pytest.mark.parametrize("compiler,flags", [("gcc", ["-std=c99", "-x", "c"]), ("g++", ["-std=c++11", "-x", "c++"])])
def test_header_is_strict_c99_and_cxx11(tmp_path, compiler, flags):
    """include/sr_states_hip.h compiles warning-free, pedantic, with nothing but <stdint.h>."""
    import subprocess
    from pathlib import Path

    include = Path(__file__).resolve().parents[1] / "include"
    source = tmp_path / "use_header.c"
    source.write_text('#include "sr_states_hip.h"\n'
                      "int main(void) { sr_row r; r.numel = 1; return r.numel == 1 && sr_abi_version() == SR_ABI_VERSION ? 0 : 1; }\n")
    subprocess.run([compiler, *flags, "-Wall", "-Wextra", "-Werror", "-pedantic", "-I", str(include), "-c",
                    str(source), "-o", str(tmp_path / "use_header.o")], check=True)
