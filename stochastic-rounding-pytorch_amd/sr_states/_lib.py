"""ctypes binding of libsr_states_hip.so (the C ABI declared in include/sr_states_hip.h).

torch is imported first so that the library's ``libamdhip64.so.7`` dependency
resolves to the HIP runtime torch already loaded: streams and device pointers
handed over from torch are then valid in the library.  There is no fallback:
if the library is missing every entry point raises.
"""

from __future__ import annotations

import contextlib
import ctypes
import threading
from functools import cache
from pathlib import Path

import numpy as np
import torch  # noqa: F401  (load torch's HIP runtime before the library)

LIBRARY_PATH = Path(__file__).with_name("libsr_states_hip.so")
ABI_VERSION = 5
# Elements per lane of a launch (SR_LANE_ELEMENTS / _NARROW); lane_elements()
# gives the width of a particular launch.
LANE_ELEMENTS, LANE_ELEMENTS_NARROW = 4, 8

# enum sr_dtype / sr_rule
SR_F32, SR_BF16, SR_F16, SR_E4M3, SR_E5M2 = range(5)
SR_NEAREST, SR_STOCHASTIC = 0, 1
ROW_VECTOR = 1
ROW_KEYED = 2
# Scratch limits of sr_adamw_multi_noalloc (SR_NOALLOC_MAX_ROWS / _TILES).
NOALLOC_MAX_ROWS, NOALLOC_MAX_TILES = 4096, 1 << 22

DTYPE_CODES = {
    torch.float32: SR_F32,
    torch.bfloat16: SR_BF16,
    torch.float16: SR_F16,
    torch.float8_e4m3fn: SR_E4M3,
    torch.float8_e5m2: SR_E5M2,
}
RULE_CODES = {"nearest": SR_NEAREST, "stochastic": SR_STOCHASTIC}

# struct sr_row (64 bytes), built on the host and uploaded as bytes.
ROW_DTYPE = np.dtype(
    [
        ("ptr", "<u8", (4,)),
        ("numel", "<i8"),
        ("tile_begin", "<u4"),
        ("tile_end", "<u4"),
        ("param_index", "<u4"),
        ("shard_start", "<u4"),
        ("flags", "<u4"),
        ("reserved", "<u4"),
    ]
)
assert ROW_DTYPE.itemsize == 64


class AdamWHparams(ctypes.Structure):
    _fields_ = [
        ("beta1", ctypes.c_float),
        ("beta2", ctypes.c_float),
        ("one_minus_beta1", ctypes.c_float),
        ("one_minus_beta2", ctypes.c_float),
        ("neg_step_size", ctypes.c_float),
        ("correction2_sqrt", ctypes.c_float),
        ("decay", ctypes.c_float),
        ("eps", ctypes.c_float),
    ]


class SgdmHparams(ctypes.Structure):
    _fields_ = [("momentum", ctypes.c_float), ("neg_lr", ctypes.c_float)]


_vp, _i64, _u32, _u64, _int = (
    ctypes.c_void_p,
    ctypes.c_int64,
    ctypes.c_uint32,
    ctypes.c_uint64,
    ctypes.c_int,
)

# name -> (restype, argtypes); the complete exported surface of the header.
SIGNATURES = {
    "sr_abi_version": (_int, []),
    "sr_last_error": (ctypes.c_char_p, []),
    "sr_lane_elements": (_int, [_int, _int, _int, _int]),
    "sr_update_key": (_u32, [_u64, _u64, _u32]),
    "sr_state_key": (_u32, [_u32, _u32]),
    "sr_cast": (_int, [_vp, _vp, _i64, _int, _int, _u32, _u32, _int, _vp]),
    "sr_neighbors": (_int, [_vp, _vp, _vp, _i64, _int, _vp]),
    "sr_adamw_step": (
        _int,
        [_vp, _vp, _vp, _vp, _i64, _int, _int, _int, _int, _int, _int,
         ctypes.POINTER(AdamWHparams), _u32, _u32, _int, _vp],
    ),
    "sr_adamw_multi": (
        _int,
        [_vp, _vp, _vp, _int, _u32, _int, _int, _int, _int, _int, _int,
         ctypes.POINTER(AdamWHparams), _u64, _u64, _int, _vp],
    ),
    "sr_adamw_multi_noalloc": (
        _int,
        [_vp, _vp, _int, _u32, _int, _int, _int, _int, _int, _int,
         ctypes.POINTER(AdamWHparams), _u64, _u64, _int, _vp],
    ),
    "sr_sgdm_step": (
        _int,
        [_vp, _vp, _vp, _i64, _int, _int, _int, _int, ctypes.POINTER(SgdmHparams),
         _u32, _u32, _int, _vp],
    ),
    "sr_sgdm_multi": (
        _int,
        [_vp, _vp, _int, _u32, _int, _int, _int, _int, ctypes.POINTER(SgdmHparams),
         _u64, _u64, _int, _vp],
    ),
}

_lock = threading.Lock()
_handle: ctypes.CDLL | None = None


def library() -> ctypes.CDLL:
    """Load the HIP library once; raise if it has not been built."""
    global _handle
    if _handle is not None:
        return _handle
    with _lock:
        if _handle is None:
            if not LIBRARY_PATH.exists():
                raise RuntimeError(
                    f"sr_states HIP library not built: {LIBRARY_PATH} is missing "
                    "(run stochastic-rounding-pytorch_amd/build.py)"
                )
            handle = ctypes.CDLL(str(LIBRARY_PATH))
            for name, (restype, argtypes) in SIGNATURES.items():
                function = getattr(handle, name)
                function.restype = restype
                function.argtypes = argtypes
            version = handle.sr_abi_version()
            if version != ABI_VERSION:
                raise RuntimeError(f"library ABI {version} does not match binding ABI {ABI_VERSION}")
            _handle = handle
    return _handle


def check(name: str, status: int) -> None:
    if status != 0:
        message = library().sr_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed ({status}): {message}")


def call(name: str, *args) -> None:
    """Call a status-returning entry point and raise RuntimeError on failure."""
    check(name, getattr(library(), name)(*args))


@cache
def lane_elements(*dtypes: torch.dtype) -> int:
    """Elements per lane of a launch with (parameter, gradient, state0, state1) dtypes.

    SGDM passes its momentum dtype twice.
    """
    lanes = library().sr_lane_elements(*(DTYPE_CODES[d] for d in dtypes))
    if lanes <= 0:
        raise ValueError(f"no lane width for operand dtypes {dtypes}")
    return lanes


# torch's C accessors of the current device and of the current stream's raw
# handle: about 0.1 us each, where the public torch.cuda.current_stream(d)
# .cuda_stream builds a Stream object (2 us) and the torch.cuda.device
# context manager costs 1.4 us, which set the floor of a small launch.  The
# public forms stand in where a torch build lacks them.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_current_device = getattr(torch._C, "_cuda_getDevice", None) or torch.cuda.current_device


def _index(device: torch.device) -> int:
    return _current_device() if device.index is None else device.index


def stream_handle(device: torch.device) -> int:
    """The raw handle of the current stream on ``device``: the launch stream."""
    if _raw_stream is not None:
        return _raw_stream(_index(device))
    return torch.cuda.current_stream(device).cuda_stream


def on_device(device: torch.device):
    """A context in which ``device`` is current: nothing to set when it already is."""
    if _current_device() == _index(device):
        return contextlib.nullcontext()
    return torch.cuda.device(device)


_launcher = None


def launcher():
    """The native entries of the single-tensor launches (sr_states/_launch), bound to this library."""
    global _launcher
    if _launcher is None:
        from . import _launch as module

        lib = library()
        module.bind(*(ctypes.cast(getattr(lib, name), ctypes.c_void_p).value
                      for name in ("sr_cast", "sr_adamw_step", "sr_sgdm_step")))
        _launcher = module
    return _launcher


def low64(value: int) -> int:
    return int(value) & 0xFFFFFFFFFFFFFFFF


def low32(value: int) -> int:
    return int(value) & 0xFFFFFFFF
