"""Allocating casts on the GPU (sr_states/triton/cast.py and sr_cast.py).

Every cast launches the HIP cast kernel: counter(i) = i + seed + offset mod
2^32, one hash per element for stochastic rules.  ``block_size``,
``num_warps`` and ``store_mode`` are validated against the reference's
choices.  On CDNA a wavefront is 64 lanes, so ``num_warps`` selects the
wavefronts per workgroup; the tile is fixed at 8 elements per lane and the
output bits are always stored directly.  None of them changes a result.
"""

from __future__ import annotations

import torch

from .. import _lib
from ..rounding import native_codes, validate_rounding
from ._common import validate_device

CAST_BLOCK_SIZES = (128, 256, 512, 1024, 2048, 4096)
CAST_NUM_WARPS = (1, 2, 4, 8)
CAST_STORE_MODES = ("convert", "bits")
_DEFAULT_THREADS = 256


def native_cast(x, *, dtype, rule, seed=0, offset=0, threads=_DEFAULT_THREADS, out=None):
    """Cast contiguous FP32 ``x`` with HIP rule code ``rule``.

    Returns a new tensor, or writes into ``out`` (contiguous, ``dtype``, x's
    shape and device, disjoint from x) when given.
    """
    device = x.device
    if device.type != "cuda":
        raise ValueError(f"sr_states casts run on the GPU; got a {device.type} tensor")
    validate_device(device)
    output = torch.empty_like(x, dtype=dtype, memory_format=torch.contiguous_format) if out is None else out
    # The native entry checks `output` (dtype, shape, device, contiguity and
    # no byte shared with x), then calls sr_cast with x's device current.
    status = _lib.launcher().cast(x, output, _lib.DTYPE_CODES[dtype], rule, int(seed) & 0xFFFFFFFF,
                                  int(offset) & 0xFFFFFFFF, threads, _lib.stream_handle(device))
    if status:
        _lib.check("sr_cast", status)
    return output


NEIGHBOR_DTYPES = (torch.bfloat16, torch.float16, torch.float8_e4m3fn, torch.float8_e5m2)


def native_neighbors(x, dtype):
    """(lower, upper): the ordered ``dtype`` neighbours of contiguous GPU FP32 ``x``."""
    if x.device.type != "cuda":
        raise ValueError(f"sr_states neighbors run on the GPU; got a {x.device.type} tensor")
    validate_device(x.device)
    lower = torch.empty(x.shape, dtype=dtype, device=x.device)
    upper = torch.empty(x.shape, dtype=dtype, device=x.device)
    if x.numel():
        with _lib.on_device(x.device):
            _lib.call(
                "sr_neighbors",
                x.data_ptr(),
                lower.data_ptr(),
                upper.data_ptr(),
                x.numel(),
                _lib.DTYPE_CODES[dtype],
                _lib.stream_handle(x.device),
            )
    return lower, upper


def _launch_shape(block_size, num_warps):
    if block_size not in CAST_BLOCK_SIZES:
        raise ValueError(f"block_size must be one of {CAST_BLOCK_SIZES}")
    if num_warps not in CAST_NUM_WARPS:
        raise ValueError(f"num_warps must be one of {CAST_NUM_WARPS}")
    return 64 * num_warps


def _check_input(x, what):
    if x.device.type != "cuda":
        raise ValueError(f"{what} requires a GPU tensor")
    if x.dtype != torch.float32:
        raise TypeError(f"expected torch.float32 input, got {x.dtype}")
    if not x.is_contiguous():
        raise ValueError(f"{what} requires a contiguous input")


def cast(x, *, dtype, rounding="stochastic", seed=0, offset=0, block_size=256, num_warps=4):
    """Cast contiguous GPU FP32 input with a built-in rule (triton/cast.py:32-60)."""
    validate_rounding(dtype, rounding, backend="hip")
    _check_input(x, "HIP cast")
    threads = _launch_shape(block_size, num_warps)
    _, rule = native_codes(dtype, rounding)
    return native_cast(x, dtype=dtype, rule=rule, seed=seed, offset=offset, threads=threads)


def sr_cast_bf16(x, *, seed, offset=0, block_size=256, num_warps=4, store_mode="convert"):
    """Stochastically cast contiguous GPU FP32 input to BF16 (triton/sr_cast.py:89-115)."""
    return _cast_bf16(x, seed, offset, block_size, num_warps, store_mode, _lib.SR_STOCHASTIC)


def rn_cast_bf16(x, *, block_size=256, num_warps=4):
    """Round to nearest, ties to even, through the same launch path (triton/sr_cast.py:117-128)."""
    return _cast_bf16(x, 0, 0, block_size, num_warps, "convert", _lib.SR_NEAREST)


def _cast_bf16(x, seed, offset, block_size, num_warps, store_mode, rule):
    _check_input(x, "BF16 cast")
    threads = _launch_shape(block_size, num_warps)
    if store_mode not in CAST_STORE_MODES:
        raise ValueError(f"store_mode must be one of {CAST_STORE_MODES}")
    return native_cast(
        x, dtype=torch.bfloat16, rule=rule, seed=seed, offset=offset, threads=threads
    )
