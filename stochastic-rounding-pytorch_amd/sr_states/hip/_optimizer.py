"""Validation shared by the fused HIP updates (sr_states/triton/_optimizer.py)."""

from __future__ import annotations

import math
from bisect import bisect_left

import torch

from ..formats import StateFormat, resolve_formats
from ..optim._dtensor import DTensor
from ..rounding import native_codes, validate_rounding

# Workgroup sizes (threads).  Results do not depend on the choice.
BLOCK_SIZES = (128, 256, 512, 1024)
# The reference's default is 256 (triton/adamw.py:262, triton/sgd.py:189).
# On MI355X, 128-thread workgroups stream 0.9-1.4% faster than 256 on the
# 1.5 G-element AdamW, the 2^26-element tensor and the SGDM workload, and tie
# on the FP8 mixed one, with four elements per lane and non-temporal
# accesses.  Either value is valid for both backends, so checkpoints load
# both ways.
DEFAULT_BLOCK_SIZE = 128
_PARAMETER_DTYPES = (torch.float32, torch.bfloat16)


def validate_options(rounding, block_size, state_dtype):
    validate_rounding(state_dtype, rounding, backend="hip")
    if block_size not in BLOCK_SIZES:
        raise ValueError(f"block_size must be one of {BLOCK_SIZES}")


def nonnegative(name, value):
    if not math.isfinite(value) or value < 0:
        raise ValueError(f"invalid {name}: {value}")


def validate_tensor_layout(tensors):
    """Same device, identical shapes, contiguous; FP32/BF16 parameter and gradient."""
    parameter, gradient, *_ = tensors
    device, shape = parameter.device, parameter.shape
    for tensor in tensors:
        if tensor.device != device:
            raise ValueError("all tensors must be on the same GPU device")
        if tensor.shape != shape:
            raise ValueError("all tensors must have identical shapes")
        if not tensor.is_contiguous():
            raise ValueError("fused state updates require contiguous tensors")
    if parameter.dtype not in _PARAMETER_DTYPES or gradient.dtype not in _PARAMETER_DTYPES:
        raise TypeError("parameter and gradient must be FP32 or BF16")


def validate_no_overlap(spans):
    """Reject any byte a written span shares with another span of the same device.

    ``spans`` holds (start, end, written) byte ranges.  Read-only ranges
    (gradients) may share storage with each other.  Sorted by start, the
    written ranges must each end before the next one begins; they are then
    ordered by their ends too, so a read range [a, b) meets a written one
    exactly when the last written range starting before b ends after a.
    """
    spans = list(spans)
    written = sorted((start, end) for start, end, write in spans if write)
    starts = [start for start, _ in written]
    clash = any(end > next_start for (_, end), next_start in zip(written, starts[1:]))
    for start, end, write in spans:
        if clash:
            break
        if not write:
            last = bisect_left(starts, end) - 1
            clash = last >= 0 and written[last][1] > start
    if clash:
        raise ValueError("parameter, gradient, and state must not overlap optimizer writes")


def reject_dtensors(*tensors):
    """The functional updates take local tensors (the native entries check the rest)."""
    if DTensor is not None:
        for tensor in tensors:
            if isinstance(tensor, DTensor):
                raise TypeError(
                    "fused state updates take local tensors: pass each DTensor's to_local() and the "
                    "flat index of the shard's first element as offset"
                )


# Successful resolutions of the functional updates' formats.  Only built-in
# rules have HIP implementations, and a registration can never replace one,
# so a resolution that succeeded once holds for the life of the process.
_NATIVE_CODES: dict = {}


def resolve_native_codes(names, states, formats, rounding, block_size):
    """Each state's (sr_dtype, sr_rule) for one functional update (triton/adamw.py:196-205).

    ``formats`` None takes every state's own dtype with ``rounding``
    (stochastic by default).  Raises as ``resolve_formats`` and
    ``validate_options`` do, and when a state's dtype is not its format's.
    """
    dtypes = tuple(state.dtype for state in states)
    key = (names, dtypes, formats, rounding, block_size)
    try:
        return _NATIVE_CODES[key]
    except KeyError:
        pass
    except TypeError:  # unhashable formats (a dict): resolve every time
        key = None
    if formats is None:
        rule = "stochastic" if rounding is None else rounding
        resolved = resolve_formats(names, tuple(StateFormat(d, rule) for d in dtypes), backend="hip")
    else:
        resolved = resolve_formats(names, formats, rounding=rounding, backend="hip")
    for dtype, fmt in zip(dtypes, resolved):
        validate_options(fmt.rounding, block_size, fmt.dtype)
        if dtype != fmt.dtype:
            raise ValueError("state dtype does not match its state format")
    codes = tuple(native_codes(fmt.dtype, fmt.rounding) for fmt in resolved)
    if key is not None and len(_NATIVE_CODES) < 1024:
        _NATIVE_CODES[key] = codes
    return codes
