"""Validation shared by the fused HIP updates (sr_states/triton/_optimizer.py)."""

from __future__ import annotations

import math
from bisect import bisect_left

import torch

from ..optim._dtensor import is_dtensor
from ..rounding import validate_rounding

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


def validate_tensors(parameter, gradient, *states):
    tensors = (parameter, gradient, *states)
    if any(is_dtensor(t) for t in tensors):
        raise TypeError(
            "fused state updates take local tensors: pass each DTensor's to_local() and the "
            "flat index of the shard's first element as offset"
        )
    if parameter.device.type != "cuda":
        raise ValueError("fused state updates require GPU tensors")
    validate_tensor_layout(tensors)
    if parameter.numel():
        validate_no_overlap(
            (t.data_ptr(), t.data_ptr() + t.nbytes, role != 1) for role, t in enumerate(tensors)
        )
