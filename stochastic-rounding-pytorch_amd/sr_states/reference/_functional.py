"""Drivers that give the fused single-tensor updates the functional reference's contract.

The reference's functional updates (sr_states/reference/adamw.py:54-105,
reference/sgd.py:44-72) read any floating-point inputs through ``.float()``,
compute in FP32, return the parameter in its own dtype and each state through
``cast`` with counter base ``state_key(seed, k)`` and shard start ``offset``.
The fused kernels take contiguous FP32/BF16 parameters and gradients and
states already held in their storage formats; ``updated`` reaches the
reference's contract from there without any CPU arithmetic:

- inputs the kernel takes as they are (states in their formats, each with a
  HIP rule) are copied and updated by one fused launch;
- otherwise every state is widened to FP32 (exact) and updated with FP32
  identity storage, which leaves the unrounded FP32 moments in the copies;
  each is then stored through ``cast`` with the key and counters the fused
  kernel uses, so a rule registered with ``register_rounding`` is applied
  exactly where the reference applies it.  For built-in rules both routes
  give the same bytes.

Parameters outside FP32/BF16 are updated in an FP32 copy and converted back
with ``Tensor.to`` (round to nearest even for floating-point dtypes,
truncation for integer ones), which is the reference's own final step;
gradients outside FP32/BF16 are widened with ``Tensor.float``.  So integer
and boolean inputs are read as the reference's ``.float()`` reads them;
complex ones are refused (``.float()`` would drop their imaginary parts).
"""

from __future__ import annotations

import torch

from .._hash import state_key
from ..formats import StateFormat
from ..optim._dtensor import DTensor
from ..rounding import cast, has_native

_KERNEL_DTYPES = (torch.float32, torch.bfloat16)
_FP32_IDENTITY = StateFormat(torch.float32, "nearest")


def check_inputs(tensors) -> None:
    """Reject inputs no GPU update can take before any copy is made."""
    if not all(isinstance(tensor, torch.Tensor) for tensor in tensors):
        raise TypeError("parameter, gradient and states must be tensors")
    for tensor in tensors:
        if DTensor is not None and isinstance(tensor, DTensor):
            raise TypeError(
                "functional state updates take local tensors: pass each DTensor's to_local() and "
                "the flat index of the shard's first element as offset"
            )
        if tensor.dtype.is_complex:
            raise TypeError(f"expected real tensors, got {tensor.dtype}")
        if tensor.device.type != "cuda":
            raise ValueError(f"sr_states updates run on the GPU; got a {tensor.device.type} tensor")


def kernel_ready(parameter, gradient, states, formats) -> bool:
    """Whether the fused kernel can update these tensors in place as they are."""
    return (
        parameter.dtype in _KERNEL_DTYPES
        and gradient.dtype in _KERNEL_DTYPES
        and all(t.is_contiguous() for t in (parameter, gradient, *states))
        and all(s.dtype == f.dtype and has_native(f.dtype, f.rounding) for s, f in zip(states, formats))
    )


def _copy(tensor, dtype):
    return tensor.to(dtype=dtype, memory_format=torch.contiguous_format, copy=True)


@torch.no_grad()
def updated(fused, parameter, gradient, states, formats, *, seed, offset, **hyperparameters):
    """(parameter', *stored states) of one update; the inputs are left unchanged.

    ``fused(parameter, gradient, *states, formats=..., seed=..., offset=...,
    **hyperparameters)`` is the in-place single-tensor HIP update.
    """
    check_inputs((parameter, gradient, *states))
    work_p = _copy(parameter, parameter.dtype if parameter.dtype in _KERNEL_DTYPES else torch.float32)
    if gradient.dtype not in _KERNEL_DTYPES:
        gradient = _copy(gradient, torch.float32)
    elif not gradient.is_contiguous():
        gradient = _copy(gradient, gradient.dtype)
    if all(s.dtype == f.dtype and has_native(f.dtype, f.rounding) for s, f in zip(states, formats)):
        stored = [_copy(s, s.dtype) for s in states]
        fused(work_p, gradient, *stored, formats=tuple(formats), seed=seed, offset=offset, **hyperparameters)
    else:
        work = [_copy(s, torch.float32) for s in states]
        fused(
            work_p, gradient, *work, formats=(_FP32_IDENTITY,) * len(work), seed=seed, offset=offset,
            **hyperparameters,
        )
        stored = [
            cast(w, dtype=f.dtype, rounding=f.rounding, seed=state_key(seed, k), offset=offset)
            for k, (w, f) in enumerate(zip(work, formats))
        ]
    if work_p.dtype != parameter.dtype:
        work_p = work_p.to(parameter.dtype)
    return (work_p, *stored)


@torch.no_grad()
def update_in_place(fused, parameter, gradient, states, formats, *, seed, offset, **hyperparameters):
    """Apply one update to ``parameter`` and ``states`` in place.

    Tensors the kernel takes as they are are updated by one fused launch with
    no copies; others are updated out of place and written back with
    ``Tensor.copy_``, as the reference's in-place updates do.
    """
    check_inputs((parameter, gradient, *states))
    if kernel_ready(parameter, gradient, states, formats):
        fused(parameter, gradient, *states, formats=tuple(formats), seed=seed, offset=offset, **hyperparameters)
        return
    new_p, *new_states = updated(
        fused, parameter, gradient, states, formats, seed=seed, offset=offset, **hyperparameters
    )
    parameter.copy_(new_p)
    for state, value in zip(states, new_states):
        state.copy_(value)
