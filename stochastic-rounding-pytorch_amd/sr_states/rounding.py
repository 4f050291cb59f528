"""Named rounding routines shared by casts and optimizers (sr_states/rounding.py).

The built-in (dtype, rule) pairs -- FP32, BF16, FP16, FP8 E4M3/E5M2 with
"nearest" or "stochastic" -- are implemented by the HIP library and run on
the GPU.  ``register_rounding`` keeps the reference's registry contract for
user rules: a registered ``reference`` callable is applied by :func:`cast`
and by optimizers that compute through ``_step_parameter``.  The fused HIP
optimizers accept only rules with a native implementation and reject the
others when the optimizer is built.
"""

from __future__ import annotations

from collections.abc import Callable
from dataclasses import dataclass

import torch

from . import _lib


@dataclass(frozen=True)
class _Routine:
    reference: Callable
    # (sr_dtype, sr_rule) codes of the HIP implementation, or None.
    native: tuple[int, int] | None = None


_ROUTINES: dict[tuple[torch.dtype, str], _Routine] = {}
_BACKENDS = ("reference", "hip")


def register_rounding(
    name: str, dtype: torch.dtype, *, reference: Callable, triton: Callable | None = None
) -> None:
    """Register a rounding rule for one storage dtype (sr_states/rounding.py:28-67).

    ``reference(x, *, dtype, seed, offset)`` receives FP32 values and returns a
    tensor of ``dtype`` with the same shape and device without mutating ``x``.
    Names and dtypes are stored in checkpoints; callables are not.  Replacing a
    registration is forbidden.  Rules registered here have no HIP
    implementation, so fused HIP optimizers reject them; ``cast`` and the
    reference-named optimizers (one parameter at a time for such groups)
    apply ``reference``.

    ``triton`` is the reference's optional Triton callback for its fused
    kernels.  It is accepted so that registrations written for the reference
    run unchanged, checked to be callable as the reference checks it, and
    not used: there is no Triton JIT in this backend.
    """
    if not isinstance(name, str) or not name:
        raise ValueError("rounding name must be a nonempty string")
    if not isinstance(dtype, torch.dtype) or not dtype.is_floating_point:
        raise ValueError("dtype must be a floating-point torch.dtype")
    if not callable(reference) or (triton is not None and not callable(triton)):
        raise TypeError("rounding implementations must be callable")
    key = (dtype, name)
    if key in _ROUTINES:
        raise ValueError(f"rounding {name!r} is already registered for {dtype}")
    _ROUTINES[key] = _Routine(reference)


def validate_rounding(dtype: torch.dtype, rounding: str, *, backend: str = "reference") -> None:
    """Validate a dtype/rule/backend combination without touching the GPU."""
    if backend not in _BACKENDS:
        raise ValueError(f"unknown rounding backend: {backend!r}")
    if (
        not isinstance(dtype, torch.dtype)
        or not isinstance(rounding, str)
        or (dtype, rounding) not in _ROUTINES
    ):
        raise ValueError(
            f"no rounding {rounding!r} registered for state_dtype={dtype}; "
            "register before loading checkpoints"
        )
    if backend == "hip" and _ROUTINES[dtype, rounding].native is None:
        raise ValueError(f"rounding {rounding!r} for {dtype} has no HIP implementation")


def has_native(dtype: torch.dtype, rounding: str) -> bool:
    """Whether a registered (dtype, rule) pair runs inside the fused HIP kernels."""
    routine = _ROUTINES.get((dtype, rounding))
    return routine is not None and routine.native is not None


def native_codes(dtype: torch.dtype, rounding: str) -> tuple[int, int]:
    """(sr_dtype, sr_rule) of a rule with a HIP implementation."""
    validate_rounding(dtype, rounding, backend="hip")
    return _ROUTINES[dtype, rounding].native


def cast(
    x: torch.Tensor,
    *,
    dtype: torch.dtype,
    rounding: str = "stochastic",
    seed: int = 0,
    offset: int = 0,
) -> torch.Tensor:
    """Apply a registered rounding routine to FP32 input, preserving shape/device.

    Built-in rules run the HIP cast: FP8 casts saturate finite overflow and
    Inf to signed max finite and keep NaN; FP16/BF16 keep IEEE overflow/Inf;
    signed zero is preserved; minifloat SR uses a 24-bit probability grid.
    Element i uses counter i + seed + offset (mod 2^32).  FP32 built-ins
    return the input unchanged, as ``Tensor.to(torch.float32)`` does.
    """
    if x.dtype != torch.float32:
        raise TypeError(f"expected torch.float32 input, got {x.dtype}")
    try:
        routine = _ROUTINES.get((dtype, rounding))
    except TypeError:  # an unhashable rule: validate_rounding names the error
        routine = None
    if routine is not None and routine.native is not None:
        # A built-in rule: the HIP cast returns x's shape and device in dtype.
        return routine.reference(x, dtype=dtype, seed=seed, offset=offset)
    validate_rounding(dtype, rounding)
    result = _ROUTINES[dtype, rounding].reference(x, dtype=dtype, seed=seed, offset=offset)
    if not isinstance(result, torch.Tensor):
        raise TypeError("rounding routine must return a tensor")
    if result.dtype != dtype or result.shape != x.shape or result.device != x.device:
        raise ValueError(
            "rounding routine must preserve shape/device and return the requested dtype"
        )
    return result


def _builtin(code: int, rule: int) -> Callable:
    if code == _lib.SR_F32:
        def routine(x, *, dtype, seed, offset):
            return x
    else:
        def routine(x, *, dtype, seed, offset):
            # Imported here: sr_states.hip imports this module.
            from .hip.cast import native_cast

            return native_cast(x if x.is_contiguous() else x.contiguous(), dtype=dtype, rule=rule,
                               seed=seed, offset=offset)

    routine.__name__ = f"hip_cast_{code}_{rule}"
    return routine


for _dtype, _code in _lib.DTYPE_CODES.items():
    for _name, _rule in _lib.RULE_CODES.items():
        _ROUTINES[_dtype, _name] = _Routine(_builtin(_code, _rule), (_code, _rule))
