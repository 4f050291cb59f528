"""AdamW hyperparameters: validation and the FP32 launch scalars."""

from __future__ import annotations

import math

from .. import _lib


def validate_adamw(group):
    """Reject invalid AdamW group values (sr_states/optim/adamw.py:12-18)."""
    for name in ("lr", "eps", "weight_decay"):
        if not math.isfinite(group[name]) or group[name] < 0:
            raise ValueError(f"invalid {name}: {group[name]}")
    betas = group["betas"]
    if len(betas) != 2 or any(not 0 <= beta < 1 for beta in betas):
        raise ValueError(f"invalid beta values: {betas}")


def adamw_scalars(lr, beta1, beta2, eps, weight_decay, step) -> tuple:
    """Launch scalars for one bias-correction step, as Python doubles.

    In the order of sr_adamw_hparams' fields: beta1, beta2, 1 - beta1,
    1 - beta2, -lr / (1 - beta1^step), sqrt(1 - beta2^step),
    1 - lr * weight_decay, eps.  The eager reference evaluates each in Python
    double precision and rounds it to FP32 when it meets an FP32 tensor
    (sr_states/reference/adamw.py:86-96); the launches round each the same
    way (ctypes' c_float conversion, or a C cast in the native entries).
    """
    bias_correction1 = 1.0 - beta1**step
    bias_correction2 = 1.0 - beta2**step
    return (beta1, beta2, 1.0 - beta1, 1.0 - beta2, -lr / bias_correction1, bias_correction2**0.5,
            1.0 - lr * weight_decay, eps)


def adamw_hparams(lr, beta1, beta2, eps, weight_decay, step) -> _lib.AdamWHparams:
    """``adamw_scalars`` rounded to FP32 in the C ABI's sr_adamw_hparams."""
    return _lib.AdamWHparams(*adamw_scalars(lr, beta1, beta2, eps, weight_decay, step))


def __getattr__(name):
    """``AdamWReferenceSR``/``AdamWReferenceRN``, defined with the other reference-named optimizers."""
    if name in ("AdamWReferenceSR", "AdamWReferenceRN"):
        from . import eager

        return getattr(eager, name)
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
