"""Momentum-SGD hyperparameters: validation and the FP32 launch scalars."""

from __future__ import annotations

import math

from .. import _lib


def validate_sgdm(group):
    """Reject invalid SGDM group values (sr_states/optim/sgd.py:12-16)."""
    if not math.isfinite(group["lr"]) or group["lr"] < 0:
        raise ValueError(f"invalid learning rate: {group['lr']}")
    if not 0 <= group["momentum"] < 1:
        raise ValueError(f"invalid momentum value: {group['momentum']}")


def sgdm_scalars(lr, momentum) -> tuple:
    """Scalars of ``u = u*momentum + g; p = p + (-lr)*u`` (reference/sgd.py:62-64), as doubles."""
    return (momentum, -lr)


def sgdm_hparams(lr, momentum) -> _lib.SgdmHparams:
    """``sgdm_scalars`` rounded to FP32 in the C ABI's sr_sgdm_hparams."""
    return _lib.SgdmHparams(*sgdm_scalars(lr, momentum))


def __getattr__(name):
    """``SGDMReferenceSR``/``SGDMReferenceRN``, defined with the other reference-named optimizers."""
    if name in ("SGDMReferenceSR", "SGDMReferenceRN"):
        from . import eager

        return getattr(eager, name)
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
