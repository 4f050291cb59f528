"""Functional AdamW under the reference's names (sr_states/reference/adamw.py:12-127).

``adamw_step`` returns the updated parameter and the stored moments;
``adamw_step_`` writes them back in place.  Both run the fused HIP update on
gfx950 and take GPU tensors only.  The arithmetic is the fused kernel's:
``m' = fma(g, 1-beta1, beta1*m)``, ``v' = fma((1-beta2)*g, g, beta2*v)``,
``p' = p*(1-lr*wd) + (-lr/(1-beta1**step))*m' / (sqrt(v')/sqrt(1-beta2**step) + eps)``,
with the parameter computed from the unrounded FP32 moments, rounded to its
own dtype (nearest even), and each moment stored through its format with
counter base ``state_key(seed, k)`` and shard start ``offset``.

Like the reference, they check no hyperparameter: any learning rate,
epsilon and weight decay are taken (a negative learning rate ascends).  The
one limit is the launch's exact division by sqrt(1 - beta2**step), which
takes every beta2 in [0, 1); beta1 = 1 divides by zero as in the reference.
``step`` is any real number of at least 1 (a Python or NumPy integer or
float), which only the bias corrections use, as in the reference
(reference/adamw.py:73-84); a tensor is refused, where the reference's
``addcdiv_`` fails on one.
"""

from __future__ import annotations

import numbers

import torch

from ..formats import resolve_formats
from ..hip.adamw import adamw_step_any_hyperparameters_
from ._functional import update_in_place, updated

_NAMES = ("exp_avg", "exp_avg_sq")


def _formats(step, state_dtype, formats, rounding):
    if not isinstance(step, numbers.Real):
        raise TypeError(f"step must be a real number, not {type(step).__name__}")
    if step < 1:
        raise ValueError("step must be at least 1")
    return resolve_formats(_NAMES, formats, state_dtype=state_dtype, rounding=rounding)


def adamw_step(
    parameter: torch.Tensor,
    gradient: torch.Tensor,
    exp_avg: torch.Tensor,
    exp_avg_sq: torch.Tensor,
    *,
    lr: float,
    beta1: float,
    beta2: float,
    eps: float,
    weight_decay: float,
    step: int,
    state_dtype: torch.dtype | None = None,
    formats: tuple | dict | None = None,
    rounding: str | None = None,
    seed: int = 0,
    offset: int = 0,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Return one AdamW update as new tensors (reference/adamw.py:12-51).

    Each moment derives its counter base from the update key ``seed``;
    ``offset`` is the flat starting index of this shard.  The moments are
    returned in their storage formats (BF16 stochastic by default) and the
    parameter in its own dtype; the inputs are not modified.
    """
    resolved = _formats(step, state_dtype, formats, rounding)
    return tuple(
        updated(
            adamw_step_any_hyperparameters_, parameter, gradient, (exp_avg, exp_avg_sq), resolved, seed=seed,
            offset=offset, lr=lr, beta1=beta1, beta2=beta2, eps=eps, weight_decay=weight_decay, step=step,
        )
    )


@torch.no_grad()
def adamw_step_(
    parameter: torch.Tensor,
    gradient: torch.Tensor,
    exp_avg: torch.Tensor,
    exp_avg_sq: torch.Tensor,
    *,
    lr: float,
    beta1: float,
    beta2: float,
    eps: float,
    weight_decay: float,
    step: int,
    state_dtype: torch.dtype | None = None,
    formats: tuple | dict | None = None,
    rounding: str | None = None,
    seed: int = 0,
    offset: int = 0,
) -> None:
    """Apply the update in place, including state write-back (reference/adamw.py:108-127).

    Contiguous FP32/BF16 parameters and gradients with states held in their
    formats are updated by one fused launch; other inputs are updated out of
    place and copied back.
    """
    resolved = _formats(step, state_dtype, formats, rounding)
    update_in_place(
        adamw_step_any_hyperparameters_, parameter, gradient, (exp_avg, exp_avg_sq), resolved, seed=seed,
        offset=offset, lr=lr, beta1=beta1, beta2=beta2, eps=eps, weight_decay=weight_decay, step=step,
    )
