"""Functional momentum SGD under the reference's names (sr_states/reference/sgd.py:12-84).

``sgdm_step`` returns the updated parameter and the stored momentum;
``sgdm_step_`` writes them back in place.  Both run the fused HIP update on
gfx950 and take GPU tensors only: ``u' = fma(momentum_factor, u, g)``,
``p' = p - lr*u'`` from the unrounded FP32 momentum, the parameter rounded to
its own dtype (nearest even) and the momentum stored through its format with
counter base ``state_key(seed, 0)`` and shard start ``offset``.

Like the reference, they check no hyperparameter: any ``lr`` and
``momentum_factor`` are taken.
"""

from __future__ import annotations

import torch

from ..formats import resolve_formats
from ..hip.sgd import sgdm_step_any_hyperparameters_
from ._functional import update_in_place, updated

_NAMES = ("momentum_buffer",)


def sgdm_step(
    parameter: torch.Tensor,
    gradient: torch.Tensor,
    momentum: torch.Tensor,
    *,
    lr: float,
    momentum_factor: float,
    state_dtype: torch.dtype | None = None,
    formats: tuple | dict | None = None,
    rounding: str | None = None,
    seed: int = 0,
    offset: int = 0,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Return one momentum-SGD update as new tensors (reference/sgd.py:12-41).

    The momentum derives its counter base from the update key ``seed``;
    ``offset`` is the flat starting index of this shard.  The inputs are not
    modified.
    """
    resolved = resolve_formats(_NAMES, formats, state_dtype=state_dtype, rounding=rounding)
    return tuple(
        updated(
            sgdm_step_any_hyperparameters_, parameter, gradient, (momentum,), resolved, seed=seed, offset=offset,
            lr=lr, momentum_factor=momentum_factor,
        )
    )


@torch.no_grad()
def sgdm_step_(
    parameter: torch.Tensor,
    gradient: torch.Tensor,
    momentum: torch.Tensor,
    *,
    lr: float,
    momentum_factor: float,
    state_dtype: torch.dtype | None = None,
    formats: tuple | dict | None = None,
    rounding: str | None = None,
    seed: int = 0,
    offset: int = 0,
) -> None:
    """Apply the update in place, including state write-back (reference/sgd.py:75-84)."""
    resolved = resolve_formats(_NAMES, formats, state_dtype=state_dtype, rounding=rounding)
    update_in_place(
        sgdm_step_any_hyperparameters_, parameter, gradient, (momentum,), resolved, seed=seed, offset=offset,
        lr=lr, momentum_factor=momentum_factor,
    )
