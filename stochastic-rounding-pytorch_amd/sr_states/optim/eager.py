"""Per-parameter optimizers under the reference's eager names.

``AdamWReferenceSR``/``AdamWReferenceRN`` (sr_states/optim/adamw.py:21-79)
and ``SGDMReferenceSR``/``SGDMReferenceRN`` (sr_states/optim/sgd.py:19-69)
take the reference's arguments, group keys and checkpoint layout and update
one parameter at a time through the functional ``adamw_step_``/``sgdm_step_``,
so each parameter costs one HIP launch.  Their bytes equal those of the fused
multi-tensor ``AdamWHip``/``SGDMHip``, which update a whole group per launch.
Unlike the fused optimizers they accept rounding rules registered with
``register_rounding``: the moments are then updated in FP32 and stored
through the registered routine.
"""

from __future__ import annotations

from ..reference.adamw import adamw_step_
from ..reference.sgd import sgdm_step_
from ._state import StateOptimizer
from .adamw import validate_adamw
from .sgd import validate_sgdm


class AdamWReferenceSR(StateOptimizer):
    """AdamW with FP32 arithmetic and a configurable format for each moment."""

    _state_names = ("exp_avg", "exp_avg_sq")
    _uses_step = True
    _update = staticmethod(adamw_step_.__wrapped__)

    def __init__(
        self,
        params,
        lr=1e-3,
        betas=(0.9, 0.999),
        eps=1e-8,
        weight_decay=1e-2,
        *,
        state_format=None,
        state_dtype=None,
        rounding=None,
        seed=0,
    ):
        super().__init__(
            params,
            {"lr": lr, "betas": betas, "eps": eps, "weight_decay": weight_decay},
            state_format=state_format,
            state_dtype=state_dtype,
            rounding=rounding,
            seed=seed,
        )

    def _validate_group(self, group):
        validate_adamw(group)

    def _step_parameter(self, parameter, state, group, formats, step, seed, offset):
        local_p, local_g, exp_avg, exp_avg_sq = self._local_tensors(parameter, state)
        beta1, beta2 = group["betas"]
        self._update(
            local_p,
            local_g,
            exp_avg,
            exp_avg_sq,
            lr=group["lr"],
            beta1=beta1,
            beta2=beta2,
            eps=group["eps"],
            weight_decay=group["weight_decay"],
            step=step,
            formats=formats,
            seed=seed,
            offset=offset,
        )


class AdamWReferenceRN(AdamWReferenceSR):
    """Round-to-nearest AdamW (BF16 by default); the formats choose only dtypes."""

    _forced_rounding = "nearest"


class SGDMReferenceSR(StateOptimizer):
    """Momentum SGD with FP32 arithmetic; BF16 stochastic storage by default."""

    _state_names = ("momentum_buffer",)
    _uses_step = False
    _update = staticmethod(sgdm_step_.__wrapped__)

    def __init__(
        self,
        params,
        lr,
        momentum=0.9,
        *,
        state_format=None,
        state_dtype=None,
        rounding=None,
        seed=0,
    ):
        super().__init__(
            params,
            {"lr": lr, "momentum": momentum},
            state_format=state_format,
            state_dtype=state_dtype,
            rounding=rounding,
            seed=seed,
        )

    def _validate_group(self, group):
        validate_sgdm(group)

    def _step_parameter(self, parameter, state, group, formats, step, seed, offset):
        local_p, local_g, momentum = self._local_tensors(parameter, state)
        self._update(
            local_p,
            local_g,
            momentum,
            lr=group["lr"],
            momentum_factor=group["momentum"],
            formats=formats,
            seed=seed,
            offset=offset,
        )


class SGDMReferenceRN(SGDMReferenceSR):
    """Round-to-nearest momentum SGD (BF16 by default); the formats choose only dtypes."""

    _forced_rounding = "nearest"
