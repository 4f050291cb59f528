"""Optimizers under the reference's eager names: fused groups, or one parameter at a time.

``AdamWReferenceSR``/``AdamWReferenceRN`` (sr_states/optim/adamw.py:21-79)
and ``SGDMReferenceSR``/``SGDMReferenceRN`` (sr_states/optim/sgd.py:19-69)
take the reference's arguments, group keys and checkpoint layout.  The
reference updates one parameter at a time through the functional
``adamw_step_``/``sgdm_step_``; its bytes equal those of the fused
multi-tensor ``AdamWHip``/``SGDMHip``, which update a whole group per launch.
So a group runs as one fused launch per bucket whenever the fused launch
takes it as it is, and one parameter at a time through the functional
updates otherwise:

- a state format without a HIP implementation (a rule registered with
  ``register_rounding``: the moments are then updated in FP32 and stored
  through the registered routine);
- hyperparameters outside the fused optimizers' ranges (the reference's
  eager updates compute with any);
- a parameter, gradient or state the fused launch refuses (another dtype
  than FP32/BF16, a strided layout, storage shared between parameters,
  whose updates the reference applies in order);
- a stream under HIP graph capture;
- a parameter the reference's walk raises at (a sparse gradient, a DTensor
  placement without a flat shard start, more than 2**32 elements).

The fused launch validates the whole group before it queues anything, so
a refused group is updated per parameter from the start.  For the last
kind, that walk updates every parameter ahead of the bad one and records
its step before it raises the same error at the same parameter, as the
reference's lazy loop does (sr_states/optim/_state.py:154-182).
"""

from __future__ import annotations

import torch

from ..hip._common import validate_update_device
from ..hip._multi_tensor import prepare_group
from ..hip._optimizer import DEFAULT_BLOCK_SIZE
from ..hip.adamw import AdamWHip
from ..hip.sgd import SGDMHip
from ..reference.adamw import adamw_step_
from ..reference.sgd import sgdm_step_
from ..rounding import has_native
from ._state import StateOptimizer
from .adamw import validate_adamw
from .sgd import validate_sgdm


class _FusedGroups(StateOptimizer):
    """Groups the fused multi-tensor launch takes as they are run on it; others per parameter."""

    # Cleared on an instance, every group runs per parameter (the tests
    # compare the two routes).
    _fused_route = True

    def _group_block_size(self, group):
        return DEFAULT_BLOCK_SIZE

    def _step_group(self, group, formats, items, rng_step):
        prepared = self._fused_prepare(group, formats, items)
        if prepared is not None:
            self._launch_prepared(group, formats, prepared, rng_step)
            return
        first_index = 0
        for other in self.param_groups:
            if other is group:
                break
            first_index += len(other["params"])
        # A fresh walk: the fused preparation may have consumed `items`.
        super()._step_group(group, formats, self._group_items(group, formats, first_index), rng_step)

    def _fused_prepare(self, group, formats, items):
        """The fused launches of the group, or None to update it per parameter."""
        if not self._fused_route or not all(has_native(f.dtype, f.rounding) for f in formats):
            return None
        if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
            return None
        try:
            self._validate_group(group)
            # Validates every parameter, gradient and state of the group, and
            # their disjointness, before anything is queued.
            return prepare_group(self, group, formats, items, validate_update_device)
        except (ValueError, TypeError, RuntimeError):
            # RuntimeError covers the walk's sparse-gradient refusal and
            # NotImplementedError (unsupported DTensor placements): the
            # per-parameter route updates the parameters ahead of the bad one
            # before raising it again.
            return None


class AdamWReferenceSR(_FusedGroups):
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

    _launch_prepared = AdamWHip._launch_prepared

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


class SGDMReferenceSR(_FusedGroups):
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

    _launch_prepared = SGDMHip._launch_prepared

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
