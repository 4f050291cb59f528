"""Fused AdamW on gfx950 with FP32 arithmetic and per-moment storage formats.

Drop-in for sr_states/triton/adamw.py: ``AdamWHip`` takes the arguments of
``AdamWTriton`` and launches one fused multi-tensor kernel per bucket;
``hip_adamw_step_`` is the single-tensor functional update.
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from .. import _lib
from ..optim._state import StateOptimizer
from ..optim.adamw import adamw_hparams, adamw_scalars, validate_adamw
from ..rounding import native_codes
from ._common import validate_device, validate_update_device
from ._multi_tensor import prepare_group, upload
from ._optimizer import (
    DEFAULT_BLOCK_SIZE,
    nonnegative,
    reject_dtensors,
    resolve_native_codes,
    validate_options,
)

_STATE_NAMES = ("exp_avg", "exp_avg_sq")


def _launch(tables, dtypes, hparams, seed, rng_step, block_size, stream, row_scalars=None):
    """One sr_adamw_multi call; dtypes = (p, g, m, m_rule, v, v_rule) codes.

    ``row_scalars`` is None when every row shares ``hparams``, else a device
    tensor of per-row (neg_step_size, correction2_sqrt) FP32 pairs.
    """
    _lib.call(
        "sr_adamw_multi",
        tables.device_records.data_ptr(),
        tables.device_tile_rows.data_ptr(),
        None if row_scalars is None else row_scalars.data_ptr(),
        tables.nrows,
        tables.total_tiles,
        *dtypes,
        ctypes.byref(hparams),
        seed,
        rng_step,
        block_size,
        stream,
    )


def _validate_hyperparameters(lr, betas, eps, weight_decay):
    nonnegative("learning rate", lr)
    nonnegative("epsilon", eps)
    nonnegative("weight_decay", weight_decay)
    if len(betas) != 2 or any(not 0 <= beta < 1 for beta in betas):
        raise ValueError(f"invalid beta values: {betas}")


@torch.no_grad()
def hip_adamw_step_(
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
    seed: int = 0,
    offset: int = 0,
    rounding: str | None = None,
    formats: tuple | dict | None = None,
    block_size: int = DEFAULT_BLOCK_SIZE,
) -> None:
    """Update parameter and moments in place (triton/adamw.py:160-221).

    Inputs are contiguous, disjoint GPU tensors of one shape; parameter and
    gradient are FP32 or BF16; each moment uses its own storage format.  The
    parameter update uses the unrounded FP32 moments.  ``step`` starts at one;
    ``seed`` is the update key and ``offset`` the flat index of the first
    element.
    """
    codes = resolve_native_codes(_STATE_NAMES, (exp_avg, exp_avg_sq), formats, rounding, block_size)
    _validate_hyperparameters(lr, (beta1, beta2), eps, weight_decay)
    _launch_step(parameter, gradient, exp_avg, exp_avg_sq, codes,
                 adamw_scalars(lr, beta1, beta2, eps, weight_decay, _positive_step(step)), seed, offset, block_size)


def adamw_step_any_hyperparameters_(
    parameter, gradient, exp_avg, exp_avg_sq, *, lr, beta1, beta2, eps, weight_decay, step, seed=0, offset=0,
    formats=None,
):
    """``hip_adamw_step_`` for the reference's functional updates, which check no hyperparameter.

    sr_states/reference/adamw.py:54-105 computes with any learning rate,
    epsilon, weight decay and betas; so does this.  The one limit is the
    launch's: the division by sqrt(1 - beta2^step) is exact for constants
    in [2^-27, 1], which every beta2 in [0, 1) gives, and the library
    refuses others with an error.  beta1 = 1 divides by zero here as in the
    reference.  ``step`` may be any real number of at least 1, which the
    reference's bias corrections take (its callers check it).  Its callers
    run under no_grad; the launch itself records nothing for autograd.
    """
    codes = resolve_native_codes(_STATE_NAMES, (exp_avg, exp_avg_sq), formats, None, DEFAULT_BLOCK_SIZE)
    scalars = adamw_scalars(lr, beta1, beta2, eps, weight_decay, step)
    correction = scalars[5]  # sqrt(1 - beta2**step): complex when beta2**step > 1
    if isinstance(correction, complex) or not 0 < correction <= 1:
        raise ValueError(
            f"sqrt(1 - beta2**step) must lie in (0, 1] for the fused update; got beta2={beta2}, step={step}"
        )
    _launch_step(parameter, gradient, exp_avg, exp_avg_sq, codes, scalars, seed, offset, DEFAULT_BLOCK_SIZE)


def _positive_step(step):
    if not isinstance(step, int) or isinstance(step, bool) or step < 1:
        raise ValueError("step must be a positive integer")
    return step


def _launch_step(parameter, gradient, exp_avg, exp_avg_sq, codes, scalars, seed, offset, block_size):
    (m_code, m_rule), (v_code, v_rule) = codes
    reject_dtensors(parameter, gradient, exp_avg, exp_avg_sq)
    device = parameter.device
    if device.type != "cuda":
        raise ValueError("fused state updates require GPU tensors")
    validate_device(device)
    # The native entry checks devices, shapes, layout, dtypes and overlap with
    # the messages of sr_states/triton/_optimizer.py:24-60, then launches.
    status = _lib.launcher().adamw_step(
        parameter, gradient, exp_avg, exp_avg_sq, m_code, m_rule, v_code, v_rule, scalars, _lib.low32(seed),
        _lib.low32(offset), block_size, _lib.stream_handle(device),
    )
    _lib.check("sr_adamw_step", status)


class AdamWHip(StateOptimizer):
    """Fused AdamW with FP32 arithmetic and independently stored moments.

    Same arguments, group keys and checkpoint layout as ``AdamWTriton``
    (triton/adamw.py:245-319).  ``block_size`` is the workgroup size in
    threads; results do not depend on it.
    """

    _state_names = _STATE_NAMES
    _uses_step = True
    _rounding_backend = "hip"

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
        block_size=DEFAULT_BLOCK_SIZE,
    ):
        super().__init__(
            params,
            {
                "lr": lr,
                "betas": betas,
                "eps": eps,
                "weight_decay": weight_decay,
                "block_size": block_size,
            },
            state_format=state_format,
            state_dtype=state_dtype,
            rounding=rounding,
            seed=seed,
        )

    def _group_block_size(self, group):
        return group.get("block_size", self.defaults["block_size"])

    def _validate_group(self, group):
        validate_adamw(group)
        validate_options("nearest", self._group_block_size(group), torch.float32)

    def _step_parameter(self, parameter, state, group, formats, step, seed, offset):
        beta1, beta2 = group["betas"]
        hip_adamw_step_(
            *self._local_tensors(parameter, state),
            lr=group["lr"],
            beta1=beta1,
            beta2=beta2,
            eps=group["eps"],
            weight_decay=group["weight_decay"],
            step=step,
            seed=seed,
            offset=offset,
            formats=formats,
            block_size=self._group_block_size(group),
        )

    def _step_group(self, group, formats, items, rng_step):
        self._launch_prepared(
            group, formats, prepare_group(self, group, formats, items, validate_update_device), rng_step
        )

    def _launch_prepared(self, group, formats, prepared, rng_step):
        """Queue the launches ``prepare_group`` returned, then record the steps."""
        launches, record_steps = prepared
        beta1, beta2 = group["betas"]
        (m_code, m_rule), (v_code, v_rule) = (native_codes(f.dtype, f.rounding) for f in formats)
        seed, rng_word = _lib.low64(group["sr_seed"]), _lib.low64(rng_step)
        block_size = self._group_block_size(group)

        def hparams(step):
            return adamw_hparams(
                group["lr"], beta1, beta2, group["eps"], group["weight_decay"], step
            )

        for launch in launches:
            dtypes = (*launch.codes, m_code, m_rule, v_code, v_rule)
            with _lib.on_device(launch.device):
                if isinstance(launch.steps, int):
                    scalars, row_scalars = hparams(launch.steps), None
                else:
                    # Rows at different steps: each row's bias-correction pair.
                    per_step = {step: hparams(step) for step in set(launch.steps)}
                    pairs = np.array(
                        [(per_step[s].neg_step_size, per_step[s].correction2_sqrt) for s in launch.steps],
                        dtype=np.float32,
                    )
                    scalars, row_scalars = per_step[launch.steps[0]], upload(pairs, launch.device)
                stream = _lib.stream_handle(launch.device)
                _launch(launch.tables, dtypes, scalars, seed, rng_word, block_size, stream, row_scalars)
        record_steps()


class AdamWHipRN(AdamWHip):
    """Fused AdamW whose states always use round-to-nearest storage."""

    _forced_rounding = "nearest"
