"""Fused momentum SGD on gfx950 with configurable momentum storage.

Drop-in for sr_states/triton/sgd.py: ``SGDMHip`` takes the arguments of
``SGDMTriton``; ``hip_sgdm_step_`` is the single-tensor functional update.
"""

from __future__ import annotations

import ctypes

import torch

from .. import _lib
from ..optim._state import StateOptimizer
from ..optim.sgd import sgdm_hparams, sgdm_scalars, validate_sgdm
from ..rounding import native_codes
from ._common import validate_device, validate_update_device
from ._multi_tensor import prepare_group
from ._optimizer import (
    DEFAULT_BLOCK_SIZE,
    nonnegative,
    reject_dtensors,
    resolve_native_codes,
    validate_options,
)

_STATE_NAMES = ("momentum_buffer",)


def _launch(tables, dtypes, hparams, seed, rng_step, block_size, stream):
    """One sr_sgdm_multi call; dtypes = (p, g, u, u_rule) codes."""
    _lib.call(
        "sr_sgdm_multi",
        tables.device_records.data_ptr(),
        tables.device_tile_rows.data_ptr(),
        tables.nrows,
        tables.total_tiles,
        *dtypes,
        ctypes.byref(hparams),
        seed,
        rng_step,
        block_size,
        stream,
    )


@torch.no_grad()
def hip_sgdm_step_(
    parameter: torch.Tensor,
    gradient: torch.Tensor,
    momentum: torch.Tensor,
    *,
    lr: float,
    momentum_factor: float,
    seed: int,
    offset: int = 0,
    rounding: str | None = None,
    formats: tuple | dict | None = None,
    block_size: int = DEFAULT_BLOCK_SIZE,
) -> None:
    """Apply one fused momentum-SGD update in place (triton/sgd.py:115-171).

    ``parameter``, ``gradient`` and ``momentum`` are same-shaped contiguous
    GPU tensors; parameter and gradient are FP32 or BF16 and the momentum uses
    any built-in storage format.  ``seed`` is the update key and ``offset``
    the flat index of the first element.
    """
    codes = resolve_native_codes(_STATE_NAMES, (momentum,), formats, rounding, block_size)
    nonnegative("learning rate", lr)
    if not 0 <= momentum_factor < 1:
        raise ValueError(f"invalid momentum value: {momentum_factor}")
    _launch_step(parameter, gradient, momentum, codes, sgdm_scalars(lr, momentum_factor), seed, offset, block_size)


def sgdm_step_any_hyperparameters_(parameter, gradient, momentum, *, lr, momentum_factor, seed=0, offset=0,
                                   formats=None):
    """``hip_sgdm_step_`` for the reference's functional updates, which check no hyperparameter.

    sr_states/reference/sgd.py:44-72 computes with any learning rate and
    momentum factor; so does this.  Its callers run under no_grad; the
    launch itself records nothing for autograd.
    """
    codes = resolve_native_codes(_STATE_NAMES, (momentum,), formats, None, DEFAULT_BLOCK_SIZE)
    _launch_step(parameter, gradient, momentum, codes, sgdm_scalars(lr, momentum_factor), seed, offset,
                 DEFAULT_BLOCK_SIZE)


def _launch_step(parameter, gradient, momentum, codes, scalars, seed, offset, block_size):
    ((code, rule),) = codes
    reject_dtensors(parameter, gradient, momentum)
    device = parameter.device
    if device.type != "cuda":
        raise ValueError("fused state updates require GPU tensors")
    validate_device(device)
    # The native entry checks devices, shapes, layout, dtypes and overlap with
    # the messages of sr_states/triton/_optimizer.py:24-60, then launches.
    status = _lib.launcher().sgdm_step(
        parameter, gradient, momentum, code, rule, scalars, _lib.low32(seed), _lib.low32(offset), block_size,
        _lib.stream_handle(device),
    )
    _lib.check("sr_sgdm_step", status)


class SGDMHip(StateOptimizer):
    """Fused momentum SGD; BF16 stochastic momentum storage by default.

    Same arguments, group keys and checkpoint layout as ``SGDMTriton``
    (triton/sgd.py:174-237).  There is no Nesterov, dampening or weight decay
    option, as in the reference.
    """

    _state_names = _STATE_NAMES
    _uses_step = False
    _rounding_backend = "hip"

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
        block_size=DEFAULT_BLOCK_SIZE,
    ):
        super().__init__(
            params,
            {"lr": lr, "momentum": momentum, "block_size": block_size},
            state_format=state_format,
            state_dtype=state_dtype,
            rounding=rounding,
            seed=seed,
        )

    def _group_block_size(self, group):
        return group.get("block_size", self.defaults["block_size"])

    def _validate_group(self, group):
        validate_sgdm(group)
        validate_options("nearest", self._group_block_size(group), torch.float32)

    def _step_parameter(self, parameter, state, group, formats, step, seed, offset):
        hip_sgdm_step_(
            *self._local_tensors(parameter, state),
            lr=group["lr"],
            momentum_factor=group["momentum"],
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
        code, rule = native_codes(formats[0].dtype, formats[0].rounding)
        hparams = sgdm_hparams(group["lr"], group["momentum"])
        seed, rng_word = _lib.low64(group["sr_seed"]), _lib.low64(rng_step)
        block_size = self._group_block_size(group)
        for launch in launches:
            with _lib.on_device(launch.device):
                _launch(
                    launch.tables,
                    (*launch.codes, code, rule),
                    hparams,
                    seed,
                    rng_word,
                    block_size,
                    _lib.stream_handle(launch.device),
                )
        record_steps()


class SGDMHipRN(SGDMHip):
    """Fused momentum SGD whose momentum always uses round-to-nearest storage."""

    _forced_rounding = "nearest"
