"""Functional updates and casts under the names of the reference's ``sr_states.reference``.

``adamw_step``/``adamw_step_`` and ``sgdm_step``/``sgdm_step_`` keep the
reference's signatures and results and run the fused HIP kernels;
``stochastic_round_bf16`` and ``cast`` run the HIP cast, and
``bf16_neighbors``/``minifloat_neighbors`` the HIP neighbour kernel.
Everything here takes GPU tensors.
"""

from ..rounding import cast
from .adamw import adamw_step, adamw_step_
from .rounding import bf16_neighbors, minifloat_neighbors, stochastic_round_bf16
from .sgd import sgdm_step, sgdm_step_

__all__ = [
    "adamw_step",
    "adamw_step_",
    "bf16_neighbors",
    "cast",
    "minifloat_neighbors",
    "sgdm_step",
    "sgdm_step_",
    "stochastic_round_bf16",
]
