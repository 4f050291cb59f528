"""SR-States for MI355X: stochastic-rounding optimizer states on gfx950.

The public surface follows the reference package ``sr_states``:
``StateFormat``, ``StateOptimizer``, ``cast``, ``register_rounding`` and the
optimizers ``AdamWReferenceSR/RN`` and ``SGDMReferenceSR/RN`` (the fused
launch for the groups it takes, one parameter at a time otherwise) at the
top level, the functional updates in ``sr_states.reference``, and the
fused multi-tensor optimizers and casts in ``sr_states.hip`` (the
counterpart of ``sr_states.triton``).  All arithmetic runs in the HIP
library ``libsr_states_hip.so``; there is no CPU execution path.
"""

from ._hash import state_key, update_key
from .formats import StateFormat
from .hip import (
    AdamWHip,
    AdamWHipRN,
    SGDMHip,
    SGDMHipRN,
    hip_adamw_step_,
    hip_sgdm_step_,
    is_hip_available,
    rn_cast_bf16,
    sr_cast_bf16,
)
from .optim._state import StateOptimizer
from .optim.eager import AdamWReferenceRN, AdamWReferenceSR, SGDMReferenceRN, SGDMReferenceSR
from .rounding import cast, register_rounding

__all__ = [
    "AdamWHip",
    "AdamWHipRN",
    "AdamWReferenceRN",
    "AdamWReferenceSR",
    "SGDMHip",
    "SGDMHipRN",
    "SGDMReferenceRN",
    "SGDMReferenceSR",
    "StateFormat",
    "StateOptimizer",
    "cast",
    "hip_adamw_step_",
    "hip_sgdm_step_",
    "is_hip_available",
    "register_rounding",
    "rn_cast_bf16",
    "sr_cast_bf16",
    "state_key",
    "update_key",
]

__version__ = "0.1.0"
