"""Fused gfx950 (MI355X) kernels: the HIP counterpart of ``sr_states.triton``."""

from ._common import is_hip_available
from .adamw import AdamWHip, AdamWHipRN, hip_adamw_step_
from .cast import cast, rn_cast_bf16, sr_cast_bf16
from .sgd import SGDMHip, SGDMHipRN, hip_sgdm_step_

__all__ = [
    "AdamWHip",
    "AdamWHipRN",
    "SGDMHip",
    "SGDMHipRN",
    "cast",
    "hip_adamw_step_",
    "hip_sgdm_step_",
    "is_hip_available",
    "rn_cast_bf16",
    "sr_cast_bf16",
]
