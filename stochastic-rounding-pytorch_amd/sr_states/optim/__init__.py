"""Optimizer frame and hyperparameter validation shared by the HIP optimizers."""

from ._state import StateOptimizer
from .adamw import adamw_hparams, validate_adamw
from .sgd import sgdm_hparams, validate_sgdm

__all__ = ["StateOptimizer", "adamw_hparams", "sgdm_hparams", "validate_adamw", "validate_sgdm"]
