"""Casting names of the reference's functional package (sr_states/reference/rounding.py:1-14)."""

import torch

from ..rounding import cast

__all__ = ["cast", "stochastic_round_bf16"]


def stochastic_round_bf16(x, *, seed, offset=0):
    """``cast(x, dtype=torch.bfloat16, rounding="stochastic", ...)`` on the GPU."""
    return cast(x, dtype=torch.bfloat16, rounding="stochastic", seed=seed, offset=offset)
