"""Casting names of the reference's functional package (sr_states/reference/rounding.py:1-14).

``bf16_neighbors`` and ``minifloat_neighbors`` return, for each FP32 input,
the two values of the target format that stochastic rounding chooses
between, as the reference's checking helpers do (sr_states/_bf16.py:77-101,
sr_states/_minifloat.py:73-99); the HIP neighbour kernel computes them.
"""

import torch

from ..hip.cast import native_neighbors
from ..rounding import cast

__all__ = ["bf16_neighbors", "cast", "minifloat_neighbors", "stochastic_round_bf16"]

_MINIFLOAT_DTYPES = (torch.float8_e4m3fn, torch.float8_e5m2, torch.float16)


def stochastic_round_bf16(x, *, seed, offset=0):
    """``cast(x, dtype=torch.bfloat16, rounding="stochastic", ...)`` on the GPU."""
    return cast(x, dtype=torch.bfloat16, rounding="stochastic", seed=seed, offset=offset)


def _fp32(x):
    if x.dtype != torch.float32:
        raise TypeError(f"expected torch.float32 input, got {x.dtype}")
    return x.contiguous()


def bf16_neighbors(x):
    """Ordered BF16 neighbours (lower, upper) bracketing each FP32 input.

    A value BF16 represents gives itself twice; NaN and infinities give
    their ordinary BF16 conversion twice.
    """
    return native_neighbors(_fp32(x), torch.bfloat16)


def minifloat_neighbors(x, *, dtype):
    """Ordered E4M3, E5M2 or FP16 neighbours (lower, upper) after the format's saturation policy.

    Values on the format's grid give themselves twice.  E4M3 and E5M2 clamp
    magnitudes (infinities included) to their maximum; FP16 brackets finite
    magnitudes above its maximum by the maximum and infinity.  NaN gives NaN.
    """
    x = _fp32(x)
    if dtype not in _MINIFLOAT_DTYPES:
        raise ValueError("neighbors supports E4M3, E5M2, and FP16")
    return native_neighbors(x, dtype)
