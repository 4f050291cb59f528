"""Optimizer RNG keys (sr_states/_hash.py:18-28 of the reference).

The derivation runs in the HIP library's host code, the same source the
kernels use on the device, so host-side keys and device-side keys cannot
drift apart.
"""

from __future__ import annotations

from ._lib import library, low32, low64


def update_key(seed: int, step: int, param_index: int) -> int:
    """32-bit key of one parameter update from the low 64 bits of seed and step."""
    return int(library().sr_update_key(low64(seed), low64(step), low32(param_index)))


def state_key(key: int, state_index: int) -> int:
    """Counter base of one optimizer state derived from an update key."""
    return int(library().sr_state_key(low32(key), low32(state_index)))
