"""Device checks for the HIP backend (the gfx950 analogue of triton/_common.py)."""

from __future__ import annotations

from functools import cache

import torch

from .. import _lib

SUPPORTED_ARCH = "gfx950"


def is_hip_available() -> bool:
    """Whether a GPU is visible and the HIP library is built."""
    return torch.cuda.is_available() and _lib.LIBRARY_PATH.exists()


@cache
def _device_arch(device: torch.device) -> str:
    """The device's architecture without its feature suffixes (gfx950 of gfx950:sramecc+:xnack-)."""
    return torch.cuda.get_device_properties(device).gcnArchName.split(":")[0]


def validate_device(device: torch.device) -> None:
    """Reject tensors the gfx950 library cannot run on, before any launch."""
    if not isinstance(device, torch.device):
        device = torch.device(device)
    if device.type != "cuda":
        raise ValueError("fused state updates require GPU tensors")
    arch = _device_arch(device)
    if arch != SUPPORTED_ARCH:
        raise ValueError(f"the sr_states HIP library is built for {SUPPORTED_ARCH}, not {arch}")


def validate_update_device(device, *dtypes) -> None:
    """Device check for an optimizer bucket; every storage dtype runs on gfx950."""
    validate_device(device)
