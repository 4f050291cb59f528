"""ctypes binding of liboracle.so, the plain-C checker (oracle/sr_oracle.c).

TEST INFRASTRUCTURE: imported only by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg.  Arrays are torch CPU tensors; storage dtypes
use the product's codes (0 FP32, 1 BF16, 2 FP16, 3 E4M3, 4 E5M2).
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent
LIBRARY = HERE / "liboracle.so"

CODES = {
    torch.float32: 0,
    torch.bfloat16: 1,
    torch.float16: 2,
    torch.float8_e4m3fn: 3,
    torch.float8_e5m2: 4,
}
RULES = {"nearest": 0, "stochastic": 1}

_lib = None


def build(force: bool = False) -> Path:
    """Compile liboracle.so with the committed Makefile recipe."""
    if force or not LIBRARY.exists() or LIBRARY.stat().st_mtime < (HERE / "sr_oracle.c").stat().st_mtime:
        subprocess.run(["make", "-B", "-C", str(HERE), "liboracle.so"], check=True, capture_output=True)
    return LIBRARY


def lib():
    global _lib
    if _lib is None:
        build()
        handle = ctypes.CDLL(str(LIBRARY))
        vp, i64, u32, u64, c_int, c_float = (
            ctypes.c_void_p, ctypes.c_int64, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int,
            ctypes.c_float,
        )
        handle.oc_hash.restype = u32
        handle.oc_hash.argtypes = [u32]
        handle.oc_update_key.restype = u32
        handle.oc_update_key.argtypes = [u64, u64, u32]
        handle.oc_state_key.restype = u32
        handle.oc_state_key.argtypes = [u32, u32]
        handle.oc_encode.restype = u32
        handle.oc_encode.argtypes = [c_float, c_int, c_int, u32]
        handle.oc_decode.restype = c_float
        handle.oc_decode.argtypes = [u32, c_int]
        handle.oc_cast.restype = None
        handle.oc_cast.argtypes = [vp, vp, i64, c_int, c_int, u32, u32]
        handle.oc_adamw.restype = None
        handle.oc_adamw.argtypes = [vp, c_int, vp, c_int, vp, c_int, c_int, vp, c_int, c_int, i64,
                                    vp, u32, u32]
        handle.oc_sgdm.restype = None
        handle.oc_sgdm.argtypes = [vp, c_int, vp, c_int, vp, c_int, c_int, i64, c_float, c_float,
                                   u32, u32]
        _lib = handle
    return _lib


def _cpu(t: torch.Tensor) -> torch.Tensor:
    if t.device.type != "cpu" or not t.is_contiguous():
        raise ValueError("the C oracle takes contiguous CPU tensors")
    return t


def cast(x: torch.Tensor, *, dtype, rounding="stochastic", seed=0, offset=0) -> torch.Tensor:
    """C restatement of sr_states.cast (counter = i + seed + offset)."""
    x = _cpu(x.contiguous())
    if x.dtype != torch.float32:
        raise TypeError("expected torch.float32 input")
    y = torch.empty(x.shape, dtype=dtype)
    lib().oc_cast(x.data_ptr(), y.data_ptr(), x.numel(), CODES[dtype], RULES[rounding],
                  int(seed) & 0xFFFFFFFF, int(offset) & 0xFFFFFFFF)
    return y


def adamw_hparams(lr, beta1, beta2, eps, weight_decay, step) -> torch.Tensor:
    """The eight FP32 launch scalars, rounded from Python doubles."""
    return torch.tensor(
        [beta1, beta2, 1.0 - beta1, 1.0 - beta2, -lr / (1.0 - beta1**step),
         (1.0 - beta2**step) ** 0.5, 1.0 - lr * weight_decay, eps],
        dtype=torch.float32,
    )


def adamw_step_(p, g, m, v, *, lr, beta1, beta2, eps, weight_decay, step, formats, seed, offset=0):
    """In-place C AdamW; ``formats`` = ((m_dtype, m_rule), (v_dtype, v_rule))."""
    for t in (p, g, m, v):
        _cpu(t)
    hp = adamw_hparams(lr, beta1, beta2, eps, weight_decay, step)
    (m_dtype, m_rule), (v_dtype, v_rule) = formats
    lib().oc_adamw(
        p.data_ptr(), CODES[p.dtype], g.data_ptr(), CODES[g.dtype], m.data_ptr(), CODES[m_dtype],
        RULES[m_rule], v.data_ptr(), CODES[v_dtype], RULES[v_rule], p.numel(), hp.data_ptr(),
        int(seed) & 0xFFFFFFFF, int(offset) & 0xFFFFFFFF,
    )


def sgdm_step_(p, g, u, *, lr, momentum_factor, formats, seed, offset=0):
    """In-place C momentum SGD; ``formats`` = ((u_dtype, u_rule),)."""
    for t in (p, g, u):
        _cpu(t)
    ((u_dtype, u_rule),) = formats
    lib().oc_sgdm(
        p.data_ptr(), CODES[p.dtype], g.data_ptr(), CODES[g.dtype], u.data_ptr(), CODES[u_dtype],
        RULES[u_rule], p.numel(), float(momentum_factor), float(-lr), int(seed) & 0xFFFFFFFF,
        int(offset) & 0xFFFFFFFF,
    )
