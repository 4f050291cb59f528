"""CPU restatement of the reference's eager algorithm, used as a CHECKER ONLY.

TEST INFRASTRUCTURE.  Only tests/, ``__graft_entry__.smoke()`` and
``bench.py``'s cpu_baseline leg may import this module; the product package
never does.

It restates the reference's eager PyTorch path with the same torch CPU
operations in the same order, so that it reproduces that path's FP32
results on this machine (including torch's CPU square root), and times like
it.  Each function cites the reference file and lines it follows (paths
relative to the reference repository root).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

MASK32 = 0xFFFFFFFF
_MUL1, _MUL2 = 0x7FEB352D, 0x846CA68B

# ---------------------------------------------------------------------------
# Keys and counter hash (sr_states/_hash.py:5-50)
# ---------------------------------------------------------------------------


def h32(value: int) -> int:
    """sr_states/_hash.py:10-15."""
    value &= MASK32
    value ^= value >> 16
    value = (value * _MUL1) & MASK32
    value ^= value >> 15
    value = (value * _MUL2) & MASK32
    return value ^ (value >> 16)


def update_key(seed: int, step: int, param_index: int) -> int:
    """sr_states/_hash.py:18-23."""
    key = h32((seed & MASK32) ^ 0x9E3779B9)
    for word in (seed >> 32, step, step >> 32, param_index):
        key = h32(key ^ (word & MASK32))
    return key


def state_key(key: int, state_index: int) -> int:
    """sr_states/_hash.py:26-28."""
    return h32((key ^ state_index) & MASK32)


def u32_hash(indices: torch.Tensor, seed: int) -> torch.Tensor:
    """sr_states/_hash.py:31-50: hash of (index + seed) mod 2^32, in int64."""
    value = (indices.to(torch.int64) + (int(seed) % (1 << 32))) & MASK32
    value = value ^ (value >> 16)
    value = (value * _MUL1) & MASK32
    value = value ^ (value >> 15)
    value = (value * _MUL2) & MASK32
    return (value ^ (value >> 16)) & MASK32


def _counters(x: torch.Tensor, offset: int) -> torch.Tensor:
    return torch.arange(x.numel(), dtype=torch.int64) + (int(offset) % (1 << 32))


# ---------------------------------------------------------------------------
# BF16 (sr_states/_bf16.py:37-101)
# ---------------------------------------------------------------------------


def _u32(x: torch.Tensor) -> torch.Tensor:
    return x.contiguous().reshape(-1).view(torch.int32).to(torch.int64) & MASK32


def _from_u32(bits: torch.Tensor, shape) -> torch.Tensor:
    return bits.to(torch.int32).view(torch.float32).reshape(shape)


def stochastic_round_bf16(x: torch.Tensor, *, seed: int, offset: int = 0) -> torch.Tensor:
    """sr_states/_bf16.py:37-74."""
    if x.dtype != torch.float32:
        raise TypeError(f"expected torch.float32 input, got {x.dtype}")
    bits = _u32(x)
    low = u32_hash(_counters(x, offset), seed) & 0xFFFF
    truncated = bits & 0xFFFF0000
    rounded = (bits + low) & 0xFFFF0000
    special = (bits & 0x7F800000) == 0x7F800000
    nan = special & ((bits & 0x007FFFFF) != 0)
    rounded = torch.where(special, torch.where(nan, truncated | 0x00400000, truncated), rounded)
    return _from_u32(rounded, x.shape).to(torch.bfloat16)


def bf16_neighbors(x: torch.Tensor):
    """sr_states/_bf16.py:77-101: ordered BF16 neighbours of finite FP32 input."""
    bits = _u32(x)
    truncated_bits = bits & 0xFFFF0000
    truncated = _from_u32(truncated_bits, x.shape)
    exact_or_special = ((bits & 0xFFFF) == 0) | ((bits & 0x7F800000) == 0x7F800000)
    negative = ((bits & 0x80000000) != 0).reshape(x.shape)
    away = _from_u32((truncated_bits + 0x00010000) & MASK32, x.shape)
    lower = torch.where(negative, away, truncated)
    upper = torch.where(negative, truncated, away)
    converted = x.to(torch.bfloat16).to(torch.float32)
    exact_or_special = exact_or_special.reshape(x.shape)
    lower = torch.where(exact_or_special, converted, lower)
    upper = torch.where(exact_or_special, converted, upper)
    return lower.to(torch.bfloat16), upper.to(torch.bfloat16)


# ---------------------------------------------------------------------------
# Minifloats (sr_states/_minifloat.py:10-99)
# ---------------------------------------------------------------------------

# mantissa bits, minimum normal exponent, max finite, saturating
MINIFLOATS = {
    torch.float8_e4m3fn: (3, -6, 448.0, True),
    torch.float8_e5m2: (2, -14, 57344.0, True),
    torch.float16: (10, -14, 65504.0, False),
}


def _grid(a: torch.Tensor, mantissa: int, emin: int):
    """sr_states/_minifloat.py:17-26: a = (q + remainder) * ulp."""
    exponent = (((a.contiguous().view(torch.int32) >> 23) & 0xFF) - 127).clamp_min(emin)
    ulp = ((exponent - mantissa + 127) << 23).view(torch.float32)
    scale = ((127 - exponent + mantissa) << 23).view(torch.float32)
    scaled = a * scale
    q = torch.floor(scaled)
    return q, scaled - q, ulp


def nearest_minifloat(x, *, dtype, seed=0, offset=0):
    """sr_states/_minifloat.py:29-42."""
    mantissa, emin, maximum, saturate = MINIFLOATS[dtype]
    if not saturate:
        return x.to(dtype)
    a = x.abs().clamp_max(maximum)
    safe = torch.where(torch.isnan(a), torch.zeros_like(a), a)
    q, remainder, ulp = _grid(safe, mantissa, emin)
    up = (remainder > 0.5) | ((remainder == 0.5) & ((q.to(torch.int32) & 1) != 0))
    rounded = torch.copysign((q + up.to(torch.float32)) * ulp, x)
    return torch.where(torch.isnan(x), x, rounded).to(dtype)


def stochastic_minifloat(x, *, dtype, seed, offset=0):
    """sr_states/_minifloat.py:45-70: round up iff (hash >> 8) < floor(r * 2^24)."""
    mantissa, emin, maximum, saturate = MINIFLOATS[dtype]
    a = x.abs()
    if saturate:
        a = a.clamp_max(maximum)
    safe = torch.where(torch.isfinite(a), a, torch.zeros_like(a))
    q, remainder, ulp = _grid(safe, mantissa, emin)
    k = (u32_hash(_counters(x, offset), seed) >> 8).reshape(x.shape)
    threshold = torch.floor(remainder * 16777216.0)
    rounded = torch.copysign((q + (k < threshold).to(torch.float32)) * ulp, x)
    if not saturate:
        rounded = torch.where(torch.isinf(x), x, rounded)
    return torch.where(torch.isnan(x), x, rounded).to(dtype)


def minifloat_neighbors(x: torch.Tensor, *, dtype):
    """sr_states/_minifloat.py:73-99."""
    mantissa, emin, maximum, saturate = MINIFLOATS[dtype]
    a = x.abs().clamp_max(maximum)
    safe = torch.where(torch.isfinite(a), a, torch.zeros_like(a))
    q, remainder, ulp = _grid(safe, mantissa, emin)
    near = q * ulp
    away = (q + (remainder != 0).float()) * ulp
    if not saturate:
        near = torch.where(x.abs() > maximum, maximum, near)
        away = torch.where(x.abs() > maximum, float("inf"), away)
        near = torch.where(torch.isinf(x), float("inf"), near)
    near, away = torch.copysign(near, x), torch.copysign(away, x)
    lower = torch.where(torch.signbit(x), away, near)
    upper = torch.where(torch.signbit(x), near, away)
    lower = torch.where(torch.isnan(x), x, lower)
    upper = torch.where(torch.isnan(x), x, upper)
    return lower.to(dtype), upper.to(dtype)


# ---------------------------------------------------------------------------
# Rule table and cast (sr_states/rounding.py:97-142)
# ---------------------------------------------------------------------------

STATE_DTYPES = (torch.float32, torch.bfloat16, torch.float16, torch.float8_e4m3fn, torch.float8_e5m2)
RULES = ("nearest", "stochastic")


def cast(x: torch.Tensor, *, dtype, rounding="stochastic", seed=0, offset=0) -> torch.Tensor:
    """sr_states/rounding.py:97-142 for the built-in rules."""
    if x.dtype != torch.float32:
        raise TypeError(f"expected torch.float32 input, got {x.dtype}")
    if dtype not in STATE_DTYPES or rounding not in RULES:
        raise ValueError(f"no rounding {rounding!r} registered for state_dtype={dtype}")
    if dtype == torch.float32 or (dtype == torch.bfloat16 and rounding == "nearest"):
        return x.to(dtype)
    if dtype == torch.bfloat16:
        return stochastic_round_bf16(x, seed=seed, offset=offset)
    if rounding == "nearest":
        return nearest_minifloat(x, dtype=dtype, seed=seed, offset=offset)
    return stochastic_minifloat(x, dtype=dtype, seed=seed, offset=offset)


# ---------------------------------------------------------------------------
# Functional recurrences (sr_states/reference/adamw.py:54-105,
# sr_states/reference/sgd.py:44-72)
# ---------------------------------------------------------------------------


@dataclass(frozen=True)
class Fmt:
    """One state's storage dtype and rule (the reference's StateFormat)."""

    dtype: torch.dtype
    rounding: str = "stochastic"


def adamw_step(p, g, m, v, *, lr, beta1, beta2, eps, weight_decay, step, formats, seed, offset=0):
    """sr_states/reference/adamw.py:54-105; ``seed`` is the update key.

    Returns (new parameter in p's dtype, stored exp_avg, stored exp_avg_sq).
    """
    if step < 1:
        raise ValueError("step must be at least 1")
    p32, g32 = p.float(), g.float()
    m32 = m.float().mul(beta1).add(g32, alpha=1.0 - beta1)
    v32 = v.float().mul(beta2).addcmul(g32, g32, value=1.0 - beta2)
    bias_correction1 = 1.0 - beta1**step
    bias_correction2 = 1.0 - beta2**step
    denominator = v32.sqrt().div_(bias_correction2**0.5).add_(eps)
    new_p = p32.mul(1.0 - lr * weight_decay)
    new_p.addcdiv_(m32, denominator, value=-lr / bias_correction1)
    stored = [
        cast(value, dtype=fmt.dtype, rounding=fmt.rounding, seed=state_key(seed, i), offset=offset)
        for i, (value, fmt) in enumerate(zip((m32, v32), formats))
    ]
    return new_p.to(p.dtype), stored[0], stored[1]


def sgdm_step(p, g, u, *, lr, momentum_factor, formats, seed, offset=0):
    """sr_states/reference/sgd.py:44-72; ``seed`` is the update key."""
    p32 = p.float()
    u32 = u.float().mul(momentum_factor).add(g.float())
    new_p = p32.add(u32, alpha=-lr).to(p.dtype)
    fmt = formats[0]
    stored = cast(u32, dtype=fmt.dtype, rounding=fmt.rounding, seed=state_key(seed, 0), offset=offset)
    return new_p, stored


# ---------------------------------------------------------------------------
# Optimizer composition (sr_states/optim/_state.py:154-200, adamw.py, sgd.py)
# ---------------------------------------------------------------------------


class OracleOptimizer:
    """Eager restatement of StateOptimizer.step over plain tensors.

    ``groups`` is a list of dicts with "params" (list of tensors; parameters
    are updated in place), "grads" (same length, None for a parameter
    without gradient), "formats" (tuple of Fmt), "sr_seed", optional
    "sr_step" and "shard_starts", plus the hyperparameters.
    """

    state_names: tuple = ()
    uses_step = True

    def __init__(self, groups):
        self.groups = groups
        for group in groups:
            group.setdefault("sr_step", 0)
        self.state = {}

    def _rng_step(self):
        return max((int(g["sr_step"]) for g in self.groups), default=0)

    @torch.no_grad()
    def step(self):
        rng_step = self._rng_step() + 1
        for group in self.groups:
            group["sr_step"] = rng_step
        first_index = 0
        for group in self.groups:
            shards = group.get("shard_starts") or [0] * len(group["params"])
            for param_index, (p, g, shard) in enumerate(
                zip(group["params"], group["grads"], shards), start=first_index
            ):
                if g is None:
                    continue
                if p.numel() > 1 << 32:
                    raise ValueError("optimizer RNG supports at most 2**32 elements per parameter")
                state = self.state.setdefault(id(p), {})
                for name, fmt in zip(self.state_names, group["formats"]):
                    state.setdefault(name, torch.zeros_like(p, dtype=fmt.dtype))
                next_step = state.get("step", 0) + 1
                key = update_key(group["sr_seed"], rng_step, param_index)
                self._update(p, g, state, group, next_step, key, shard)
                if self.uses_step:
                    state["step"] = next_step
            first_index += len(group["params"])


class AdamWOracle(OracleOptimizer):
    """sr_states/optim/adamw.py:21-79 over the functional recurrence."""

    state_names = ("exp_avg", "exp_avg_sq")
    uses_step = True

    def _update(self, p, g, state, group, step, key, shard):
        beta1, beta2 = group["betas"]
        new_p, m, v = adamw_step(
            p, g, state["exp_avg"], state["exp_avg_sq"], lr=group["lr"], beta1=beta1,
            beta2=beta2, eps=group["eps"], weight_decay=group["weight_decay"], step=step,
            formats=group["formats"], seed=key, offset=shard,
        )
        p.copy_(new_p)
        state["exp_avg"].copy_(m)
        state["exp_avg_sq"].copy_(v)


class SGDMOracle(OracleOptimizer):
    """sr_states/optim/sgd.py:19-69 over the functional recurrence."""

    state_names = ("momentum_buffer",)
    uses_step = False

    def _update(self, p, g, state, group, step, key, shard):
        new_p, u = sgdm_step(
            p, g, state["momentum_buffer"], lr=group["lr"], momentum_factor=group["momentum"],
            formats=group["formats"], seed=key, offset=shard,
        )
        p.copy_(new_p)
        state["momentum_buffer"].copy_(u)
