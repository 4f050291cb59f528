"""The fused updates on values across the whole FP32 range, against the C oracle bit for bit.

The other parity tests draw parameters, gradients and moments from the
ranges the reference's benchmarks use.  Here every operand spans the FP32
exponent range: zeros of both signs, subnormals, values near the largest
finite one, infinities and NaN.  That drives every branch of the device
arithmetic through the kernels themselves, in the vector path and the
scalar tail:

- the square root's library fallback for nonzero second moments below
  2^-96, and the division by sqrt(1 - beta2^t) on dividends from 2^-75 to
  2^64;
- the minifloat encoders' tiny-value branch (results below the smallest
  subnormal) and their saturation and NaN handling;
- the BF16 nearest convert's NaN mapping.

The C oracle (oracle/sr_oracle.c) computes every operation with the C
library's correctly rounded arithmetic and the integer encoders.  NaN
payloads are not compared.
"""

from __future__ import annotations

import pytest
import torch
from conftest import assert_bits_or_nan

from oracle import c_oracle

pytestmark = pytest.mark.gpu

N = 8 * 256 * 3 + 5  # whole vector tiles and a scalar tail
ADAMW = {"lr": 1e-3, "beta1": 0.9, "beta2": 0.999, "eps": 1e-8, "weight_decay": 1e-2, "step": 7}
SGDM = {"lr": 1e-3, "momentum_factor": 0.9}
FORMATS = [
    ((torch.float32, "nearest"), (torch.float32, "nearest")),
    ((torch.bfloat16, "stochastic"), (torch.bfloat16, "stochastic")),
    ((torch.bfloat16, "nearest"), (torch.bfloat16, "nearest")),
    ((torch.float16, "stochastic"), (torch.float16, "stochastic")),
    ((torch.float16, "nearest"), (torch.float32, "nearest")),
    ((torch.float8_e4m3fn, "stochastic"), (torch.bfloat16, "stochastic")),
    ((torch.float8_e5m2, "stochastic"), (torch.float8_e4m3fn, "nearest")),
]


def _wide(gen, n, low, high, *, signed=True):
    """Values 2^U(low, high) with random signs, and every 97th one special."""
    exponent = torch.randint(low, high, (n,), generator=gen).double()
    mantissa = 1 + torch.rand(n, generator=gen, dtype=torch.float64)
    values = mantissa * torch.pow(2.0, exponent)
    if signed:
        values = torch.where(torch.rand(n, generator=gen) < 0.5, -values, values)
    values = values.float()
    specials = torch.tensor([0.0, -0.0, 2.0**-149, 2.0**-130, 3.0e38, float("inf"), -float("inf"),
                             float("nan")])
    if not signed:
        specials = specials.abs()
    values[::97] = specials[torch.arange(len(values[::97])) % len(specials)]
    return values


def _inputs(kind, p_dtype, g_dtype, formats, seed):
    gen = torch.Generator().manual_seed(seed)
    p = _wide(gen, N, -140, 100).to(p_dtype)
    g = _wide(gen, N, -149, 64).to(g_dtype)
    m = _wide(gen, N, -149, 64).to(formats[0][0])
    if kind == "sgdm":
        return [p, g, m]
    v = _wide(gen, N, -149, 100, signed=False).to(formats[1][0])
    return [p, g, m, v]


@pytest.mark.parametrize("kind", ["adamw", "sgdm"])
@pytest.mark.parametrize("p_dtype,g_dtype", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16)])
@pytest.mark.parametrize("formats", FORMATS, ids=lambda f: "-".join(f"{d}/{r}" for d, r in f))
@pytest.mark.parametrize("seed", [1, 2])
def test_whole_range_operands_match_the_c_oracle(cuda, kind, p_dtype, g_dtype, formats, seed):
    import sr_states
    from sr_states import StateFormat

    formats = formats[: 2 if kind == "adamw" else 1]
    key, offset = 0x2545F491 ^ seed, 2**32 - 977
    initial = _inputs(kind, p_dtype, g_dtype, formats, seed)
    expected = [t.clone() for t in initial]
    actual = [t.to(cuda) for t in initial]
    fmts = tuple(StateFormat(d, r) for d, r in formats)
    if kind == "adamw":
        c_oracle.adamw_step_(*expected, formats=formats, seed=key, offset=offset, **ADAMW)
        sr_states.hip_adamw_step_(*actual, seed=key, offset=offset, formats=fmts, **ADAMW)
        # The library square root must have been needed: some second moments
        # fall below 2^-96 and are not zero.
        v_new = expected[3].float()
        assert ((v_new > 0) & (v_new < 2.0**-96)).any() or formats[1][0] != torch.float32
    else:
        c_oracle.sgdm_step_(*expected, formats=formats, seed=key, offset=offset, **SGDM)
        sr_states.hip_sgdm_step_(*actual, seed=key, offset=offset, formats=fmts, **SGDM)
    for name, a, e in zip(("parameter", "gradient", "state 0", "state 1"), actual, expected):
        assert_bits_or_nan(a, e, f"{kind} {name}")
