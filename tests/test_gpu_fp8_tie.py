"""FP8 round-to-nearest ties through the fused HIP updates.

The reference's fusion-boundary case (tests/test_triton_states.py:85-113):
with an E4M3-nearest momentum u = 15/512 and gradient -8/512, the eager order
u' = RN(RN(0.9 u) + g) lands exactly on the subnormal tie 5.5/512, which
rounds to even, 6/512.  A contracted FMA (fma(u, 0.9, g)) gives a value just
off the tie and can store 5/512.  The fused SGDM, functional and through the
optimizer, must store 6/512 for every element, with either sign and either
parameter dtype, and equal the C oracle byte for byte.

The AdamW analogue: the eager first moment is m' = fma(g, 1 - beta1,
RN(m beta1)) (sr_states/reference/adamw.py:81).  With m = 2^-9 (the smallest
E4M3 subnormal), beta1 = 0.9 and g = 331/512 that is exactly the E4M3 tie
0.06640625 between 0.0625 and 0.0703125, stored as the even 0.0625.  The
other association, fma(m, beta1, RN(g (1 - beta1))), and the unfused sum
both land just above the tie and store 0.0703125, so a kernel that fused or
split the moment's operations differently fails here.
"""

from __future__ import annotations

import pytest
import torch
from conftest import assert_bits_or_nan

import sr_states
from oracle import c_oracle
from sr_states import StateFormat

pytestmark = pytest.mark.gpu

E4M3_NEAREST = StateFormat(torch.float8_e4m3fn, "nearest")
TIE_M, TIE_G, TIE_EVEN = 2.0**-9, 331 / 512, 0.0625


def _signs(n, device):
    return (1 - 2 * (torch.arange(n, device=device) % 2)).float()


@pytest.mark.parametrize("p_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n", [1, 1003])
def test_sgdm_functional_stores_the_even_neighbour(cuda, p_dtype, n):
    signs = _signs(n, cuda)
    p = torch.ones(n, device=cuda, dtype=p_dtype)
    g = (-signs * (8 / 512)).to(p_dtype)
    u = (signs * (15 / 512)).to(torch.float8_e4m3fn)
    expected = [t.cpu().clone() for t in (p, g, u)]
    sr_states.hip_sgdm_step_(p, g, u, lr=1e-3, momentum_factor=0.9, seed=0, formats=(E4M3_NEAREST,))
    assert torch.equal(u.float(), signs * (6 / 512))
    c_oracle.sgdm_step_(*expected, lr=1e-3, momentum_factor=0.9,
                        formats=[(torch.float8_e4m3fn, "nearest")], seed=0)
    assert_bits_or_nan(u.cpu(), expected[2], "momentum")
    assert_bits_or_nan(p.cpu(), expected[0], "parameter")


@pytest.mark.parametrize("p_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n", [1, 1003])
def test_sgdm_optimizer_stores_the_even_neighbour(cuda, p_dtype, n):
    """Step 1 stores u = g1 = 15/512 exactly; step 2 lands on the tie."""
    signs = _signs(n, cuda)
    parameter = torch.nn.Parameter(torch.ones(n, device=cuda, dtype=p_dtype))
    opt = sr_states.SGDMHip([parameter], lr=1e-3, momentum=0.9, state_format=E4M3_NEAREST, seed=5)
    grads = [(signs * (15 / 512)).to(p_dtype), (-signs * (8 / 512)).to(p_dtype)]
    p_ref = parameter.detach().cpu().clone()
    u_ref = torch.zeros(n, dtype=torch.float8_e4m3fn)
    for step, g in enumerate(grads, start=1):
        parameter.grad = g
        opt.step()
        key = sr_states.update_key(5, step, 0)
        c_oracle.sgdm_step_(p_ref, g.cpu(), u_ref, lr=1e-3, momentum_factor=0.9,
                            formats=[(torch.float8_e4m3fn, "nearest")], seed=key)
    stored = opt.state[parameter]["momentum_buffer"]
    assert torch.equal(stored.float(), signs * (6 / 512))
    assert_bits_or_nan(stored.cpu(), u_ref, "momentum")
    assert_bits_or_nan(parameter.detach().cpu(), p_ref, "parameter")


ADAMW = {"lr": 1e-3, "beta1": 0.9, "beta2": 0.999, "eps": 1e-8, "weight_decay": 0.0}


@pytest.mark.parametrize("p_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n", [1, 1003])
def test_adamw_first_moment_tie_stores_the_even_neighbour(cuda, p_dtype, n):
    signs = _signs(n, cuda)
    p = torch.ones(n, device=cuda, dtype=p_dtype)
    g = signs * TIE_G
    m = (signs * TIE_M).to(torch.float8_e4m3fn)
    v = torch.zeros(n, device=cuda, dtype=torch.bfloat16)
    expected = [t.cpu().clone() for t in (p, g, m, v)]
    formats = (E4M3_NEAREST, StateFormat(torch.bfloat16, "nearest"))
    sr_states.hip_adamw_step_(p, g, m, v, step=3, seed=9, formats=formats, **ADAMW)
    assert torch.equal(m.float(), signs * TIE_EVEN)
    c_oracle.adamw_step_(*expected, step=3, seed=9,
                         formats=[(torch.float8_e4m3fn, "nearest"), (torch.bfloat16, "nearest")], **ADAMW)
    for name, got, want in zip(("parameter", "exp_avg", "exp_avg_sq"), (p, m, v), expected[:1] + expected[2:]):
        assert_bits_or_nan(got.cpu(), want, name)


def test_adamw_optimizer_first_moment_tie(cuda):
    """Step 1 stores m = RN_E4M3(RN(0.1 g1)) = 2^-9; step 2 lands on the tie."""
    n = 1003
    signs = _signs(n, cuda)
    parameter = torch.nn.Parameter(torch.ones(n, device=cuda))
    formats = {"exp_avg": E4M3_NEAREST, "exp_avg_sq": StateFormat(torch.bfloat16, "nearest")}
    opt = sr_states.AdamWHip([parameter], lr=1e-3, weight_decay=0.0, state_format=formats, seed=4)
    grads = [signs * (10 / 512), signs * TIE_G]
    p_ref = parameter.detach().cpu().clone()
    states = [torch.zeros(n, dtype=torch.float8_e4m3fn), torch.zeros(n, dtype=torch.bfloat16)]
    for step, g in enumerate(grads, start=1):
        parameter.grad = g
        opt.step()
        if step == 1:
            assert torch.equal(opt.state[parameter]["exp_avg"].float(), signs * TIE_M)
        c_oracle.adamw_step_(p_ref, g.cpu(), *states, step=step, seed=sr_states.update_key(4, step, 0),
                             formats=[(torch.float8_e4m3fn, "nearest"), (torch.bfloat16, "nearest")],
                             **ADAMW)
    stored = opt.state[parameter]
    assert torch.equal(stored["exp_avg"].float(), signs * TIE_EVEN)
    assert_bits_or_nan(stored["exp_avg"].cpu(), states[0], "exp_avg")
    assert_bits_or_nan(stored["exp_avg_sq"].cpu(), states[1], "exp_avg_sq")
    assert_bits_or_nan(parameter.detach().cpu(), p_ref, "parameter")
