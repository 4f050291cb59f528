"""FP16/FP8 state formats through the fused optimizers on the device.

Mirrors tests/test_minifloat_gpu.py: the three spellings of one state format
(state_dtype + rounding, one StateFormat, a per-state dict) give identical
bytes, and mixed E4M3/E5M2 states follow the reference recurrence step by
step and resume from a checkpoint mid-run.  The reference compares its fused
path with its eager CPU classes (FP32 parameters to rtol 1e-5); here the
comparison is with the C oracle, which restates the eager recurrence
operation for operation, so parameters must match bit for bit as well.
"""

from __future__ import annotations

import copy

import pytest
import torch
from conftest import assert_bits_or_nan

from oracle import c_oracle, sr_oracle

pytestmark = pytest.mark.gpu

MODES = ("stochastic", "nearest")


@pytest.mark.parametrize("kind", ["adamw", "sgdm"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.float8_e4m3fn,
                                   torch.float8_e5m2])
@pytest.mark.parametrize("mode", MODES)
def test_shorthand_single_and_dict_are_identical(cuda, kind, dtype, mode):
    """tests/test_minifloat_gpu.py:166-186."""
    import sr_states
    from sr_states import StateFormat

    cls = sr_states.AdamWHip if kind == "adamw" else sr_states.SGDMHip
    fmt = StateFormat(dtype, mode)
    params = [torch.nn.Parameter(torch.linspace(-1, 1, 257, device=cuda)) for _ in range(3)]
    args = [{"state_dtype": dtype, "rounding": mode}, {"state_format": fmt},
            {"state_format": dict.fromkeys(cls._state_names, fmt)}]
    opts = [cls([p], lr=0.001, seed=17, **arg) for p, arg in zip(params, args)]
    for step in range(3):
        for p, opt in zip(params, opts):
            p.grad = torch.sin(torch.arange(257, device=cuda) + step)
            opt.step()
        for p, opt in zip(params[1:], opts[1:]):
            assert torch.equal(p, params[0])
            for name in cls._state_names:
                assert_bits_or_nan(opt.state[p][name], opts[0].state[params[0]][name], name)


@pytest.mark.parametrize("kind", ["adamw", "sgdm"])
@pytest.mark.parametrize("mode", MODES)
def test_mixed_states_match_the_recurrence_and_resume(cuda, kind, mode):
    """tests/test_minifloat_gpu.py:88-133 against the C oracle."""
    import sr_states
    from sr_states import StateFormat

    n, lr, seed = 1027, 2.0**-10, 27
    p = torch.nn.Parameter(torch.linspace(-1, 1, n, device=cuda))
    p_ref = p.detach().cpu().clone()
    if kind == "adamw":
        formats = {"exp_avg": StateFormat(torch.float8_e4m3fn, mode),
                   "exp_avg_sq": StateFormat(torch.float8_e5m2, mode)}
        oracle_formats = ((torch.float8_e4m3fn, mode), (torch.float8_e5m2, mode))
        opt = sr_states.AdamWHip([p], lr=lr, betas=(0.5, 0.5), eps=0.125, weight_decay=0.0,
                                 state_format=formats, seed=seed)
    else:
        oracle_formats = ((torch.float8_e4m3fn, mode),)
        opt = sr_states.SGDMHip([p], lr=lr, momentum=0.5, state_format=StateFormat(torch.float8_e4m3fn, mode),
                                seed=seed)
    states_ref = [torch.zeros(n, dtype=dtype) for dtype, _ in oracle_formats]
    r = resumed = None
    for step in range(8):
        # Dyadic gradients and betas make the moment arithmetic exact.
        grad = ((torch.arange(n, device=cuda) + step) % 15 - 7).float() * 2**-5
        p.grad = grad
        opt.step()
        key = sr_oracle.update_key(seed, step + 1, 0)
        if kind == "adamw":
            c_oracle.adamw_step_(p_ref, grad.cpu(), *states_ref, lr=lr, beta1=0.5, beta2=0.5, eps=0.125,
                                 weight_decay=0.0, step=step + 1, formats=oracle_formats, seed=key)
        else:
            c_oracle.sgdm_step_(p_ref, grad.cpu(), *states_ref, lr=lr, momentum_factor=0.5, formats=oracle_formats,
                                seed=key)
        assert_bits_or_nan(p.detach().cpu(), p_ref, f"parameter after step {step + 1}")
        for name, expected in zip(opt._state_names, states_ref):
            assert_bits_or_nan(opt.state[p][name], expected, f"{name} after step {step + 1}")
        if resumed is not None:
            r.grad = grad
            resumed.step()
            assert torch.equal(p, r)
            for name in opt._state_names:
                assert_bits_or_nan(resumed.state[r][name], opt.state[p][name], f"resumed {name}")
        if step == 3:
            r = torch.nn.Parameter(p.detach().clone())
            cls = type(opt)
            resumed = cls([r], **({"lr": 0.1} if kind == "sgdm" else {}))
            resumed.load_state_dict(copy.deepcopy(opt.state_dict()))
