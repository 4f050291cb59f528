"""Seeded random parameter groups through the fused optimizers, against the C oracle.

Each case draws an optimizer (AdamW or momentum SGD), one to three groups
with their own state formats (all nine policies, per state), learning rates,
betas, seeds and starting RNG steps, one to five parameters per group (FP32
or BF16, with FP32 or BF16 gradients, of sizes around the tile edges,
aligned or not), a workgroup size, and a few steps in which a random subset
of parameters has gradients.  After every step each parameter and state must
equal the C oracle's replay byte for byte, parameters included.  The replay
follows the reference's contract (sr_states/optim/_state.py:154-200): one
RNG step per optimizer step for every group, parameter indices counted over
all groups including parameters without gradients, and per-parameter AdamW
steps.
"""

from __future__ import annotations

import random

import pytest
import torch
from conftest import assert_bits_or_nan

from oracle import c_oracle, sr_oracle

pytestmark = pytest.mark.gpu

STATE_DTYPES = (torch.float32, torch.bfloat16, torch.float16, torch.float8_e4m3fn, torch.float8_e5m2)
SIZES = (1, 2, 3, 7, 255, 256, 511, 512, 513, 1023, 1024, 2049, 4099, 70001)


class _MixedGradientParameter(torch.nn.Parameter):
    """Parameter whose gradient may have another dtype (tests/test_triton_multi_tensor.py:22-31)."""

    @property
    def grad(self):
        return getattr(self, "_gradient", None)

    @grad.setter
    def grad(self, value):
        self._gradient = value


def _draw_case(rng, cuda):
    kind = rng.choice(["adamw", "sgd"])
    names = ("exp_avg", "exp_avg_sq") if kind == "adamw" else ("momentum_buffer",)
    groups = []
    for _ in range(rng.randint(1, 3)):
        params = []
        for _ in range(rng.randint(1, 5)):
            n = rng.choice(SIZES)
            p_dtype = rng.choice((torch.float32, torch.bfloat16))
            g_dtype = rng.choice((torch.float32, torch.bfloat16))
            values = torch.linspace(-rng.uniform(0.1, 2), rng.uniform(0.1, 2), n + 1, device=cuda)
            data = values.to(p_dtype)[1:] if rng.random() < 0.4 else values[:n].to(p_dtype).clone()
            params.append((_MixedGradientParameter(data), g_dtype))
        formats = tuple((rng.choice(STATE_DTYPES), rng.choice(("stochastic", "nearest"))) for _ in names)
        group = {"seed": rng.choice((0, 7, -(2**48) - 1, 2**63 + 12345, rng.getrandbits(64))),
                 "start": rng.choice((0, 0, 5, 2**32 - 2)), "lr": rng.uniform(1e-4, 0.1), "formats": formats}
        if kind == "adamw":
            group.update(betas=(rng.uniform(0.5, 0.95), rng.uniform(0.9, 0.9999)), eps=rng.choice((1e-8, 1e-6, 0.125)),
                         weight_decay=rng.choice((0.0, 0.01, 0.1)))
        else:
            group.update(momentum=rng.uniform(0.0, 0.99))
        groups.append((params, group))
    return kind, names, groups


@pytest.mark.parametrize("case", range(32))
def test_random_groups_match_the_c_oracle(cuda, case):
    import sr_states
    from sr_states import StateFormat

    rng = random.Random(9000 + case)
    kind, names, groups = _draw_case(rng, cuda)
    adamw = kind == "adamw"
    param_groups = []
    for params, g in groups:
        entry = {"params": [p for p, _ in params], "lr": g["lr"], "sr_seed": g["seed"], "sr_step": g["start"],
                 "state_format": {name: StateFormat(d, r) for name, (d, r) in zip(names, g["formats"])}}
        if adamw:
            entry.update(betas=g["betas"], eps=g["eps"], weight_decay=g["weight_decay"])
        else:
            entry.update(momentum=g["momentum"])
        param_groups.append(entry)
    block_size = rng.choice((128, 256, 512, 1024))
    opt = (sr_states.AdamWHip(param_groups, block_size=block_size) if adamw
           else sr_states.SGDMHip(param_groups, lr=0.01, block_size=block_size))

    flat = [(p, g_dtype, g) for params, g in groups for p, g_dtype in params]
    expected = {p: p.detach().cpu().clone() for p, _, _ in flat}
    states, steps = {}, {}
    gen = torch.Generator(device=cuda).manual_seed(case)
    rng_step = max(g["start"] for _, g in groups)
    for step in range(rng.randint(1, 3)):
        with_grad = [rng.random() < 0.8 for _ in flat]
        for (p, g_dtype, _), has in zip(flat, with_grad):
            p.grad = (torch.randn(p.numel(), device=cuda, generator=gen) * 1e-2).to(g_dtype) if has else None
        opt.step()
        rng_step += 1
        assert opt._rng_step() == rng_step
        for index, ((p, _, g), has) in enumerate(zip(flat, with_grad)):
            if not has:
                continue
            states.setdefault(p, [torch.zeros(p.numel(), dtype=d) for d, _ in g["formats"]])
            steps[p] = steps.get(p, 0) + 1
            key = sr_oracle.update_key(g["seed"], rng_step, index)
            grad = p.grad.cpu()
            if adamw:
                c_oracle.adamw_step_(expected[p], grad, *states[p], lr=g["lr"], beta1=g["betas"][0],
                                     beta2=g["betas"][1], eps=g["eps"], weight_decay=g["weight_decay"],
                                     step=steps[p], formats=g["formats"], seed=key)
            else:
                c_oracle.sgdm_step_(expected[p], grad, *states[p], lr=g["lr"], momentum_factor=g["momentum"],
                                    formats=g["formats"], seed=key)
        for index, (p, _, _) in enumerate(flat):
            what = f"case {case} step {step + 1} parameter {index} ({p.numel()} elements, {p.dtype})"
            assert_bits_or_nan(p.detach().cpu(), expected[p], what)
            for name, state in zip(names, states.get(p, ())):
                assert_bits_or_nan(opt.state[p][name].cpu(), state, f"{what} {name}")
            if adamw:
                assert opt.state[p].get("step") == steps.get(p)
