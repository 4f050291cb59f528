"""Mixed-precision training with ``torch.amp.GradScaler`` around the fused optimizers, on the GPU.

The scaler unscales the gradients in place, then calls ``step()`` only when
they are finite; skipped steps must leave parameters, states and the RNG
step untouched, so that the next applied step draws the bits the reference
would draw (optim/_state.py:154-200: one RNG step per call of ``step``).
Each applied step is replayed through the C oracle from the unscaled
gradients it saw: parameters and states equal byte for byte.
"""

from __future__ import annotations

import pytest
import torch
from conftest import assert_bits_or_nan

import sr_states
from oracle import c_oracle, sr_oracle

pytestmark = pytest.mark.gpu

HYPER = {"lr": 1e-3, "beta1": 0.9, "beta2": 0.999, "eps": 1e-8, "weight_decay": 1e-2}


@pytest.mark.parametrize("cls", [sr_states.AdamWHip, sr_states.AdamWReferenceSR], ids=lambda c: c.__name__)
def test_grad_scaler_skips_overflowing_steps_and_applies_the_rest(cuda, cls):
    gen = torch.Generator().manual_seed(0)
    model = torch.nn.Sequential(torch.nn.Linear(64, 96), torch.nn.ReLU(), torch.nn.Linear(96, 8))
    for p in model.parameters():
        p.data = torch.randn(p.shape, generator=gen) * 0.1
    model = model.to(cuda)
    initial = [p.detach().cpu().clone() for p in model.parameters()]
    optimizer = cls(model.parameters(), lr=HYPER["lr"], weight_decay=HYPER["weight_decay"], seed=9)
    # A scale far above FP16's range: the first backward passes overflow and
    # their steps are skipped while the scaler backs off.
    scaler = torch.amp.GradScaler("cuda", init_scale=2.0**28, growth_interval=1000)
    applied, skipped = [], 0
    for t in range(24):
        x = torch.randn(32, 64, generator=gen).to(cuda)
        y = torch.randn(32, 8, generator=gen).to(cuda)
        optimizer.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.float16):
            loss = torch.nn.functional.mse_loss(model(x).float(), y)
        scaler.scale(loss).backward()
        scaler.unscale_(optimizer)
        grads = [p.grad.detach().cpu().clone() for p in model.parameters()]
        rng_before = optimizer._rng_step()
        scale = scaler.get_scale()
        scaler.step(optimizer)
        scaler.update()
        if scaler.get_scale() < scale:  # found an inf or NaN: step() was not called
            skipped += 1
            assert optimizer._rng_step() == rng_before
            assert any(not torch.isfinite(g).all() for g in grads)
        else:
            assert optimizer._rng_step() == rng_before + 1
            applied.append(grads)
    assert skipped >= 2 and len(applied) >= 10

    params = [p.clone() for p in initial]
    states = [[torch.zeros_like(p, dtype=torch.bfloat16) for _ in range(2)] for p in params]
    for rng_step, grads in enumerate(applied, start=1):
        for index, (p, g, (m, v)) in enumerate(zip(params, grads, states)):
            c_oracle.adamw_step_(p, g, m, v, step=rng_step, formats=((torch.bfloat16, "stochastic"),) * 2,
                                 seed=sr_oracle.update_key(9, rng_step, index), **HYPER)
    for p, want, (m, v) in zip(model.parameters(), params, states):
        assert_bits_or_nan(p.detach().cpu(), want, "parameter")
        assert_bits_or_nan(optimizer.state[p]["exp_avg"].cpu(), m, "exp_avg")
        assert_bits_or_nan(optimizer.state[p]["exp_avg_sq"].cpu(), v, "exp_avg_sq")
        assert optimizer.state[p]["step"] == len(applied)
