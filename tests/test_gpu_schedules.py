"""Learning-rate schedules and hyperparameter changes between steps, on the GPU.

Schedulers (``torch.optim.lr_scheduler``) and training scripts change a
group's ``lr`` (and sometimes ``betas``, ``eps``, ``weight_decay`` or
``momentum``) between steps.  The reference reads every value from the group
when its step runs (optim/_state.py:154-200, triton/adamw.py:289-319,
triton/sgd.py:214-237).  Here the steps after the first reuse their tables
(the steady-state path), so these tests check that the reuse still takes each
step's values: every parameter and state equals the C oracle's replay with
the value in force at that step, byte for byte.
"""

from __future__ import annotations

import math

import pytest
import torch
from conftest import assert_bits_or_nan

import sr_states
from oracle import c_oracle, sr_oracle
from sr_states import StateFormat

pytestmark = pytest.mark.gpu

SHAPES = [(33, 17), (1000,), (5,), (4, 4, 4)]
SEED = 23


def _model(device):
    gen = torch.Generator().manual_seed(0)
    return [torch.nn.Parameter(torch.randn(s, generator=gen).to(device)) for s in SHAPES]


def _gradients(params, step):
    gen = torch.Generator().manual_seed(100 + step)
    for param in params:
        param.grad = (torch.randn(param.shape, generator=gen) * 0.1).to(param.device)


def _groups(params, **second):
    return [{"params": params[:2]}, {"params": params[2:], **second}]


def _replay(kind, steps, formats, schedule):
    """C-oracle replay: ``schedule(t)`` gives each group's hyperparameters at step t."""
    params = [p.detach().cpu().clone() for p in _model("cpu")]
    states = [[torch.zeros_like(p, dtype=fmt[0]) for fmt in formats] for p in params]
    for t in range(1, steps + 1):
        _gradients(params, t - 1)
        for index, (p, s) in enumerate(zip(params, states)):
            hp = schedule(t)[0 if index < 2 else 1]
            key = sr_oracle.update_key(SEED, t, index)
            if kind == "adamw":
                c_oracle.adamw_step_(p, p.grad, *s, lr=hp["lr"], beta1=hp["betas"][0], beta2=hp["betas"][1],
                                     eps=hp["eps"], weight_decay=hp["weight_decay"], step=t, formats=formats,
                                     seed=key)
            else:
                c_oracle.sgdm_step_(p, p.grad, *s, lr=hp["lr"], momentum_factor=hp["momentum"],
                                    formats=formats, seed=key)
    return params, states


def _assert_run(params, optimizer, expected):
    want_params, want_states = expected
    for p, want_p, want_s in zip(params, want_params, want_states):
        assert_bits_or_nan(p.detach().cpu(), want_p, "parameter")
        for name, want in zip(optimizer._state_names, want_s):
            assert_bits_or_nan(optimizer.state[p][name].cpu(), want, name)


ADAMW_CLASSES = [sr_states.AdamWHip, sr_states.AdamWReferenceSR]
SGDM_CLASSES = [sr_states.SGDMHip, sr_states.SGDMReferenceSR]


@pytest.mark.parametrize("cls", ADAMW_CLASSES, ids=lambda c: c.__name__)
def test_adamw_follows_a_cosine_schedule_with_warmup(cuda, cls):
    steps, base = 8, (1e-3, 3e-3)

    def factor(epoch):  # LambdaLR's epoch: 0 before the first step
        return (epoch + 1) / 3 if epoch < 2 else 0.5 * (1 + math.cos(math.pi * (epoch - 2) / (steps - 2)))

    formats = ((torch.float8_e4m3fn, "stochastic"), (torch.bfloat16, "stochastic"))
    params = _model(cuda)
    optimizer = cls(_groups(params, lr=base[1]), lr=base[0], seed=SEED,
                    state_format={"exp_avg": StateFormat(*formats[0]), "exp_avg_sq": StateFormat(*formats[1])})
    scheduler = torch.optim.lr_scheduler.LambdaLR(optimizer, factor)
    used = []
    for t in range(steps):
        _gradients(params, t)
        used.append([g["lr"] for g in optimizer.param_groups])
        optimizer.step()
        scheduler.step()
    assert len({tuple(u) for u in used}) == steps  # a new rate at every step

    def schedule(t):
        return [{"lr": used[t - 1][k], "betas": (0.9, 0.999), "eps": 1e-8, "weight_decay": 1e-2} for k in (0, 1)]

    _assert_run(params, optimizer, _replay("adamw", steps, formats, schedule))


@pytest.mark.parametrize("cls", SGDM_CLASSES, ids=lambda c: c.__name__)
def test_sgdm_follows_step_and_exponential_decay(cuda, cls):
    steps = 7
    formats = ((torch.float16, "stochastic"),)
    params = _model(cuda)
    optimizer = cls(_groups(params, lr=0.05), lr=0.1, momentum=0.9, seed=SEED, state_dtype=torch.float16)
    scheduler = torch.optim.lr_scheduler.SequentialLR(
        optimizer,
        [torch.optim.lr_scheduler.StepLR(optimizer, step_size=2, gamma=0.5),
         torch.optim.lr_scheduler.ExponentialLR(optimizer, gamma=0.7)],
        milestones=[4],
    )
    used = []
    for t in range(steps):
        _gradients(params, t)
        used.append([g["lr"] for g in optimizer.param_groups])
        optimizer.step()
        scheduler.step()

    def schedule(t):
        return [{"lr": used[t - 1][k], "momentum": 0.9} for k in (0, 1)]

    _assert_run(params, optimizer, _replay("sgdm", steps, formats, schedule))


@pytest.mark.parametrize("cls", ADAMW_CLASSES, ids=lambda c: c.__name__)
def test_adamw_takes_every_group_value_in_force_at_each_step(cuda, cls):
    """betas, eps and weight_decay changed by hand between steps, one group at a time."""
    formats = ((torch.bfloat16, "stochastic"),) * 2
    hp = [{"lr": 1e-3, "betas": (0.9, 0.999), "eps": 1e-8, "weight_decay": 1e-2},
          {"lr": 3e-3, "betas": (0.9, 0.999), "eps": 1e-8, "weight_decay": 1e-2}]
    changes = {2: (1, {"betas": (0.8, 0.99)}), 3: (0, {"eps": 1e-6, "weight_decay": 0.1}),
               4: (1, {"lr": 1e-2, "weight_decay": 0.0}), 5: (0, {"betas": (0.0, 0.5), "lr": 5e-4})}
    params = _model(cuda)
    optimizer = cls(_groups(params, lr=3e-3), lr=1e-3, seed=SEED)
    history = []
    for t in range(1, 7):
        if t in changes:
            group, values = changes[t]
            optimizer.param_groups[group].update(values)
            hp[group] = {**hp[group], **values}
        history.append([dict(h) for h in hp])
        _gradients(params, t - 1)
        optimizer.step()
    _assert_run(params, optimizer, _replay("adamw", 6, formats, lambda t: history[t - 1]))


@pytest.mark.parametrize("cls", SGDM_CLASSES, ids=lambda c: c.__name__)
def test_sgdm_takes_the_momentum_in_force_at_each_step(cuda, cls):
    formats = ((torch.bfloat16, "stochastic"),)
    params = _model(cuda)
    optimizer = cls(_groups(params, lr=0.02), lr=0.01, momentum=0.9, seed=SEED)
    history = []
    for t in range(1, 6):
        if t == 3:
            optimizer.param_groups[1]["momentum"] = 0.5
        if t == 4:
            optimizer.param_groups[0]["momentum"] = 0.0
        history.append([{"lr": g["lr"], "momentum": g["momentum"]} for g in optimizer.param_groups])
        _gradients(params, t - 1)
        optimizer.step()
    _assert_run(params, optimizer, _replay("sgdm", 5, formats, lambda t: history[t - 1]))


def test_a_schedule_survives_a_checkpoint(cuda):
    """Optimizer and scheduler state saved at step 3 and loaded into fresh objects continue identically."""
    formats = ((torch.bfloat16, "stochastic"),) * 2

    def build(params):
        optimizer = sr_states.AdamWHip(_groups(params, lr=3e-3), lr=1e-3, seed=SEED)
        return optimizer, torch.optim.lr_scheduler.ExponentialLR(optimizer, gamma=0.8)

    params = _model(cuda)
    optimizer, scheduler = build(params)
    used = []
    for t in range(3):
        _gradients(params, t)
        used.append([g["lr"] for g in optimizer.param_groups])
        optimizer.step()
        scheduler.step()
    saved = (optimizer.state_dict(), scheduler.state_dict())
    resumed_params = [torch.nn.Parameter(p.detach().clone()) for p in params]
    resumed, resumed_scheduler = build(resumed_params)
    resumed.load_state_dict(saved[0])
    resumed_scheduler.load_state_dict(saved[1])
    for t in range(3, 6):
        _gradients(params, t)
        _gradients(resumed_params, t)
        used.append([g["lr"] for g in optimizer.param_groups])
        assert [g["lr"] for g in resumed.param_groups] == used[-1]
        for opt, sched in ((optimizer, scheduler), (resumed, resumed_scheduler)):
            opt.step()
            sched.step()
    for p, q in zip(params, resumed_params):
        assert torch.equal(p, q)
        for name in optimizer._state_names:
            assert torch.equal(optimizer.state[p][name], resumed.state[q][name])

    def schedule(t):
        return [{"lr": used[t - 1][k], "betas": (0.9, 0.999), "eps": 1e-8, "weight_decay": 1e-2} for k in (0, 1)]

    _assert_run(params, optimizer, _replay("adamw", 6, formats, schedule))
