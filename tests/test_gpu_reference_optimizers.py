"""The optimizers under the reference's names, on the GPU (their fused route:
every group here is one the fused launch takes).

Mirrors tests/test_reference_optimizers.py:1-103 of the reference (FP32
states against torch.optim, BF16 state bytes, the RNG position carried by a
checkpoint, deterministic round-to-nearest states) and
tests/test_state_optimizers.py:91-107 (closures and sparse gradients) for
``AdamWReferenceSR/RN`` and ``SGDMReferenceSR/RN``.  The torch optimizers
run on the CPU, as in the reference's tests, so the tolerances are the
reference's own: these optimizers compute the reference's update in
correctly rounded FP32, byte for byte, on the device.
"""

from __future__ import annotations

import copy

import pytest
import torch
from conftest import assert_bits_or_nan

from sr_states import AdamWReferenceRN, AdamWReferenceSR, SGDMReferenceRN, SGDMReferenceSR

pytestmark = pytest.mark.gpu


def _state_bytes(state):
    return sum(v.numel() * v.element_size() for v in state.values() if torch.is_tensor(v))


def test_sgdm_fp32_state_matches_torch_sgd(cuda):
    initial = torch.linspace(-1, 1, 257)
    ours = torch.nn.Parameter(initial.to(cuda))
    theirs = torch.nn.Parameter(initial.clone())
    ours_optim = SGDMReferenceSR([ours], lr=0.03, momentum=0.8, state_dtype=torch.float32)
    torch_optim = torch.optim.SGD([theirs], lr=0.03, momentum=0.8)
    for step in range(5):
        gradient = torch.sin(initial * (step + 1))
        ours.grad = gradient.to(cuda)
        theirs.grad = gradient.clone()
        ours_optim.step()
        torch_optim.step()
    torch.testing.assert_close(ours.detach().cpu(), theirs.detach(), rtol=1e-6, atol=1e-7)
    torch.testing.assert_close(ours_optim.state[ours]["momentum_buffer"].cpu(),
                               torch_optim.state[theirs]["momentum_buffer"], rtol=1e-6, atol=1e-7)


def test_adamw_fp32_state_matches_torch_adamw(cuda):
    initial = torch.linspace(-1, 1, 257)
    ours = torch.nn.Parameter(initial.to(cuda))
    theirs = torch.nn.Parameter(initial.clone())
    options = {"lr": 3e-3, "betas": (0.8, 0.95), "eps": 1e-6, "weight_decay": 0.1}
    ours_optim = AdamWReferenceSR([ours], state_dtype=torch.float32, **options)
    torch_optim = torch.optim.AdamW([theirs], foreach=False, **options)
    for step in range(5):
        gradient = torch.cos(initial * (step + 1))
        ours.grad = gradient.to(cuda)
        theirs.grad = gradient.clone()
        ours_optim.step()
        torch_optim.step()
    torch.testing.assert_close(ours.detach().cpu(), theirs.detach(), rtol=2e-6, atol=2e-7)
    for name in ("exp_avg", "exp_avg_sq"):
        torch.testing.assert_close(ours_optim.state[ours][name].cpu(), torch_optim.state[theirs][name],
                                   rtol=2e-6, atol=2e-7)


@pytest.mark.parametrize("cls", [AdamWReferenceSR, SGDMReferenceSR])
def test_bf16_state_uses_half_the_fp32_state_bytes(cuda, cls):
    p_bf16 = torch.nn.Parameter(torch.ones(128, device=cuda))
    p_fp32 = torch.nn.Parameter(torch.ones(128, device=cuda))
    bf16_optim = cls([p_bf16], lr=1e-3, state_dtype=torch.bfloat16)
    fp32_optim = cls([p_fp32], lr=1e-3, state_dtype=torch.float32)
    p_bf16.grad = torch.ones_like(p_bf16)
    p_fp32.grad = torch.ones_like(p_fp32)
    bf16_optim.step()
    fp32_optim.step()
    assert _state_bytes(bf16_optim.state[p_bf16]) * 2 == _state_bytes(fp32_optim.state[p_fp32])


@pytest.mark.parametrize("cls", [SGDMReferenceSR, AdamWReferenceSR])
def test_optimizer_state_dict_restores_rng_position(cuda, cls):
    """The resumed optimizer's own seed (999) gives way to the checkpoint's (44)."""
    initial = torch.linspace(-1, 1, 1024, device=cuda)
    first = torch.nn.Parameter(initial.clone())
    first_optim = cls([first], lr=0.01, seed=44)
    first.grad = torch.sin(initial)
    first_optim.step()

    resumed = torch.nn.Parameter(first.detach().clone())
    resumed_optim = cls([resumed], lr=0.01, seed=999)
    resumed_optim.load_state_dict(copy.deepcopy(first_optim.state_dict()))
    gradient = torch.cos(initial)
    first.grad = gradient.clone()
    resumed.grad = gradient.clone()
    first_optim.step()
    resumed_optim.step()
    assert torch.equal(first, resumed)
    for name in cls._state_names:
        assert torch.equal(first_optim.state[first][name], resumed_optim.state[resumed][name])
    # The seed matters: a fresh optimizer on seed 999 rounds the first step differently.
    other = torch.nn.Parameter(initial.clone())
    other_optim = cls([other], lr=0.01, seed=999)
    other.grad = torch.sin(initial)
    other_optim.step()
    name = cls._state_names[0]
    assert not torch.equal(other_optim.state[other][name], first_optim.state[first][name])


def test_round_to_nearest_variants_store_deterministic_bf16_state(cuda):
    runs = []
    for seed in (0, 12345):
        sgd_parameter = torch.nn.Parameter(torch.linspace(-1, 1, 64, device=cuda))
        sgd_parameter.grad = torch.cos(sgd_parameter.detach())
        sgd = SGDMReferenceRN([sgd_parameter], lr=0.01, seed=seed)
        sgd.step()
        expected_momentum = sgd_parameter.grad.float().to(torch.bfloat16)
        assert torch.equal(sgd.state[sgd_parameter]["momentum_buffer"], expected_momentum)

        adam_parameter = torch.nn.Parameter(torch.linspace(-1, 1, 64, device=cuda))
        adam_parameter.grad = torch.sin(adam_parameter.detach())
        adam = AdamWReferenceRN([adam_parameter], lr=0.01, seed=seed)
        adam.step()
        adam.step()
        states = [adam.state[adam_parameter][name] for name in ("exp_avg", "exp_avg_sq")]
        assert all(s.dtype == torch.bfloat16 for s in states)
        runs.append((adam_parameter.detach().clone(), *states))
    for a, b in zip(*runs):
        assert_bits_or_nan(a, b)


@pytest.mark.parametrize("cls", [AdamWReferenceSR, SGDMReferenceSR])
def test_closure_and_sparse_gradient(cuda, cls):
    p = torch.nn.Parameter(torch.ones(4, device=cuda))
    optimizer = cls([p], lr=0.01)

    def closure():
        optimizer.zero_grad()
        loss = p.square().sum()
        loss.backward()
        return loss

    assert optimizer.step(closure).item() == 4
    p.grad = torch.sparse_coo_tensor([[0]], [1.0], size=(4,), device=cuda, check_invariants=True)
    rng_step = optimizer._rng_step()
    with pytest.raises(RuntimeError, match="sparse"):
        optimizer.step()
    assert optimizer._rng_step() == rng_step + 1
