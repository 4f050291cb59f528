"""States of a group's parameters as views into one allocation per state name.

The optimizers place the states a step's walk creates (or a checkpoint load
restores) for plain contiguous GPU parameters in one zeroed allocation per
state name and dtype, each view on a 512-byte boundary, where the reference
allocates each state on its own.  Here the bytes of parameters and states
over several steps must equal those of the same optimizer with one
allocation per state (``_shared_state_allocations = False``), for the fused
optimizers and the reference-named ones; the views must be disjoint,
aligned and of the parameter's shape; a parameter whose gradient first
appears at a later step must get a fresh zero state; and a checkpoint must
load into shared views holding the saved bytes.
"""

from __future__ import annotations

import pytest
import torch
from conftest import assert_bits_or_nan

import sr_states
from sr_states import AdamWHip, AdamWReferenceSR, SGDMHip, SGDMReferenceSR

pytestmark = pytest.mark.gpu

SHAPES = [(37, 11), (768,), (129,), (64, 64), (1,), (5, 7, 3), (1000,)]
CLASSES = [AdamWHip, SGDMHip, AdamWReferenceSR, SGDMReferenceSR]


def _make(cls, cuda, shared, formats=None):
    gen = torch.Generator().manual_seed(11)
    params = [torch.nn.Parameter((torch.randn(s, generator=gen) * 0.02).to(cuda)) for s in SHAPES]
    kwargs = {"lr": 1e-3, "weight_decay": 0.01} if cls in (AdamWHip, AdamWReferenceSR) else {"lr": 0.1}
    if formats is not None:
        kwargs["state_format"] = formats
    opt = cls([{"params": params[:4]}, {"params": params[4:]}], seed=9, **kwargs)
    opt._shared_state_allocations = shared
    return params, opt


def _grads(params, step, skip=()):
    gen = torch.Generator().manual_seed(100 + step)
    for index, p in enumerate(params):
        g = torch.randn(p.shape, generator=gen) * 1e-3
        p.grad = None if index in skip else g.to(p.device)


@pytest.mark.parametrize("cls", CLASSES, ids=lambda c: c.__name__)
def test_shared_states_give_the_same_bytes_as_separate_ones(cuda, cls):
    runs = []
    for shared in (True, False):
        params, opt = _make(cls, cuda, shared)
        for step in range(4):
            # The third parameter has no gradient until step 2: its states
            # come from a later walk's allocation.
            _grads(params, step, skip=(2,) if step < 2 else ())
            opt.step()
        torch.cuda.synchronize()
        runs.append((params, opt))
    (shared_params, shared_opt), (own_params, own_opt) = runs
    for index, (a, b) in enumerate(zip(shared_params, own_params)):
        assert_bits_or_nan(a.detach().cpu(), b.detach().cpu(), f"parameter {index}")
        for name in shared_opt._state_names:
            assert_bits_or_nan(shared_opt.state[a][name].cpu(), own_opt.state[b][name].cpu(), f"{name} {index}")
        assert shared_opt.state[a].get("step") == own_opt.state[b].get("step")


@pytest.mark.parametrize("cls", [AdamWHip, SGDMReferenceSR], ids=lambda c: c.__name__)
def test_one_walk_places_each_state_name_in_one_allocation(cuda, cls):
    params, opt = _make(cls, cuda, True)
    _grads(params, 0, skip=(5,))
    opt.step()
    torch.cuda.synchronize()
    for group in opt.param_groups:
        for name in opt._state_names:
            views = [opt.state[p][name] for p in group["params"] if p.grad is not None]
            bases = {v.untyped_storage().data_ptr() for v in views}
            assert len(bases) == 1, f"{name}: {len(bases)} allocations in one group"
            spans = sorted((v.data_ptr(), v.data_ptr() + v.numel() * v.element_size()) for v in views)
            assert all(start % 512 == 0 for start, _ in spans)
            assert all(end <= start for (_, end), (start, _) in zip(spans, spans[1:])), "views overlap"
            for p in group["params"]:
                if p.grad is not None:
                    assert opt.state[p][name].shape == p.shape and opt.state[p][name].is_contiguous()
        # Different state names never share an allocation.
        if len(opt._state_names) == 2:
            first = group["params"][0]
            a, b = (opt.state[first][n].untyped_storage().data_ptr() for n in opt._state_names)
            assert a != b
    # The parameter without a gradient owns no state.
    assert params[5] not in opt.state or not opt.state[params[5]]
    # Its gradient appears: a fresh allocation, zeroed, then updated.
    _grads(params, 1)
    opt.step()
    torch.cuda.synchronize()
    assert set(opt._state_names) <= set(opt.state[params[5]])


def test_checkpoint_loads_into_shared_views(cuda):
    formats = {"exp_avg": sr_states.StateFormat(torch.float8_e4m3fn), "exp_avg_sq": sr_states.StateFormat(torch.bfloat16)}
    params, opt = _make(AdamWHip, cuda, False, formats)
    for step in range(2):
        _grads(params, step)
        opt.step()
    saved = opt.state_dict()
    saved_bytes = {k: {n: v.clone() for n, v in entry.items() if torch.is_tensor(v)}
                   for k, entry in saved["state"].items()}
    fresh, restored = _make(AdamWHip, cuda, True, formats)
    with torch.no_grad():
        for a, b in zip(params, fresh):
            b.copy_(a)
    restored.load_state_dict(saved)
    for group in restored.param_groups:
        for name in restored._state_names:
            bases = {restored.state[p][name].untyped_storage().data_ptr() for p in group["params"]}
            assert len(bases) == 1
    for index, p in enumerate(fresh):
        for name in restored._state_names:
            value = restored.state[p][name]
            assert value.dtype == formats[name].dtype and value.shape == p.shape
            assert torch.equal(value.view(torch.uint8).cpu(), saved_bytes[index][name].view(torch.uint8).cpu())
    # Both continue identically.
    for optimizer, group_params in ((opt, params), (restored, fresh)):
        _grads(group_params, 5)
        optimizer.step()
    torch.cuda.synchronize()
    for a, b in zip(params, fresh):
        assert torch.equal(a.detach().view(torch.int32).cpu(), b.detach().view(torch.int32).cpu())
        for name in opt._state_names:
            assert torch.equal(opt.state[a][name].view(torch.uint8).cpu(), restored.state[b][name].view(torch.uint8).cpu())


def test_allocations_split_at_the_limit_give_the_same_bytes(cuda, monkeypatch):
    """With a 4 KiB limit the group's states spread over several allocations; bytes unchanged."""
    from sr_states.optim import _state

    monkeypatch.setattr(_state, "_SHARED_MAX_BYTES", 4096)
    runs = []
    for shared in (True, False):
        params, opt = _make(AdamWHip, cuda, shared)
        for step in range(3):
            _grads(params, step)
            opt.step()
        torch.cuda.synchronize()
        runs.append((params, opt))
    (params, opt), (own_params, own_opt) = runs
    bases = {opt.state[p]["exp_avg"].untyped_storage().data_ptr() for p in params}
    assert 2 < len(bases) < len(params) + 1
    for index, (a, b) in enumerate(zip(params, own_params)):
        assert_bits_or_nan(a.detach().cpu(), b.detach().cpu(), f"parameter {index}")
        for name in opt._state_names:
            assert_bits_or_nan(opt.state[a][name].cpu(), own_opt.state[b][name].cpu(), f"{name} {index}")
