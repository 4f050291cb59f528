"""Placement of states in shared allocations (sr_states/optim/_state.py), on the CPU.

``_shared_zeros`` lays consecutive states out in zeroed allocations, each
view on a 512-byte boundary, starting a new allocation when the next state
would take one past ``_SHARED_MAX_BYTES`` (a state larger than that alone
gets one of its own).  ``_shareable`` admits only plain contiguous GPU
tensors, so CPU parameters, as in the reference, get an allocation each.
With it widened to CPU tensors, the optimizers' bookkeeping: one walk's
states share an allocation per name, a walk stopped at a refused parameter
leaves the later ones stateless, and checkpoints load into shared views.
"""

from __future__ import annotations

import pytest
import torch

from sr_states.optim import _state


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float8_e4m3fn])
def test_views_are_aligned_disjoint_and_zero(dtype):
    sizes = (1, 100, 255, 256, 257, 4099, 7)
    params = [torch.empty(n) for n in sizes]
    places = _state._shared_zeros(params, dtype, "cpu")
    assert len({id(slab) for slab, _ in places}) == 1
    itemsize = torch.empty((), dtype=dtype).element_size()
    spans = []
    for p, (slab, offset) in zip(params, places):
        view = _state._view(slab, offset, p)
        assert view.shape == p.shape and view.dtype == dtype
        assert (offset * itemsize) % 512 == 0
        assert torch.count_nonzero(view.float()) == 0
        spans.append((offset, offset + p.numel()))
    assert all(end <= start for (_, end), (start, _) in zip(spans, spans[1:]))


def test_allocations_split_at_the_limit(monkeypatch):
    monkeypatch.setattr(_state, "_SHARED_MAX_BYTES", 4096)  # 2048 BF16 elements
    params = [torch.empty(n) for n in (100, 1000, 500, 3000, 10, 10)]
    places = _state._shared_zeros(params, torch.bfloat16, "cpu")
    groups = [id(slab) for slab, _ in places]
    # 256 + 1024 + 512 = 1792 fit; 3000 elements exceed the limit alone; 10, 10 share.
    assert groups[0] == groups[1] == groups[2]
    assert len({groups[2], groups[3], groups[4]}) == 3
    assert groups[4] == groups[5]
    assert places[3][0].numel() == 3072


def test_only_contiguous_gpu_tensors_share():
    assert not _state._shareable(torch.empty(8))  # CPU, as in the reference
    assert not _state._shareable(torch.empty(0))


# The optimizers' bookkeeping, on the CPU: _shareable is widened to CPU
# tensors and the update itself is recorded instead of launched (the same
# walk runs on the GPU in tests/test_gpu_shared_states.py).

from sr_states import AdamWReferenceSR, SGDMReferenceSR  # noqa: E402


@pytest.fixture
def cpu_shareable(monkeypatch):
    monkeypatch.setattr(
        _state, "_shareable",
        lambda p: isinstance(p, torch.Tensor) and p.numel() > 0 and p.is_contiguous(),
    )


def _recorder(cls, calls):
    class Recorder(cls):
        def _step_parameter(self, parameter, state, group, formats, step, seed, offset):
            calls.append(parameter)

    return Recorder


def _storage(t):
    return t.untyped_storage().data_ptr()


@pytest.mark.parametrize("cls", [AdamWReferenceSR, SGDMReferenceSR])
def test_one_walk_shares_an_allocation_per_state_name(cpu_shareable, cls):
    calls = []
    a, b, c, d = (torch.nn.Parameter(torch.ones(n)) for n in (3, 5, 700, 1))
    opt = _recorder(cls, calls)([a, b, c, d], lr=0.1)
    a.grad, c.grad, d.grad = torch.ones(3), torch.ones(700), torch.ones(1)
    opt.step()
    assert calls == [a, c, d]
    assert b not in opt.state
    for name in opt._state_names:
        views = [opt.state[p][name] for p in (a, c, d)]
        assert len({_storage(v) for v in views}) == 1
        base = _storage(views[0])
        offsets = sorted(v.data_ptr() - base for v in views)
        assert all(o % 512 == 0 for o in offsets)
        assert all(v.shape == p.shape and not v.any() for v, p in zip(views, (a, c, d)))
    if len(opt._state_names) == 2:
        first, second = opt._state_names
        assert _storage(opt.state[a][first]) != _storage(opt.state[a][second])
    # A gradient that appears later: a fresh allocation, and nothing reserved for it earlier.
    b.grad = torch.ones(5)
    opt.step()
    for name in opt._state_names:
        assert _storage(opt.state[b][name]) != _storage(opt.state[a][name])


def test_a_walk_stopped_early_leaves_the_later_parameters_stateless(cpu_shareable):
    calls = []
    a, c, bad, e = (torch.nn.Parameter(torch.ones(4)) for _ in range(4))
    opt = _recorder(AdamWReferenceSR, calls)([a, c, bad, e], lr=0.1)
    a.grad = c.grad = e.grad = torch.ones(4)
    bad.grad = torch.sparse_coo_tensor([[0]], [1.0], (4,))
    with pytest.raises(RuntimeError, match="sparse"):
        opt.step()
    assert calls == [a, c]
    assert bad not in opt.state and e not in opt.state
    assert _storage(opt.state[a]["exp_avg"]) == _storage(opt.state[c]["exp_avg"])
    # The next step drops the reservation: e's states come from a new allocation.
    bad.grad = torch.ones(4)
    opt.step()
    assert calls[2:] == [a, c, bad, e]
    assert _storage(opt.state[e]["exp_avg"]) == _storage(opt.state[bad]["exp_avg"])
    assert _storage(opt.state[e]["exp_avg"]) != _storage(opt.state[a]["exp_avg"])


def test_separate_allocations_when_sharing_is_off(cpu_shareable):
    calls = []
    a, c = (torch.nn.Parameter(torch.ones(4)) for _ in range(2))
    opt = _recorder(AdamWReferenceSR, calls)([a, c], lr=0.1)
    opt._shared_state_allocations = False
    a.grad = c.grad = torch.ones(4)
    opt.step()
    assert _storage(opt.state[a]["exp_avg"]) != _storage(opt.state[c]["exp_avg"])


def test_a_checkpoint_loads_into_shared_views(cpu_shareable):
    calls = []
    params = [torch.nn.Parameter(torch.ones(n)) for n in (3, 1000, 17)]
    opt = _recorder(AdamWReferenceSR, calls)(params, lr=0.1)
    opt._shared_state_allocations = False
    for p in params:
        p.grad = torch.ones_like(p)
    opt.step()
    for k, p in enumerate(params):
        for j, name in enumerate(opt._state_names):
            opt.state[p][name].copy_(torch.arange(p.numel()) * (k + 1) + j)
    saved = opt.state_dict()
    fresh = [torch.nn.Parameter(torch.ones_like(p)) for p in params]
    restored = _recorder(AdamWReferenceSR, [])(fresh, lr=0.1)
    restored.load_state_dict(saved)
    for name in restored._state_names:
        assert len({_storage(restored.state[p][name]) for p in fresh}) == 1
    for k, (p, q) in enumerate(zip(params, fresh)):
        for name in opt._state_names:
            assert torch.equal(restored.state[q][name].view(torch.int16), opt.state[p][name].view(torch.int16))
            assert restored.state[q][name].data_ptr() != opt.state[p][name].data_ptr()
        assert restored.state[q]["step"] == 1
