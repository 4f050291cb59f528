"""A bad parameter mid-group: the reference-named optimizers update the ones ahead of it first.

The reference's lazy loop (sr_states/optim/_state.py:154-182) updates every
parameter ahead of a sparse gradient, or of a DTensor parameter its walk
refuses, records their ``step`` and then raises; the parameters after it
keep no state (tests/test_multi_tensor_tables.py:159-175).  Here the first
group runs on the fused launch and the second, [a dense, b without a
gradient, c dense, d bad, e dense], meets ``d``.  Every updated parameter
and state must equal, byte for byte, the C oracle's update with the key the
reference gives it; ``b``, ``d`` and ``e`` must be untouched and stateless.
"""

from __future__ import annotations

import pytest
import torch
from conftest import assert_bits_or_nan

from sr_states import AdamWReferenceRN, AdamWReferenceSR, SGDMReferenceRN, SGDMReferenceSR
from oracle import c_oracle, sr_oracle

pytestmark = pytest.mark.gpu

SIZES = (4099, 6144, 257, 1000, 3001, 12, 77)  # group 1: two; group 2: a, b, c, d, e
CASES = [
    (AdamWReferenceSR, "stochastic"),
    (AdamWReferenceRN, "nearest"),
    (SGDMReferenceSR, "stochastic"),
    (SGDMReferenceRN, "nearest"),
]


def _oracle_update(cls, rule, p, g, key):
    """The oracle's first step of one parameter from zero states: (p, *states) on the CPU."""
    p = p.detach().cpu().clone()
    g = g.detach().cpu()
    if issubclass(cls, AdamWReferenceSR):
        m, v = (torch.zeros(p.shape, dtype=torch.bfloat16) for _ in range(2))
        c_oracle.adamw_step_(p, g, m, v, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01,
                             step=1, formats=((torch.bfloat16, rule),) * 2, seed=key)
        return p, m, v
    u = torch.zeros(p.shape, dtype=torch.bfloat16)
    c_oracle.sgdm_step_(p, g, u, lr=0.1, momentum_factor=0.9, formats=((torch.bfloat16, rule),), seed=key)
    return p, u


def _run(cls, rule, cuda, make_bad, error, match):
    gen = torch.Generator().manual_seed(5)
    params = [torch.nn.Parameter((torch.randn(n, generator=gen) * 0.02).to(cuda)) for n in SIZES]
    for index, p in enumerate(params):
        if index != 3:  # b has no gradient
            p.grad = (torch.randn(p.shape, generator=gen) * 1e-3).to(cuda)
    params[5] = make_bad(cuda)
    initial = [p.detach().clone() for p in params]
    lr = 1e-3 if issubclass(cls, AdamWReferenceSR) else 0.1
    opt = cls([{"params": params[:2], "sr_seed": 7}, {"params": params[2:]}], lr=lr, seed=3)
    with pytest.raises(error, match=match):
        opt.step()
    torch.cuda.synchronize()
    assert opt._rng_step() == 1
    for index in (0, 1, 2, 4):
        p = params[index]
        key = sr_oracle.update_key(7 if index < 2 else 3, 1, index)
        want = _oracle_update(cls, rule, initial[index], p.grad, key)
        state = opt.state[p]
        got = (p.detach(), *(state[name] for name in opt._state_names))
        for name, a, b in zip(("param",) + opt._state_names, got, want):
            assert_bits_or_nan(a, b, f"{cls.__name__} parameter {index} {name}")
        if opt._uses_step:
            assert state["step"] == 1
        else:
            assert "step" not in state
    for index in (3, 5, 6):
        assert params[index] not in opt.state, index
        assert torch.equal(_local(params[index].detach()), _local(initial[index])), index


def _local(tensor):
    return getattr(tensor, "_local_tensor", tensor)


def _sparse(cuda):
    bad = torch.nn.Parameter(torch.ones(2, device=cuda))
    bad.grad = torch.sparse_coo_tensor([[0]], [1.0], (2,), device=cuda, check_invariants=True)
    return bad


@pytest.mark.parametrize("cls, rule", CASES)
def test_sparse_gradient_mid_group(cuda, cls, rule):
    _run(cls, rule, cuda, _sparse, RuntimeError, "does not support sparse gradients")


@pytest.mark.parametrize("cls, rule", CASES)
def test_unsupported_dtensor_placement_mid_group(cuda, cls, rule):
    pytest.importorskip("torch.distributed.tensor")
    from torch.distributed.device_mesh import DeviceMesh
    from torch.distributed.tensor import DTensor, Partial

    def partial(device):
        mesh = DeviceMesh("cuda", torch.arange(2), mesh_dim_names=("partial_failure_gpu",),
                          _init_backend=False, _rank=0)
        local = dict(shape=(4, 3), stride=(3, 1), run_check=False)
        bad = torch.nn.Parameter(DTensor.from_local(torch.zeros(4, 3, device=device), mesh, (Partial(),), **local))
        bad.grad = DTensor.from_local(torch.ones(4, 3, device=device), mesh, (Partial(),), **local)
        return bad

    _run(cls, rule, cuda, partial, NotImplementedError, "Shard and Replicate")
