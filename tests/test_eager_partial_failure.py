"""The reference-named optimizers stop at a bad parameter the way the reference's loop does.

The reference's ``_step_group`` consumes its lazy item walk one parameter at
a time (sr_states/optim/_state.py:154-182), so a sparse gradient, or a
DTensor parameter the walk refuses, raises only after every parameter ahead
of it in the group was updated and had its ``step`` recorded; the parameters
after it keep no state (tests/test_multi_tensor_tables.py:159-175).  The
optimizers under the reference's eager names run a group on the fused launch
when it takes the group, which collects the whole walk first; these tests
record the per-parameter updates (the launch itself needs a GPU and is
covered by tests/test_gpu_partial_failure.py) and check that the calls,
their RNG keys and the recorded steps are the reference's.
"""

from __future__ import annotations

import pytest
import torch

from sr_states import AdamWReferenceRN, AdamWReferenceSR, SGDMReferenceRN, SGDMReferenceSR

from oracle import sr_oracle

OPTIMIZERS = [AdamWReferenceSR, AdamWReferenceRN, SGDMReferenceSR, SGDMReferenceRN]


def _recording(cls, calls):
    class Recorder(cls):
        def _step_parameter(self, parameter, state, group, formats, step, seed, offset):
            calls.append((parameter, step, seed, offset))

    return Recorder


def _check(opt, calls, p, q, untouched):
    assert calls == [(p, 1, sr_oracle.update_key(7, 1, 0), 0), (q, 1, sr_oracle.update_key(3, 1, 2), 0)]
    assert opt._rng_step() == 1
    if opt._uses_step:
        assert opt.state[p]["step"] == opt.state[q]["step"] == 1
    else:
        assert "step" not in opt.state[p] and "step" not in opt.state[q]
    for parameter in untouched:
        assert parameter not in opt.state


@pytest.mark.parametrize("cls", OPTIMIZERS)
def test_sparse_gradient_raises_after_the_parameters_ahead_of_it(cls):
    calls = []
    p, skipped, q, bad, after = [torch.nn.Parameter(torch.ones(2)) for _ in range(5)]
    opt = _recording(cls, calls)(
        [{"params": [p, skipped], "sr_seed": 7}, {"params": [q, bad, after]}], lr=0.1, seed=3
    )
    p.grad = q.grad = after.grad = torch.ones(2)
    bad.grad = torch.sparse_coo_tensor([[0]], [1.0], (2,), check_invariants=True)
    with pytest.raises(RuntimeError, match="does not support sparse gradients"):
        opt.step()
    _check(opt, calls, p, q, (skipped, bad, after))


@pytest.mark.parametrize("cls", OPTIMIZERS)
def test_unsupported_dtensor_placement_raises_after_the_parameters_ahead_of_it(cls):
    pytest.importorskip("torch.distributed.tensor")
    from torch.distributed.device_mesh import DeviceMesh
    from torch.distributed.tensor import DTensor, Partial

    mesh = DeviceMesh("cpu", torch.arange(2), mesh_dim_names=("partial_failure",),
                      _init_backend=False, _rank=0)
    calls = []
    p, skipped, q, after = [torch.nn.Parameter(torch.ones(2)) for _ in range(4)]
    bad = torch.nn.Parameter(DTensor.from_local(torch.zeros(4, 3), mesh, (Partial(),), run_check=False,
                                                shape=(4, 3), stride=(3, 1)))
    bad.grad = DTensor.from_local(torch.ones(4, 3), mesh, (Partial(),), run_check=False,
                                  shape=(4, 3), stride=(3, 1))
    opt = _recording(cls, calls)(
        [{"params": [p, skipped], "sr_seed": 7}, {"params": [q, bad, after]}], lr=0.1, seed=3
    )
    p.grad = q.grad = after.grad = torch.ones(2)
    with pytest.raises(NotImplementedError, match="Shard and Replicate"):
        opt.step()
    _check(opt, calls, p, q, (skipped, bad, after))
