"""DTensor parameters on the device: every rank's update is the oracle's update of its slice.

A model's parameters are updated unsharded (plain tensors) and, for every
rank of several meshes, as DTensors holding that rank's shards.  Each local
parameter and state must equal, bit for bit, the C oracle's replay of the
same steps over the matching flat range, with the range's first flat index
as the counter offset: the random stream of an element depends only on its
flat index in the whole parameter (the reference's flat-split property,
tests/test_rng_streams.py:122-150, which its optimizers cannot use with
DTensors, sr_states/optim/_state.py:148-152).  The unsharded run is held to
the same oracle, and each shard also equals its slice of the unsharded run.

Ranks are simulated in one process on cuda:0: each rank's DeviceMesh is
built with ``_rank`` and no process group, so nothing is communicated; the
kernels see only the local shards.  Shapes leave uneven and empty shards.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from conftest import assert_bits_or_nan

pytest.importorskip("torch.distributed.tensor")
from torch.distributed.device_mesh import DeviceMesh  # noqa: E402
from torch.distributed.tensor import DTensor, Replicate, Shard  # noqa: E402

import sr_states  # noqa: E402
from oracle import c_oracle  # noqa: E402
from sr_states.optim._dtensor import shard_start  # noqa: E402

pytestmark = pytest.mark.gpu

SHAPES = [(7, 33), (130,), (5, 3, 17), (1,), (3, 1000), (2051,)]
MESHES = [
    ((2,), (Shard(0),)),
    ((3,), (Shard(0),)),
    ((4,), (Shard(0),)),
    ((2, 2), (Shard(0), Shard(0))),
    ((2, 2), (Replicate(), Shard(0))),
]
STEPS = 3


def _mesh(shape, rank):
    # Meshes compare equal whatever rank they were built for, and DTensor
    # caches sharding decisions by mesh: each simulated rank names its mesh
    # dimensions apart.
    ranks = torch.arange(int(np.prod(shape))).reshape(shape)
    names = tuple(f"rank{rank}_dim{i}" for i in range(len(shape)))
    return DeviceMesh("cuda", ranks, mesh_dim_names=names, _init_backend=False, _rank=rank)


def _shard(full, mesh, placements):
    """DTensor of ``full`` on ``mesh``: torch.chunk along each sharded dim (FSDP2's split)."""
    block = full
    for size, index, placement in zip(mesh.shape, mesh.get_coordinate(), placements):
        if isinstance(placement, Shard):
            chunks = torch.chunk(block, size, dim=placement.dim)
            if index < len(chunks):
                block = chunks[index]
            else:
                empty = list(block.shape)
                empty[placement.dim] = 0
                block = block.new_empty(empty)
    return DTensor.from_local(block.contiguous().clone(), mesh, placements, run_check=False,
                              shape=full.shape, stride=full.stride())


def _problem(cuda, seed, dtype=torch.float32):
    gen = torch.Generator(device=cuda).manual_seed(seed)
    params = [(torch.randn(shape, device=cuda, generator=gen) * 0.02).to(dtype) for shape in SHAPES]
    grads = [[(torch.randn(shape, device=cuda, generator=gen) * 1e-3).to(dtype) for shape in SHAPES]
             for _ in range(STEPS)]
    return params, grads


def _run(make, params, grads, wrap, checkpoint_after=None):
    """STEPS steps of ``make(parameters)``; ``wrap`` turns a full tensor into a parameter value."""
    parameters = [torch.nn.Parameter(wrap(p)) for p in params]
    optimizer = make(parameters)
    for step, step_grads in enumerate(grads, start=1):
        for parameter, g in zip(parameters, step_grads):
            parameter.grad = wrap(g)
        optimizer.step()
        if step == checkpoint_after:
            saved = optimizer.state_dict()
            optimizer = make(parameters)
            optimizer.load_state_dict(saved)
    return parameters, optimizer


def _replay(oracle, params, grads, index, start, stop):
    """The C oracle's STEPS updates of params[index]'s flat range [start, stop)."""
    p = params[index].reshape(-1)[start:stop].cpu().clone()
    states = [torch.zeros(stop - start, dtype=dtype) for dtype, _ in oracle["formats"]]
    for step, step_grads in enumerate(grads, start=1):
        g = step_grads[index].reshape(-1)[start:stop].cpu().clone()
        key = sr_states.update_key(oracle["seed"], step, index)
        oracle["update"](p, g, *states, step, key, start)
    return p, states


def _check_oracle(oracle, params, grads, index, start, local_p, local_states, label):
    stop = start + local_p.numel()
    if stop == start:
        return
    p, states = _replay(oracle, params, grads, index, start, stop)
    assert_bits_or_nan(local_p.reshape(-1).cpu(), p, f"{label}: parameter against the oracle")
    for k, (local, expected) in enumerate(zip(local_states, states)):
        assert_bits_or_nan(local.reshape(-1).cpu(), expected, f"{label}: state {k} against the oracle")


def _compare(full_params, full_opt, shard_params, shard_opt, names, what, oracle, params, grads, indices=None):
    """Each shard against its slice of the unsharded run and against the oracle.

    ``indices`` are the parameters' indices in ``params`` (default: their positions).
    """
    indices = range(len(shard_params)) if indices is None else indices
    for index, full, shard in zip(indices, full_params, shard_params):
        start = shard_start(shard)
        local = shard.to_local().reshape(-1)
        stop = start + local.numel()
        label = f"{what}, parameter {index} {tuple(full.shape)}, elements [{start}, {stop})"
        assert_bits_or_nan(local, full.detach().reshape(-1)[start:stop], f"{label}: parameter")
        full_state, shard_state = full_opt.state[full], shard_opt.state[shard]
        for name in names:
            stored = shard_state[name]
            assert isinstance(stored, DTensor) and stored.placements == shard.placements
            assert stored.dtype == full_state[name].dtype
            assert_bits_or_nan(stored.to_local().reshape(-1), full_state[name].reshape(-1)[start:stop],
                               f"{label}: {name}")
        assert shard_state.get("step") == full_state.get("step")
        _check_oracle(oracle, params, grads, index, start, local,
                      [shard_state[name].to_local() for name in names], label)


def _check_unsharded(full_params, full_opt, names, oracle, params, grads, what):
    for index, full in enumerate(full_params):
        _check_oracle(oracle, params, grads, index, 0, full.detach(),
                      [full_opt.state[full][name] for name in names], f"{what}, unsharded parameter {index}")


def _adamw_oracle(seed, formats):
    def update(p, g, m, v, step, key, offset):
        c_oracle.adamw_step_(p, g, m, v, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01,
                             step=step, formats=formats, seed=key, offset=offset)
    return {"seed": seed, "formats": formats, "update": update}


def _sgdm_oracle(seed, formats):
    def update(p, g, u, step, key, offset):
        c_oracle.sgdm_step_(p, g, u, lr=0.1, momentum_factor=0.9, formats=formats, seed=key, offset=offset)
    return {"seed": seed, "formats": formats, "update": update}


def _adamw_bf16_sr(parameters):
    return sr_states.AdamWHip(parameters, lr=1e-3, weight_decay=0.01, seed=11)


def _adamw_e4m3_bf16(parameters):
    formats = {"exp_avg": sr_states.StateFormat(torch.float8_e4m3fn),
               "exp_avg_sq": sr_states.StateFormat(torch.bfloat16)}
    return sr_states.AdamWHip(parameters, lr=1e-3, seed=12, state_format=formats)


def _sgdm_fp16_sr(parameters):
    return sr_states.SGDMHip(parameters, lr=0.1, state_dtype=torch.float16, seed=13)


def _adamw_reference_e4m3_bf16(parameters):
    """The eager per-parameter optimizer: one launch per local shard."""
    formats = {"exp_avg": sr_states.StateFormat(torch.float8_e4m3fn),
               "exp_avg_sq": sr_states.StateFormat(torch.bfloat16)}
    return sr_states.AdamWReferenceSR(parameters, lr=1e-3, seed=14, state_format=formats)


def _sgdm_reference_fp16_sr(parameters):
    return sr_states.SGDMReferenceSR(parameters, lr=0.1, state_dtype=torch.float16, seed=15)


OPTIMIZERS = {
    "adamw_bf16_sr": (_adamw_bf16_sr, ("exp_avg", "exp_avg_sq"),
                      _adamw_oracle(11, [(torch.bfloat16, "stochastic")] * 2)),
    "adamw_reference_e4m3_bf16": (_adamw_reference_e4m3_bf16, ("exp_avg", "exp_avg_sq"),
                                  _adamw_oracle(14, [(torch.float8_e4m3fn, "stochastic"),
                                                     (torch.bfloat16, "stochastic")])),
    "sgdm_reference_fp16_sr": (_sgdm_reference_fp16_sr, ("momentum_buffer",),
                               _sgdm_oracle(15, [(torch.float16, "stochastic")])),
    "adamw_e4m3_bf16": (_adamw_e4m3_bf16, ("exp_avg", "exp_avg_sq"),
                        _adamw_oracle(12, [(torch.float8_e4m3fn, "stochastic"), (torch.bfloat16, "stochastic")])),
    "sgdm_fp16_sr": (_sgdm_fp16_sr, ("momentum_buffer",), _sgdm_oracle(13, [(torch.float16, "stochastic")])),
}


@pytest.mark.parametrize("mesh_shape, placements", MESHES)
@pytest.mark.parametrize("kind", list(OPTIMIZERS))
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_optimizers_update_each_shard_as_its_slice_of_the_whole(cuda, kind, mesh_shape, placements, dtype):
    make, names, oracle = OPTIMIZERS[kind]
    params, grads = _problem(cuda, seed=len(kind) + len(mesh_shape), dtype=dtype)
    full_params, full_opt = _run(make, params, grads, lambda t: t.clone())
    torch.cuda.synchronize()
    _check_unsharded(full_params, full_opt, names, oracle, params, grads, kind)
    for rank in range(int(np.prod(mesh_shape))):
        mesh = _mesh(mesh_shape, rank)
        shard_params, shard_opt = _run(make, params, grads, lambda t: _shard(t, mesh, placements),
                                       checkpoint_after=2)
        torch.cuda.synchronize()
        _compare(full_params, full_opt, shard_params, shard_opt, names, f"{kind} rank {rank}", oracle,
                 params, grads)


def test_per_parameter_path_updates_each_shard_as_its_slice_of_the_whole(cuda):
    """StateOptimizer._compute subclasses store states through sr_states.cast with the shard start."""

    class SignMomentum(sr_states.StateOptimizer):
        _state_names = ("momentum_buffer",)
        _uses_step = False

        def __init__(self, params):
            super().__init__(params, {"lr": 0.01}, state_dtype=torch.bfloat16, seed=21)

        def _compute(self, p32, g32, states32, group, step):
            buffer = states32[0] * 0.9 + g32
            return p32 - group["lr"] * torch.sign(buffer), (buffer,)

    def update(p, g, u, step, key, offset):
        # The same torch operations on the CPU, and the C oracle's cast.
        buffer = u.float() * 0.9 + g
        p.copy_(p - 0.01 * torch.sign(buffer))
        u.copy_(c_oracle.cast(buffer, dtype=torch.bfloat16, rounding="stochastic",
                              seed=sr_states.state_key(key, 0), offset=offset))

    oracle = {"seed": 21, "formats": [(torch.bfloat16, "stochastic")], "update": update}
    params, grads = _problem(cuda, seed=3)
    full_params, full_opt = _run(SignMomentum, params, grads, lambda t: t.clone())
    torch.cuda.synchronize()
    _check_unsharded(full_params, full_opt, ("momentum_buffer",), oracle, params, grads, "sign momentum")
    mesh_shape, placements = (3,), (Shard(0),)
    for rank in range(3):
        mesh = _mesh(mesh_shape, rank)
        shard_params, shard_opt = _run(SignMomentum, params, grads, lambda t: _shard(t, mesh, placements))
        torch.cuda.synchronize()
        _compare(full_params, full_opt, shard_params, shard_opt, ("momentum_buffer",), f"rank {rank}", oracle,
                 params, grads)


def test_groups_mixing_dtensor_and_plain_parameters(cuda):
    """One group holding sharded and replicated-as-plain parameters: one launch covers both kinds."""
    params, grads = _problem(cuda, seed=17)
    full_params, full_opt = _run(_adamw_bf16_sr, params, grads, lambda t: t.clone())
    mesh_shape, placements = (3,), (Shard(0),)
    for rank in range(3):
        mesh = _mesh(mesh_shape, rank)
        # Even-indexed parameters sharded, odd ones whole plain tensors.
        wraps = [(lambda t: _shard(t, mesh, placements)) if k % 2 == 0 else (lambda t: t.clone())
                 for k in range(len(params))]
        parameters = [torch.nn.Parameter(wrap(p)) for wrap, p in zip(wraps, params)]
        opt = _adamw_bf16_sr(parameters)
        for step_grads in grads:
            for parameter, wrap, g in zip(parameters, wraps, step_grads):
                parameter.grad = wrap(g)
            opt.step()
        torch.cuda.synchronize()
        oracle, names = OPTIMIZERS["adamw_bf16_sr"][2], ("exp_avg", "exp_avg_sq")
        for k, (full, mixed) in enumerate(zip(full_params, parameters)):
            if k % 2 == 0:
                _compare([full], full_opt, [mixed], opt, names, f"rank {rank}", oracle, params, grads,
                         indices=[k])
            else:
                assert_bits_or_nan(mixed.detach(), full.detach(), f"rank {rank}, plain parameter {k}")
                for name in names:
                    assert_bits_or_nan(opt.state[mixed][name], full_opt.state[full][name], f"{name} {k}")
                _check_oracle(oracle, params, grads, k, 0, mixed.detach(),
                              [opt.state[mixed][name] for name in names], f"rank {rank}, plain parameter {k}")


def test_plain_and_dtensor_parameters_share_one_group(cuda):
    """A group mixing plain parameters and rank 0's shards of DTensor ones: the plain
    parameters' states share one allocation per name, the DTensor states stay DTensors
    of their own, and every parameter and state equals the C oracle's update."""
    params, grads = _problem(cuda, 21)
    mesh = _mesh((2,), 0)
    sharded = {1, 4}

    def wrap(index, tensor):
        return _shard(tensor, mesh, (Shard(0),)) if index in sharded else tensor.clone()

    parameters = [torch.nn.Parameter(wrap(i, p)) for i, p in enumerate(params)]
    optimizer = sr_states.AdamWHip(parameters, lr=1e-3, weight_decay=0.01, seed=11)
    for step_grads in grads:
        for i, (parameter, g) in enumerate(zip(parameters, step_grads)):
            parameter.grad = wrap(i, g)
        optimizer.step()
    torch.cuda.synchronize()
    names = ("exp_avg", "exp_avg_sq")
    oracle = _adamw_oracle(11, [(torch.bfloat16, "stochastic")] * 2)
    plain = [p for i, p in enumerate(parameters) if i not in sharded]
    for name in names:
        assert len({optimizer.state[p][name].untyped_storage().data_ptr() for p in plain}) == 1
    for i, parameter in enumerate(parameters):
        states = [optimizer.state[parameter][name] for name in names]
        if i in sharded:
            assert all(isinstance(s, DTensor) for s in states)
            _check_oracle(oracle, params, grads, i, shard_start(parameter), parameter.to_local(),
                          [s.to_local() for s in states], f"DTensor parameter {i}")
        else:
            _check_oracle(oracle, params, grads, i, 0, parameter.detach(), states, f"plain parameter {i}")
