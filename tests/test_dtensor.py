"""DTensor parameters: the shard start of a rank's local shard (host logic, CPU).

The reference refuses DTensor parameters (sr_states/optim/_state.py:148-152);
this backend accepts those whose local shard is one contiguous range of the
flattened parameter (FSDP2's Shard(0), and any Shard/Replicate placements
that give such ranges) and starts the shard's random stream at that range's
first flat index.  Ranks are simulated in one process: a DeviceMesh built
with ``_rank`` and no process group has that rank's coordinates, which is all
``DTensor.from_local`` and the shard computation read.

The shard starts are pinned by the data: the whole parameter holds its own
flat indices, each rank's local shard is cut from it with torch.chunk (the
split FSDP2 and DTensor's Shard use), and the shard must read
``shard_start, shard_start + 1, ...``.  The contiguity rule is checked
against brute force over every block of small shapes.
"""

from __future__ import annotations

import itertools

import numpy as np
import pytest
import torch

pytest.importorskip("torch.distributed.tensor")
from torch.distributed.device_mesh import DeviceMesh  # noqa: E402
from torch.distributed.tensor import DTensor, Partial, Replicate, Shard  # noqa: E402

from sr_states import AdamWHip, SGDMHip, hip_adamw_step_  # noqa: E402
from sr_states.optim._dtensor import flat_range_start, shard_start  # noqa: E402


def _mesh(shape, rank, device="cpu"):
    """The mesh as rank ``rank`` sees it.

    Meshes compare equal whatever rank they were built for, and DTensor
    caches sharding decisions (output specs, with their mesh) by mesh: one
    process playing several ranks names each rank's mesh dimensions apart
    so that no rank is handed another's mesh.
    """
    ranks = torch.arange(int(np.prod(shape))).reshape(shape)
    names = tuple(f"rank{rank}_dim{i}" for i in range(len(shape)))
    return DeviceMesh(device, ranks, mesh_dim_names=names, _init_backend=False, _rank=rank)


def _local_block(full, mesh_shape, coordinate, placements):
    """The local shard of ``full``: torch.chunk along each sharded dim, mesh dim by mesh dim."""
    block = full
    for size, index, placement in zip(mesh_shape, coordinate, placements):
        if isinstance(placement, Shard):
            chunks = torch.chunk(block, size, dim=placement.dim)
            if index < len(chunks):
                block = chunks[index]
            else:
                empty = list(block.shape)
                empty[placement.dim] = 0
                block = block.new_empty(empty)
    return block.contiguous()


def _dtensor(full, mesh, placements):
    local = _local_block(full, tuple(mesh.shape), mesh.get_coordinate(), placements)
    return DTensor.from_local(local, mesh, placements, run_check=False, shape=full.shape,
                              stride=full.stride())


def test_flat_range_start_matches_brute_force():
    """Every block of every shape up to 3x3x3 (and the empty extents)."""
    for rank in range(4):
        for shape in itertools.product(range(4), repeat=rank):
            flat = np.arange(int(np.prod(shape))).reshape(shape)
            ranges = [[(o, e) for o in range(n + 1) for e in range(n - o + 1)] for n in shape]
            for block in itertools.product(*ranges):
                offset, extent = zip(*block) if block else ((), ())
                picked = flat[tuple(slice(o, o + e) for o, e in block)].reshape(-1)
                got = flat_range_start(shape, extent, offset)
                if picked.size == 0:
                    assert got == 0
                elif np.array_equal(picked, np.arange(picked[0], picked[0] + picked.size)):
                    assert got == picked[0], (shape, block)
                else:
                    assert got is None, (shape, block)


CASES = [
    # (mesh shape, placements, parameter shape)
    ((2,), (Shard(0),), (7, 3)),
    ((3,), (Shard(0),), (10,)),
    ((4,), (Shard(0),), (3, 5)),  # rank 3 holds no rows
    ((4,), (Shard(0),), (5, 2, 3)),  # chunks of 2, 2, 1 and an empty one
    ((2,), (Replicate(),), (4, 4)),
    ((2, 2), (Shard(0), Shard(0)), (9, 4)),
    ((2, 2), (Replicate(), Shard(0)), (5, 4)),
    ((2, 2), (Shard(0), Replicate()), (5, 4)),
    ((2,), (Shard(1),), (1, 9)),  # only dim 1 has extent: still flat ranges
    ((2, 3), (Shard(0), Shard(1)), (4, 1, 6)),  # dim 1 of extent 1 never splits
]


@pytest.mark.parametrize("mesh_shape, placements, shape", CASES)
def test_shard_start_is_the_first_flat_index_of_the_local_shard(mesh_shape, placements, shape):
    full = torch.arange(int(np.prod(shape)), dtype=torch.float64).reshape(shape)
    covered = []
    for rank in range(int(np.prod(mesh_shape))):
        mesh = _mesh(mesh_shape, rank)
        parameter = torch.nn.Parameter(_dtensor(full, mesh, placements))
        start = shard_start(parameter)
        local = parameter.to_local().reshape(-1)
        assert torch.equal(local, torch.arange(start, start + local.numel(), dtype=torch.float64))
        if all(isinstance(p, Shard) or c == 0 for p, c in zip(placements, mesh.get_coordinate())):
            covered.extend(local.tolist())  # one replica of every shard
    assert sorted(covered) == full.reshape(-1).tolist()


@pytest.mark.parametrize(
    "mesh_shape, placements, shape",
    [((2,), (Shard(1),), (3, 4)), ((2, 2), (Shard(0), Shard(1)), (4, 4)), ((2,), (Shard(2),), (2, 2, 6))],
)
def test_shards_that_are_not_one_flat_range_are_refused(mesh_shape, placements, shape):
    full = torch.zeros(shape)
    parameter = torch.nn.Parameter(_dtensor(full, _mesh(mesh_shape, 0), placements))
    with pytest.raises(NotImplementedError, match="one contiguous range"):
        shard_start(parameter)


def test_partial_and_strided_placements_are_refused():
    from torch.distributed.tensor.placement_types import _StridedShard

    mesh = _mesh((2,), 1)
    for placement in (Partial(), _StridedShard(0, split_factor=2)):
        value = DTensor.from_local(torch.zeros(4, 3), mesh, (placement,), run_check=False,
                                   shape=(8, 3), stride=(3, 1))
        with pytest.raises(NotImplementedError, match="Shard and Replicate"):
            shard_start(torch.nn.Parameter(value))


@pytest.mark.parametrize("optimizer", [AdamWHip, SGDMHip])
def test_optimizer_refuses_unsupported_placements_before_creating_state(optimizer):
    mesh = _mesh((2,), 0)
    p = torch.nn.Parameter(_dtensor(torch.zeros(4, 6), mesh, (Shard(1),)))
    p.grad = _dtensor(torch.ones(4, 6), mesh, (Shard(1),))
    opt = optimizer([p], lr=0.01)
    with pytest.raises(NotImplementedError, match="one contiguous range"):
        opt.step()
    assert p not in opt.state


@pytest.mark.parametrize("optimizer", [AdamWHip, SGDMHip])
def test_gradient_with_other_placements_is_refused(optimizer):
    mesh = _mesh((2,), 1)
    p = torch.nn.Parameter(_dtensor(torch.zeros(6, 2), mesh, (Shard(0),)))
    p.grad = DTensor.from_local(torch.ones(6, 2), mesh, (Partial(),), run_check=False)
    with pytest.raises(ValueError, match="must be DTensors with its mesh, placements"):
        optimizer([p], lr=0.01).step()


def test_cpu_dtensor_reaches_the_device_check():
    """A supported placement on CPU fails like any CPU tensor: there is no CPU path."""
    mesh = _mesh((2,), 1)
    p = torch.nn.Parameter(_dtensor(torch.zeros(6, 2), mesh, (Shard(0),)))
    p.grad = _dtensor(torch.ones(6, 2), mesh, (Shard(0),))
    with pytest.raises(ValueError, match="GPU tensors"):
        AdamWHip([p], lr=0.01).step()


def test_functional_update_takes_local_tensors():
    mesh = _mesh((2,), 0)
    p = _dtensor(torch.zeros(4), mesh, (Shard(0),))
    m = _dtensor(torch.zeros(4, dtype=torch.bfloat16), mesh, (Shard(0),))
    with pytest.raises(TypeError, match="to_local"):
        hip_adamw_step_(p, p.clone(), m, m.clone(), lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8,
                        weight_decay=0.0, step=1)


@pytest.mark.parametrize("update", ["adamw_step", "adamw_step_", "sgdm_step", "sgdm_step_"])
def test_reference_functional_updates_take_local_tensors(update):
    """sr_states.reference refuses DTensors as the fused single-tensor updates do."""
    import sr_states.reference as functional

    mesh = _mesh((2,), 1)
    p = _dtensor(torch.zeros(4), mesh, (Shard(0),))
    m = _dtensor(torch.zeros(4, dtype=torch.bfloat16), mesh, (Shard(0),))
    if update.startswith("adamw"):
        args = (p, p.clone(), m, m.clone())
        options = dict(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.0, step=1)
    else:
        args = (p, p.clone(), m)
        options = dict(lr=1e-3, momentum_factor=0.9)
    with pytest.raises(TypeError, match="to_local"):
        getattr(functional, update)(*args, **options)


def test_eager_optimizers_reach_the_device_check_with_cpu_dtensors():
    """AdamWReferenceSR takes DTensor parameters through their local shards; on CPU it stops there."""
    from sr_states import AdamWReferenceSR

    mesh = _mesh((2,), 0)
    p = torch.nn.Parameter(_dtensor(torch.zeros(6, 2), mesh, (Shard(0),)))
    p.grad = _dtensor(torch.ones(6, 2), mesh, (Shard(0),))
    with pytest.raises(ValueError, match="run on the GPU"):
        AdamWReferenceSR([p], lr=0.01).step()
