"""DTensor parameters: the flat index at which a rank's local shard starts.

The reference refuses DTensor parameters (sr_states/optim/_state.py:148-152)
and starts every update at flat index 0.  An element's random bits depend
only on its flat index within the whole parameter: the counter is
``idx + shard_start`` (sr_states/triton/adamw.py:50-52,
sr_states/triton/sgd.py:41).  So a rank whose local shard is the range
[s, s + n) of the flattened parameter, updated with ``shard_start = s``,
stores exactly the bytes the unsharded update stores for that range; the
reference's tests check this for flat splits (tests/test_rng_streams.py:
122-150).  FSDP2 shards parameters along dim 0 (``Shard(0)``), which gives
such ranges.  This module computes ``s`` and refuses placements whose local
shard is not one contiguous range of the flattened parameter.
"""

from __future__ import annotations

import math

import torch

if torch.distributed.is_available():
    from torch.distributed.tensor import DTensor, Replicate, Shard
    from torch.distributed.tensor._utils import compute_local_shape_and_global_offset
else:  # pragma: no cover
    DTensor = None


def is_dtensor(tensor) -> bool:
    return DTensor is not None and isinstance(tensor, DTensor)


def _row_major_strides(shape):
    strides, running = [], 1
    for size in reversed(shape):
        strides.append(running)
        running *= size
    return tuple(reversed(strides))


def flat_range_start(shape, local_shape, offset) -> int | None:
    """Flat start of the block ``offset + [0, local_shape)`` of a row-major ``shape``.

    None when the block is not one contiguous range of the flattened tensor:
    that holds when, before the last dimension the block cuts short (every
    later one is whole), every dimension has extent one.  An empty block
    starts at 0.
    """
    if math.prod(local_shape) == 0:
        return 0
    cut = len(shape)
    while cut > 0 and local_shape[cut - 1] == shape[cut - 1]:
        cut -= 1
    if any(extent != 1 for extent in local_shape[: max(cut - 1, 0)]):
        return None
    return sum(o * s for o, s in zip(offset, _row_major_strides(shape)))


# Each DTensor parameter keeps (its DTensorSpec when computed, shard start)
# in this attribute.  A DTensor's spec object is replaced whenever its mesh,
# placements or shape change, so an identical spec means an identical shard
# start.  Computing one costs about 55 us (torch's
# compute_local_shape_and_global_offset); reading a kept one well under
# 1 us, every step.  (Tensors compare elementwise, so a weak dictionary
# keyed by parameter cannot hold these.)
_START_ATTRIBUTE = "_sr_states_shard_start"


def shard_start(parameter) -> int:
    """Flat index, within the whole parameter, of the local shard's first element."""
    spec = parameter._spec
    kept = getattr(parameter, _START_ATTRIBUTE, None)
    if kept is not None and kept[0] is spec:
        return kept[1]
    start = _compute_shard_start(parameter)
    setattr(parameter, _START_ATTRIBUTE, (spec, start))
    return start


def _compute_shard_start(parameter) -> int:
    placements = tuple(parameter.placements)
    for placement in placements:
        # _StridedShard (FSDP2 with tensor parallelism) subclasses Shard and
        # interleaves ranks, so only these two exact types are accepted.
        if type(placement) not in (Shard, Replicate):
            raise NotImplementedError(
                "DTensor optimizer parameters support Shard and Replicate placements, "
                f"not {placement}"
            )
    shape = tuple(parameter.shape)
    row_major = _row_major_strides(shape)
    if any(size > 1 and st != want for size, st, want in zip(shape, parameter.stride(), row_major)):
        raise NotImplementedError("DTensor optimizer parameters must be contiguous")
    local_shape, offset = compute_local_shape_and_global_offset(
        shape, parameter.device_mesh, placements
    )
    if tuple(parameter.to_local().shape) != tuple(local_shape):
        raise ValueError(
            f"local shard of shape {tuple(parameter.to_local().shape)} does not match "
            f"the {tuple(local_shape)} block its placements {placements} give"
        )
    start = flat_range_start(shape, tuple(local_shape), tuple(offset))
    if start is None:
        raise NotImplementedError(
            "DTensor optimizer parameters need local shards that are one contiguous range "
            f"of the flattened parameter; placements {placements} cut shape {shape} "
            f"into {tuple(local_shape)} blocks"
        )
    return start


def local_tensors(parameter, tensors):
    """The local shards of ``tensors`` (the parameter, its gradient, its states).

    A DTensor parameter's gradient and states must be DTensors with its
    mesh, placements and shape; a plain parameter's must be plain tensors.
    The shards are the DTensors' ``_local_tensor`` storage itself (what
    ``to_local()`` returns a view of, without its autograd bookkeeping: the
    updates run under no_grad and write in place).
    """
    if not is_dtensor(parameter):
        if any(is_dtensor(t) for t in tensors):
            raise TypeError("a plain tensor parameter needs plain tensor gradients and states")
        return tuple(tensors)
    spec = parameter._spec
    local = []
    for tensor in tensors:
        if not (
            is_dtensor(tensor)
            and (
                tensor._spec is spec
                or (
                    tensor._spec.mesh == spec.mesh
                    and tensor._spec.placements == spec.placements
                    and tensor.shape == parameter.shape
                )
            )
        ):
            raise ValueError(
                "a DTensor parameter's gradient and states must be DTensors with its mesh, "
                f"placements {tuple(parameter.placements)} and shape {tuple(parameter.shape)}"
            )
        local.append(tensor._local_tensor)
    return tuple(local)
