"""Placement of states in shared allocations (sr_states/optim/_state.py), on the CPU.

``_shared_zeros`` lays consecutive states out in zeroed allocations, each
view on a 512-byte boundary, starting a new allocation when the next state
would take one past ``_SHARED_MAX_BYTES`` (a state larger than that alone
gets one of its own).  ``_shareable`` admits only plain contiguous GPU
tensors, so CPU parameters, as in the reference, get an allocation each.
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
