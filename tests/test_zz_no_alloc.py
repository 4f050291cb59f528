"""sr_adamw_multi_noalloc, the entry point that allocates nothing, against sr_adamw_multi.

Both entry points run the same buckets through the C ABI on identical
copies of the tensors: sr_adamw_multi with row tables uploaded to device
memory, sr_adamw_multi_noalloc with the same tables in host memory, which the
library stages in its static device scratch.  Parameters and states must be
identical byte for byte on two calls in a row, the second with fewer rows and
tiles (and per-row step scalars), so stale scratch contents from the first
call would show.  Oversized and malformed tables are refused on the host
before any device work, leaving every tensor unchanged.

The first call's bucket, and the captured one, pass 2^16 tiles, so their
FP32-parameter launches run with the resident-workgroup cap.  Under HIP
graph capture the entry takes pinned host tables: a captured call is
replayed three times, each time from the same initial tensors and after
an eager call on other tables has overwritten the scratch, and every replay
must equal the eager sr_adamw_multi step.  Pageable tables are refused under
capture before anything is recorded.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch
from conftest import assert_bits_or_nan

from sr_states import _lib
from sr_states.hip._multi_tensor import build_records, build_tile_rows, tile_elements, upload
from sr_states.optim.adamw import adamw_hparams

pytestmark = pytest.mark.gpu

BLOCK = 128
SEED, RNG_STEP = 0xFEDCBA9876543210, (1 << 32) + 3
HYPER = {"lr": 1e-3, "beta1": 0.9, "beta2": 0.999, "eps": 1e-8, "weight_decay": 0.01}


def _bucket(cuda, sizes, dtypes, seed):
    """(p, g, m, v) per row; a negative size makes an unaligned view of that many elements."""
    gen = torch.Generator(device=cuda).manual_seed(seed)
    rows = []
    for size in sizes:
        n, skip = abs(size), (1 if size < 0 else 0)
        scale = (1.0, 0.1, 0.01, 0.01)
        row = []
        for k, dtype in enumerate(dtypes):
            full = torch.randn(n + skip, device=cuda, generator=gen) * scale[k]
            if k == 3:
                full = full.abs() + 1e-4
            row.append(full.to(dtype)[skip:])
        rows.append(row)
    return rows


def _tables(rows, first_index):
    dtypes = tuple(t.dtype for t in rows[0])
    tile = tile_elements(BLOCK, dtypes)
    layout = [(row[0].numel(), first_index + k, 0) for k, row in enumerate(rows)]
    pointers = [tuple(t.data_ptr() for t in row) for row in rows]
    return build_records(layout, pointers, tile), build_tile_rows(layout, tile)


def _row_scalars(steps):
    values = []
    for step in steps:
        hp = adamw_hparams(HYPER["lr"], HYPER["beta1"], HYPER["beta2"], HYPER["eps"], HYPER["weight_decay"], step)
        values += [hp.neg_step_size, hp.correction2_sqrt]
    return np.array(values, dtype=np.float32)


def _codes(rows, formats):
    (m_rule, v_rule) = (_lib.RULE_CODES[r] for _, r in formats)
    p, g, m, v = (_lib.DTYPE_CODES[t.dtype] for t in rows[0])
    return p, g, m, m_rule, v, v_rule


def _launch_device_tables(cuda, rows, formats, records, tile_rows, scalars, step):
    lib = _lib.library()
    rows_dev = upload(records, cuda)
    tiles_dev = upload(tile_rows, cuda)
    scalars_dev = upload(scalars, cuda) if scalars is not None else None
    hp = adamw_hparams(HYPER["lr"], HYPER["beta1"], HYPER["beta2"], HYPER["eps"], HYPER["weight_decay"], step)
    status = lib.sr_adamw_multi(
        rows_dev.data_ptr(), tiles_dev.data_ptr(), None if scalars_dev is None else scalars_dev.data_ptr(),
        len(records), len(tile_rows), *_codes(rows, formats), ctypes.byref(hp), SEED, RNG_STEP, BLOCK,
        _lib.stream_handle(cuda))
    _lib.check("sr_adamw_multi", status)
    torch.cuda.synchronize()


def _launch_noalloc(cuda, rows, formats, records, total_tiles, scalars, step, nrows=None):
    lib = _lib.library()
    hp = adamw_hparams(HYPER["lr"], HYPER["beta1"], HYPER["beta2"], HYPER["eps"], HYPER["weight_decay"], step)
    status = lib.sr_adamw_multi_noalloc(
        records.ctypes.data, None if scalars is None else scalars.ctypes.data,
        len(records) if nrows is None else nrows, total_tiles, *_codes(rows, formats), ctypes.byref(hp),
        SEED, RNG_STEP, BLOCK, _lib.stream_handle(cuda))
    torch.cuda.synchronize()
    return status


def _clone(rows):
    out = []
    for row in rows:
        copies = []
        for t in row:
            # Keep each view's alignment: clone the base and view it the same way.
            base = t._base if t._base is not None else t
            offset = t.storage_offset() - base.storage_offset()
            copies.append(base.clone()[offset:offset + t.numel()])
        out.append(copies)
    return out


FORMATS = [
    ((torch.bfloat16, "stochastic"), (torch.bfloat16, "stochastic")),
    ((torch.float8_e4m3fn, "stochastic"), (torch.bfloat16, "stochastic")),
    ((torch.float16, "nearest"), (torch.float32, "nearest")),
]


@pytest.mark.parametrize("formats", FORMATS, ids=lambda f: "-".join(f"{d}/{r}" for d, r in f))
@pytest.mark.parametrize("p_dtype,g_dtype", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16),
                                             (torch.float32, torch.bfloat16)])
def test_noalloc_equals_device_table_launch_on_two_calls(cuda, formats, p_dtype, g_dtype):
    dtypes = (p_dtype, g_dtype, formats[0][0], formats[1][0])
    calls = [
        # (sizes, first parameter index, per-row steps or None, step)
        # 2^25 + 2^20 elements: past 2^16 tiles, so FP32-parameter launches
        # run with their resident-workgroup cap.
        ([(1 << 25) + (1 << 20), 2_000_003, 4099, -2053, 1, 512, 70_000, 129], 0, None, 5),
        ([1027, -515, 3], 9, [1, 7, 2], 2),
    ]
    for call, (sizes, first_index, steps, step) in enumerate(calls):
        ours = _bucket(cuda, sizes, dtypes, seed=31 + call)
        theirs = _clone(ours)
        records_ours, tile_rows = _tables(ours, first_index)
        records_theirs, _ = _tables(theirs, first_index)
        assert np.array_equal(records_ours["flags"], records_theirs["flags"])
        scalars = None if steps is None else _row_scalars(steps)
        status = _launch_noalloc(cuda, ours, formats, records_ours, len(tile_rows), scalars, step)
        _lib.check("sr_adamw_multi_noalloc", status)
        _launch_device_tables(cuda, theirs, formats, records_theirs, tile_rows, scalars, step)
        for r, (a, b) in enumerate(zip(ours, theirs)):
            for name, x, y in zip(("parameter", "gradient", "exp_avg", "exp_avg_sq"), a, b):
                assert_bits_or_nan(x.cpu(), y.cpu(), f"call {call + 1}, row {r}: {name}")


def test_noalloc_refuses_oversized_and_malformed_tables(cuda):
    formats = FORMATS[0]
    rows = _bucket(cuda, [4099, 600], (torch.float32, torch.float32, torch.bfloat16, torch.bfloat16), seed=5)
    before = [[t.clone() for t in row] for row in rows]
    records, tile_rows = _tables(rows, 0)
    lib = _lib.library()

    def refused(match, **kwargs):
        status = _launch_noalloc(cuda, rows, formats, kwargs.pop("records", records),
                                 kwargs.pop("total", len(tile_rows)), kwargs.pop("scalars", None), 1, **kwargs)
        assert status == 1, status  # SR_ERR_ARGUMENT
        assert match in lib.sr_last_error().decode(), lib.sr_last_error()

    refused("row count", nrows=_lib.NOALLOC_MAX_ROWS + 1)
    refused("row count", nrows=0)
    refused("tiles outside", total=_lib.NOALLOC_MAX_TILES + 1)
    refused("rows cover", total=len(tile_rows) + 1)
    gap = records.copy()
    gap["tile_begin"][1] += 1
    refused("tiles start at", records=gap)
    short = records.copy()
    short["tile_end"][0] -= 1
    short["tile_begin"][1] -= 1
    refused("tiles for", records=short)
    null = records.copy()
    null["ptr"][1][2] = 0
    refused("null pointer", records=null)
    misaligned = records.copy()
    misaligned["ptr"][0][3] += 2
    refused("16-byte aligned", records=misaligned)
    refused("correction2_sqrt", scalars=np.array([-1e-3, 1.0, -1e-3, 0.0], dtype=np.float32))
    for row, saved in zip(rows, before):
        for t, s in zip(row, saved):
            assert torch.equal(t.view(torch.uint8), s.view(torch.uint8))


def _pinned(array):
    """A page-locked host copy of a numpy array's bytes, as a torch tensor."""
    return torch.from_numpy(np.ascontiguousarray(array).view(np.uint8).reshape(-1)).pin_memory()


def test_noalloc_under_graph_capture_replays_like_eager_calls(cuda):
    formats = FORMATS[1]
    dtypes = (torch.float32, torch.float32, formats[0][0], formats[1][0])
    # The first row takes the bucket past 2^16 tiles: the captured launch
    # carries the resident-workgroup cap.
    sizes, first_index, steps, step = [(1 << 25) + 3, 70_001, 4099, -2053, 1, 512], 3, [1, 4, 2, 9, 3, 5], 4
    ours = _bucket(cuda, sizes, dtypes, seed=77)
    initial = _clone(ours)
    theirs = _clone(ours)
    records, tile_rows = _tables(ours, first_index)
    records_theirs, _ = _tables(theirs, first_index)
    scalars = _row_scalars(steps)
    _launch_device_tables(cuda, theirs, formats, records_theirs, tile_rows, scalars, step)
    rows_pinned, scalars_pinned = _pinned(records), _pinned(scalars)
    other = _bucket(cuda, [9000, 257], dtypes, seed=78)
    other_records, other_tiles = _tables(other, 0)
    lib = _lib.library()
    hp = adamw_hparams(HYPER["lr"], HYPER["beta1"], HYPER["beta2"], HYPER["eps"], HYPER["weight_decay"], step)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        status = lib.sr_adamw_multi_noalloc(
            rows_pinned.data_ptr(), scalars_pinned.data_ptr(), len(records), len(tile_rows), *_codes(ours, formats),
            ctypes.byref(hp), SEED, RNG_STEP, BLOCK, _lib.stream_handle(cuda))
    _lib.check("sr_adamw_multi_noalloc (captured)", status)
    for replay in range(3):
        # Eager work between replays: the tensors back to their initial bytes,
        # and a call on other tables that leaves them in the scratch.
        for row, start in zip(ours, initial):
            for t, t0 in zip(row, start):
                t.copy_(t0)
        _lib.check("sr_adamw_multi_noalloc", _launch_noalloc(cuda, other, formats, other_records, len(other_tiles),
                                                             None, 1))
        graph.replay()
        torch.cuda.synchronize()
        for r, (a, b) in enumerate(zip(ours, theirs)):
            for name, x, y in zip(("parameter", "gradient", "exp_avg", "exp_avg_sq"), a, b):
                assert_bits_or_nan(x.cpu(), y.cpu(), f"replay {replay + 1}, row {r}: {name}")
    del graph
    torch.cuda.synchronize()


def test_noalloc_refuses_pageable_tables_under_capture(cuda):
    formats = FORMATS[0]
    rows = _bucket(cuda, [4099, 600], (torch.float32, torch.float32, torch.bfloat16, torch.bfloat16), seed=6)
    before = [[t.clone() for t in row] for row in rows]
    records, tile_rows = _tables(rows, 0)
    lib = _lib.library()
    hp = adamw_hparams(HYPER["lr"], HYPER["beta1"], HYPER["beta2"], HYPER["eps"], HYPER["weight_decay"], 1)
    marker = torch.zeros(1, device=cuda)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        status = lib.sr_adamw_multi_noalloc(
            records.ctypes.data, None, len(records), len(tile_rows), *_codes(rows, formats), ctypes.byref(hp),
            SEED, RNG_STEP, BLOCK, _lib.stream_handle(cuda))
        marker.add_(1)  # the graph records this kernel and nothing of the refused call
    assert status == 1, status  # SR_ERR_ARGUMENT
    assert "pinned host memory" in lib.sr_last_error().decode(), lib.sr_last_error()
    graph.replay()
    torch.cuda.synchronize()
    assert marker.item() == 1
    for row, saved in zip(rows, before):
        for t, s in zip(row, saved):
            assert torch.equal(t.view(torch.uint8), s.view(torch.uint8))
    del graph
