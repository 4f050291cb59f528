"""Multi-tensor bucketing, row tables and the optimizer frame on CPU.

Mirrors tests/test_multi_tensor_tables.py, tests/test_fp8_storage.py:137-176
and tests/test_rounding_registry.py:142-173 of the reference: the real host
dispatch runs, the kernel launch is replaced by a recorder, and the GPU device
check by a no-op.
"""

from __future__ import annotations

import copy
import importlib
import math
from contextlib import nullcontext

import numpy as np
import pytest
import torch

import sr_states
from sr_states import AdamWHip, SGDMHip, StateFormat
from sr_states import _lib
from sr_states.hip._multi_tensor import GroupTableCache, bucket_items, build_records, build_tile_rows
from sr_states.hip._optimizer import DEFAULT_BLOCK_SIZE
from sr_states.optim._state import StateOptimizer, _validate_rng_numel

from oracle import sr_oracle

MOMENT = ("m",)


class _Parameter:
    """Tensor proxy whose gradient may have another dtype."""

    def __init__(self, tensor, grad):
        self.tensor = tensor
        self.grad = grad

    def __getattr__(self, name):
        return getattr(self.tensor, name)


def item(n, index=0, step=1, *, dtype=torch.float32, offset=0, device="cpu", grad_dtype=None):
    p = _Parameter(torch.zeros(n, dtype=dtype, device=device), torch.zeros(n, dtype=grad_dtype or dtype, device=device))
    return p, {"m": torch.zeros(n, device=device)}, index, step, offset


def test_buckets_split_device_and_dtypes_and_rows_keep_their_steps():
    """tests/test_multi_tensor_tables.py:36-57, with AdamW steps kept per row.

    The reference also splits AdamW buckets by step; here a row at another
    step stays in its dtype bucket and carries its own step.
    """
    items = [item(0, 0), item(17, 2), item(5, 4, step=2), item(3, 5, dtype=torch.bfloat16),
             item(1, 6, grad_dtype=torch.bfloat16), item(2, 7, device="meta"), item(1, 9)]
    adamw = bucket_items(items, MOMENT, uses_step=True)
    sgdm = bucket_items(items, MOMENT, uses_step=False)
    assert [[r.param_index for r in rows] for rows in adamw.values()] == [[2, 4, 9], [5], [6], [7]]
    assert [[r.param_index for r in rows] for rows in sgdm.values()] == [[2, 4, 9], [5], [6], [7]]
    first = next(iter(adamw.values()))
    assert [(r.step, r.position) for r in first] == [(1, 1), (2, 2), (1, 6)]
    assert [r.step for r in next(iter(sgdm.values()))] == [None] * 3
    (device, dtypes), *_ = adamw
    assert (device.type, dtypes) == ("cpu", (torch.float32,) * 3)


def test_records_and_tile_map_layout():
    tile = 128 * _lib.LANE_ELEMENTS
    layout = [(1, 3, 2**32 - 20), (tile - 1, 4, 5), (tile, 2**32 + 6, 0), (tile + 1, 7, 2**33 + 1)]
    pointers = [(16 * k, 16 * k + 32, 64, 80 + (k == 2) * 4) for k in range(4)]
    records = build_records(layout, pointers, tile)
    assert records["numel"].tolist() == [1, tile - 1, tile, tile + 1]
    assert records["tile_begin"].tolist() == [0, 1, 2, 3]
    assert records["tile_end"].tolist() == [1, 2, 3, 5]
    assert records["param_index"].tolist() == [3, 4, 6, 7]
    assert records["shard_start"].tolist() == [2**32 - 20, 5, 0, 1]
    assert records["flags"].tolist() == [_lib.ROW_VECTOR, _lib.ROW_VECTOR, 0, _lib.ROW_VECTOR]
    assert records["ptr"][2].tolist() == [32, 64, 64, 84]
    assert build_tile_rows(layout, tile).tolist() == [0, 1, 2, 3, 3]
    # SGDM rows carry three pointers; the fourth is zero.
    assert build_records([(5, 0, 0)], [(16, 32, 48)], 1024)["ptr"][0].tolist() == [16, 32, 48, 0]


@pytest.mark.parametrize("block", [128, 256, 1024])
@pytest.mark.parametrize("lanes", [_lib.LANE_ELEMENTS, _lib.LANE_ELEMENTS_NARROW])
def test_tile_map_covers_every_element_once(block, lanes):
    """Property: each tile belongs to exactly one row and covers its elements in order."""
    gen = np.random.default_rng(5)
    layout = [(int(n), i, 0) for i, n in enumerate(gen.integers(1, 50_000, size=200))]
    tile = block * lanes
    records = build_records(layout, [(0, 0, 0)] * len(layout), tile)
    tile_rows = build_tile_rows(layout, tile)
    assert len(tile_rows) == records["tile_end"][-1]
    for r, rec in enumerate(records):
        owned = np.nonzero(tile_rows == r)[0]
        assert owned.tolist() == list(range(rec["tile_begin"], rec["tile_end"]))
        assert (rec["tile_end"] - rec["tile_begin"]) * tile >= rec["numel"] > (rec["tile_end"] - rec["tile_begin"] - 1) * tile


def test_table_cache_reuse_and_refresh():
    """tests/test_multi_tensor_tables.py:60-121: step-invariant tables, refresh on change."""
    items = [item(n, i, offset=2**32 - 20 + i) for i, n in enumerate((1, 600, 1024, 1025))]
    cache = GroupTableCache()

    def tables(rows, block):
        (launch,) = cache.prepare(bucket_items(rows, MOMENT, uses_step=True), block)
        return launch.steps, launch.tables

    steps, first = tables(items, 128)
    assert first.tile_rows.tolist() == [0, 1, 1, 2, 2, 3, 3, 3]  # 512-element tiles
    assert steps == 1
    steps, same = tables([(*row[:3], 2, row[-1]) for row in items], 128)
    assert steps == 2 and same is first
    # Rows at different steps share the launch and the tables.
    steps, mixed = tables([(*row[:3], 2 + (k == 2), row[-1]) for k, row in enumerate(items)], 128)
    assert steps == (2, 2, 3, 2) and mixed is first
    steps, resized = tables(items, 256)
    assert resized is not first and resized.tile_rows.tolist() == [0, 1, 2, 3, 3]
    # Same layout, a new gradient address: records rebuilt, tile map reused.
    p = items[1][0]
    p.grad = torch.zeros_like(p.grad)
    steps, moved = tables(items, 256)
    assert moved is not resized and moved.device_tile_rows is resized.device_tile_rows
    assert moved.records["ptr"][1][1] == p.grad.data_ptr()


@pytest.mark.parametrize("different_steps", [False, True])
def test_overlapping_writes_rejected_even_across_buckets(different_steps):
    """tests/test_multi_tensor_tables.py:124-131."""
    shared = torch.ones(12)
    a, b = item(8, 0), item(8, 1, step=1 + different_steps)
    a[0].tensor, b[0].tensor = shared[:8], shared[4:]
    with pytest.raises(ValueError, match="overlap"):
        GroupTableCache().prepare(bucket_items([a, b], MOMENT, uses_step=True), 256)


def test_shared_gradients_allowed_and_repointing_revalidates():
    """tests/test_multi_tensor_tables.py:134-144."""
    shared = torch.ones(16)
    a, b = item(8, 0), item(8, 1)
    a[0].tensor, b[0].tensor = shared[:8], shared[8:]
    b[0].grad = a[0].grad
    cache = GroupTableCache()
    cache.prepare(bucket_items([a, b], MOMENT, uses_step=True), 256)
    b[0].grad = a[0].tensor
    with pytest.raises(ValueError, match="overlap"):
        cache.prepare(bucket_items([a, b], MOMENT, uses_step=True), 256)


def test_layout_is_checked_even_when_addresses_match():
    """tests/test_multi_tensor_tables.py:147-156."""
    p, state, *rest = item(16)
    p.tensor, p.grad, state["m"] = p.tensor.view(4, 4), p.grad.view(4, 4), state["m"].view(4, 4)
    GroupTableCache().prepare(bucket_items([(p, state, *rest)], MOMENT, uses_step=True), 256)
    state["m"] = state["m"].T
    with pytest.raises(ValueError, match="contiguous"):
        bucket_items([(p, state, *rest)], MOMENT, uses_step=True)


def test_parameter_hook_keeps_order_rng_indices_and_partial_failure():
    """tests/test_multi_tensor_tables.py:159-175."""
    class Recorder(StateOptimizer):
        _state_names = MOMENT

        def _step_parameter(self, parameter, state, group, formats, step, seed, offset):
            calls.append((parameter, step, seed, offset))

    calls = []
    p, skipped, q, bad = [torch.nn.Parameter(torch.ones(2)) for _ in range(4)]
    opt = Recorder([{"params": [p, skipped], "sr_seed": 7}, {"params": [q, bad]}], {}, seed=3)
    p.grad = q.grad = torch.ones(2)
    bad.grad = torch.sparse_coo_tensor([[0]], [1.0], (2,), check_invariants=True)
    with pytest.raises(RuntimeError, match="sparse"):
        opt.step()
    assert calls == [(p, 1, sr_oracle.update_key(7, 1, 0), 0), (q, 1, sr_oracle.update_key(3, 1, 2), 0)]
    assert opt.state[p]["step"] == opt.state[q]["step"] == opt._rng_step() == 1
    assert skipped not in opt.state and bad not in opt.state


def test_rng_numel_limit():
    _validate_rng_numel(1 << 32)
    with pytest.raises(ValueError, match="at most"):
        _validate_rng_numel((1 << 32) + 1)


# -- fused host dispatch with a recording launcher ---------------------------------
@pytest.fixture
def recorder(monkeypatch):
    launches = []
    for kind in ("adamw", "sgd"):
        module = importlib.import_module(f"sr_states.hip.{kind}")

        def record(tables, dtypes, hparams, seed, rng_step, block_size, stream, row_scalars=None, *,
                   _kind=kind):
            launches.append({"kind": _kind, "tables": tables, "dtypes": dtypes, "hparams": hparams,
                             "seed": seed, "rng_step": rng_step, "block_size": block_size,
                             "row_scalars": row_scalars})

        monkeypatch.setattr(module, "_launch", record)
        monkeypatch.setattr(module, "validate_update_device", lambda *args: None)
    monkeypatch.setattr(torch.cuda, "device", lambda device: nullcontext())
    monkeypatch.setattr(_lib, "on_device", lambda device: nullcontext())
    monkeypatch.setattr(_lib, "stream_handle", lambda device: 0)
    return launches


def test_each_state_dispatches_its_own_rule(recorder):
    """tests/test_fp8_storage.py:137-176: per-moment formats reach the launch."""
    fmt = {"exp_avg": StateFormat(torch.float8_e4m3fn), "exp_avg_sq": StateFormat(torch.float8_e5m2, "nearest")}
    p = torch.nn.Parameter(torch.ones(17))
    opt = AdamWHip([p], lr=0.01, state_format=fmt, seed=3)
    p.grad = torch.ones_like(p)
    opt.step()
    opt.step()
    assert opt._rng_step() == 2 and len(recorder) == 2
    for launch in recorder:
        assert launch["dtypes"] == (_lib.SR_F32, _lib.SR_F32, _lib.SR_E4M3, _lib.SR_STOCHASTIC,
                                    _lib.SR_E5M2, _lib.SR_NEAREST)
    assert [launch["rng_step"] for launch in recorder] == [1, 2]
    assert opt.state[p]["step"] == 2
    q = torch.nn.Parameter(torch.ones(5))
    sgd = SGDMHip([q], lr=0.01, state_format=StateFormat(torch.float16), seed=-1)
    q.grad = torch.ones_like(q)
    sgd.step()
    assert recorder[-1]["dtypes"] == (_lib.SR_F32, _lib.SR_F32, _lib.SR_F16, _lib.SR_STOCHASTIC)
    assert recorder[-1]["seed"] == 2**64 - 1
    assert "step" not in sgd.state[q]


def test_launch_scalars_are_the_eager_fp32_roundings(recorder):
    lr, betas, eps, wd = 3e-4, (0.9, 0.999), 1e-8, 0.01
    p = torch.nn.Parameter(torch.ones(3))
    opt = AdamWHip([p], lr=lr, betas=betas, eps=eps, weight_decay=wd)
    for _ in range(3):
        p.grad = torch.ones_like(p)
        opt.step()
    hp = recorder[-1]["hparams"]
    f32 = lambda v: float(np.float32(v))  # noqa: E731
    assert hp.beta1 == f32(0.9) and hp.beta2 == f32(0.999)
    assert hp.one_minus_beta1 == f32(1 - 0.9) and hp.one_minus_beta2 == f32(1 - 0.999)
    assert hp.neg_step_size == f32(-lr / (1 - 0.9**3))
    assert hp.correction2_sqrt == f32(math.sqrt(1 - 0.999**3))
    assert hp.decay == f32(1 - lr * wd) and hp.eps == f32(eps)


def test_one_table_per_bucket_and_no_launch_on_validation_error(recorder):
    """tests/test_triton_multi_tensor.py:184-228 on CPU."""
    tile = DEFAULT_BLOCK_SIZE * _lib.LANE_ELEMENTS  # BF16 moments

    def parameter(n, dtype=torch.float32):
        p = torch.nn.Parameter(torch.ones(n, dtype=dtype))
        p.grad = torch.ones_like(p)
        return p

    p, q, r, empty, second = parameter(1), parameter(tile + 1), parameter(3, torch.bfloat16), parameter(0), parameter(31)
    opt = AdamWHip([{"params": [p, q, r, empty]}, {"params": [second]}], lr=0.01)
    opt.step()
    assert [launch["tables"].total_tiles for launch in recorder] == [3, 1, 1]
    assert recorder[0]["tables"].records["param_index"].tolist() == [0, 1]
    assert recorder[2]["tables"].records["param_index"].tolist() == [4]
    recorder.clear()
    opt.state[r]["exp_avg"] = torch.zeros(4, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="shapes"):
        opt.step()
    assert not recorder


def test_steps_missing_gradients_and_resume_bookkeeping(recorder):
    """tests/test_state_optimizers.py:54-88 (host bookkeeping)."""
    params = [torch.nn.Parameter(torch.linspace(-1, 1, 17)) for _ in range(3)]
    opt = AdamWHip([{"params": params[:2]}, {"params": params[2:]}], lr=0.1, seed=4)
    for index in (0, 2):
        params[index].grad = torch.ones_like(params[index]) * 0.103
    opt.step()
    assert params[1] not in opt.state
    assert [g["sr_step"] for g in opt.param_groups] == [1, 1]
    assert sum(opt.state[params[0]][n].nbytes for n in opt._state_names) == 17 * 2 * 2
    resumed = AdamWHip([{"params": [torch.nn.Parameter(p.detach().clone()) for p in params[:2]]},
                        {"params": [torch.nn.Parameter(params[2].detach().clone())]}], lr=0.5)
    resumed.load_state_dict(copy.deepcopy(opt.state_dict()))
    for _ in range(4):
        for p in params:
            p.grad = torch.ones_like(p)
        opt.step()
    assert [opt.state[p]["step"] for p in params] == [5, 4, 5]
    assert opt._rng_step() == 5


def test_closure_and_sparse_gradient_consume_the_step(recorder):
    """tests/test_state_optimizers.py:91-107."""
    p = torch.nn.Parameter(torch.ones(4))
    optimizer = SGDMHip([p], lr=0.01)

    def closure():
        optimizer.zero_grad()
        loss = p.square().sum()
        loss.backward()
        return loss

    assert optimizer.step(closure).item() == 4
    p.grad = torch.sparse_coo_tensor([[0]], [1.0], size=(4,), check_invariants=True)
    rng_step = optimizer._rng_step()
    with pytest.raises(RuntimeError, match="sparse"):
        optimizer.step()
    assert optimizer._rng_step() == rng_step + 1


def test_dtensor_with_partial_placement_is_rejected():
    """tests/test_rng_streams.py:278-296, on a real DTensor of one fake rank.

    The reference refuses every DTensor parameter there.  This backend
    accepts those whose local shard is one flat range of the parameter
    (tests/test_dtensor.py) and still refuses the others, such as a Partial
    placement, before any state exists.
    """
    import torch.distributed as dist

    pytest.importorskip("torch.testing._internal.distributed.fake_pg")
    from torch.distributed.tensor import DeviceMesh, DTensor, Partial

    dist.init_process_group("fake", store=dist.HashStore(), rank=0, world_size=1)
    try:
        value = DTensor.from_local(torch.ones(3), DeviceMesh("cpu", [0]), [Partial()])
        p = torch.nn.Parameter(value)
        p.grad = value.clone()
        optimizer = SGDMHip([p], lr=0.01)
        for _ in range(2):  # a rejected step never becomes a reusable plan
            with pytest.raises(NotImplementedError, match="DTensor optimizer parameters support"):
                optimizer.step()
        assert p not in optimizer.state
    finally:
        dist.destroy_process_group()


def test_library_is_the_only_execution_path(monkeypatch):
    """Without the HIP library every entry point raises; nothing falls back to torch."""
    monkeypatch.setattr(_lib, "_handle", None)
    monkeypatch.setattr(_lib, "LIBRARY_PATH", _lib.LIBRARY_PATH.with_name("missing.so"))
    with pytest.raises(RuntimeError, match="not built"):
        sr_states.update_key(1, 2, 3)


def test_buckets_are_tiled_at_their_lane_width(recorder):
    """Tile tables follow the library's lane width for each bucket's dtypes."""
    n, block = 5000, 256
    fp8 = {"exp_avg": StateFormat(torch.float8_e4m3fn), "exp_avg_sq": StateFormat(torch.bfloat16)}
    cases = [(torch.float32, fp8, _lib.lane_elements(torch.float32, torch.float32, torch.float8_e4m3fn, torch.bfloat16)),
             (torch.bfloat16, None, _lib.lane_elements(*(torch.bfloat16,) * 4)),
             (torch.float32, None, _lib.lane_elements(torch.float32, torch.float32, torch.bfloat16, torch.bfloat16))]
    for dtype, formats, _ in cases:
        p = torch.nn.Parameter(torch.ones(n, dtype=dtype))
        p.grad = torch.ones_like(p)
        AdamWHip([p], lr=0.01, state_format=formats, block_size=block).step()
    for launch, (_, _, lanes) in zip(recorder, cases):
        tiles = -(-n // (block * lanes))
        assert launch["tables"].total_tiles == tiles
        assert launch["tables"].records["tile_end"].tolist() == [tiles]


def test_tile_limit_is_the_launch_grid():
    """A bucket may not need more workgroups than one launch can hold."""
    from sr_states.hip._multi_tensor import MAX_TILES

    tile = 1024
    assert build_tile_rows([(tile, 0, 0), (1, 1, 0)], tile).tolist() == [0, 1]
    # One tile past the limit fails before anything is allocated.
    with pytest.raises(ValueError, match="at most"):
        build_tile_rows([(MAX_TILES * tile, 0, 0), (1, 1, 0)], tile)
