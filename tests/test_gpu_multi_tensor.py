"""Multi-tensor AdamWHip / SGDMHip on the GPU.

* The fused multi-tensor launch equals per-parameter functional updates byte
  for byte, across groups, mixed dtypes, unaligned views, shard offsets near
  2^32, missing gradients, appended groups and RNG steps crossing 2^32
  (tests/test_triton_multi_tensor.py:39-152).
* Trajectories written by the reference optimizers (tests/golden/
  reference_trajectories.pt), each step started from the reference's bytes
  of the step before: states identical, FP32 parameters within 1 ulp (the
  reference's CPU square root is not always correctly rounded) and BF16
  parameters identical, at every step.
* Launch counting, streams and checkpoint resume.
"""

from __future__ import annotations

import copy
import importlib
from itertools import chain
from pathlib import Path

import pytest
import torch
from conftest import assert_bits_or_nan, ulp_distance

from oracle import sr_oracle
from sr_states.hip._optimizer import DEFAULT_BLOCK_SIZE

pytestmark = pytest.mark.gpu

DTYPES = (torch.float32, torch.bfloat16, torch.float16, torch.float8_e4m3fn, torch.float8_e5m2)
GOLDEN = Path(__file__).parent / "golden" / "reference_trajectories.pt"


class _MixedGradientParameter(torch.nn.Parameter):
    """Parameter whose gradient may have another dtype (tests/test_triton_multi_tensor.py:22-31)."""

    @property
    def grad(self):
        return getattr(self, "_gradient", None)

    @grad.setter
    def grad(self, value):
        self._gradient = value


def assert_bytes(actual, expected):
    assert actual.dtype == expected.dtype and actual.shape == expected.shape
    assert torch.equal(actual.contiguous().view(torch.uint8), expected.contiguous().view(torch.uint8))


@pytest.mark.parametrize("kind", ["adamw", "sgd"])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rounding", ["nearest", "stochastic"])
def test_multi_tensor_matches_functional_updates_byte_for_byte(cuda, kind, dtype, rounding):
    import sr_states
    from sr_states import StateFormat

    adamw = kind == "adamw"
    cls = sr_states.AdamWHip if adamw else sr_states.SGDMHip
    update = sr_states.hip_adamw_step_ if adamw else sr_states.hip_sgdm_step_
    block_size = 128
    # The widest tile among the test's buckets (8 lanes for FP8 states).
    chunk = block_size * sr_states._lib.lane_elements(torch.float32, torch.float32, dtype, dtype)
    start_step = 2**32 + 8

    class OffsetOptimizer(cls):
        def _shard_start(self, parameter):
            return offsets[parameter]

    def make_parameter(n, ptype):
        values = torch.linspace(-0.8, 0.7, n + 1, device=cuda)
        return _MixedGradientParameter(values.to(ptype)[1:])  # an unaligned view

    f32, bf16 = torch.float32, torch.bfloat16
    layouts = [
        [(0, f32, f32), (1, f32, f32), (chunk + 13, f32, f32), (chunk, bf16, bf16), (5 * chunk, f32, f32)],
        [(chunk + 1, f32, f32), (61, f32, bf16)],
    ]
    groups = [[make_parameter(n, pd) for n, pd, _ in rows] for rows in layouts]
    # One aligned parameter so that the vector path runs too.
    aligned = _MixedGradientParameter(torch.linspace(-1, 1, 3 * chunk + 7, device=cuda))
    groups[0].append(aligned)
    layouts[0].append((aligned.numel(), f32, f32))
    formats = [(StateFormat(dtype, rounding),) * len(cls._state_names)]
    if adamw:
        second = torch.float8_e5m2 if dtype == torch.float8_e4m3fn else torch.bfloat16
        other = "nearest" if rounding == "stochastic" else "stochastic"
        formats.append((StateFormat(dtype, rounding), StateFormat(second, other)))
    else:
        formats.append((StateFormat(torch.bfloat16, rounding),))
    seeds = (-(2**48) - 1, 2**78 + 0xABCD000100000010)
    opt = OffsetOptimizer(
        [
            {"params": params, "state_format": dict(zip(cls._state_names, fmts)), "sr_seed": seed,
             "sr_step": start_step}
            for params, fmts, seed in zip(groups, formats, seeds)
        ],
        lr=0.06,
        block_size=block_size,
    )
    offsets = {p: 2**32 - 83 + i for i, p in enumerate(chain.from_iterable(groups))}
    expected = {p: p.detach().clone() for p in offsets}
    states, steps = {}, {}
    generator = torch.Generator(device=cuda).manual_seed(756)
    for i in range(4):
        if i == 2:
            later = make_parameter(35, f32)
            offsets[later] = -(2**32) - 13
            expected[later] = later.detach().clone()
            groups.append([later])
            layouts.append([(35, f32, f32)])
            formats.append(formats[0])
            opt.add_param_group(
                {"params": [later], "state_format": dict(zip(cls._state_names, formats[0])),
                 "sr_seed": seeds[0]}
            )
        old_grads = [p.grad for params in groups for p in params]
        opt.zero_grad(set_to_none=True)
        rng_step = start_step + i + 1
        index = 0
        for group, params, rows, fmt in zip(opt.param_groups, groups, layouts, formats):
            for p, (n, _, gdtype) in zip(params, rows):
                if index != 2 or i not in (1, 3):
                    p.grad = torch.randn(n, device=cuda, generator=generator).to(gdtype)
                    if p not in states:
                        states[p] = tuple(torch.zeros_like(p, dtype=f.dtype) for f in fmt)
                    steps[p] = steps.get(p, 0) + 1
                    kwargs = (
                        {"beta1": group["betas"][0], "beta2": group["betas"][1], "eps": group["eps"],
                         "weight_decay": group["weight_decay"], "step": steps[p]}
                        if adamw else {"momentum_factor": group["momentum"]}
                    )
                    update(expected[p], p.grad, *states[p], lr=group["lr"],
                           seed=sr_oracle.update_key(group["sr_seed"], rng_step, index),
                           offset=offsets[p], formats=fmt, block_size=block_size, **kwargs)
                index += 1
        del old_grads
        opt.step()
        assert opt._rng_step() == rng_step
        for p in offsets:
            assert_bytes(p.detach(), expected[p])
            for name, state in zip(cls._state_names, states.get(p, ())):
                assert_bytes(opt.state[p][name], state)
            assert opt.state[p].get("step") == (steps.get(p) if adamw else None)


def _golden_cases():
    # A missing fixture is a collection error, not zero cases.
    cases = list(torch.load(GOLDEN, weights_only=True)["cases"].items())
    assert len(cases) == 3, [name for name, _ in cases]
    return cases


@pytest.mark.parametrize("name,case", _golden_cases(), ids=lambda v: v if isinstance(v, str) else "")
def test_matches_reference_trajectories(cuda, name, case):
    """Replays tests/golden/make_reference_vectors.py on the GPU."""
    import sr_states
    from sr_states import StateFormat

    dtypes = {"torch.float32": torch.float32, "torch.bfloat16": torch.bfloat16}
    short = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16,
             "e4m3": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}
    kind = case["kind"]
    names = ("exp_avg", "exp_avg_sq") if kind == "adamw" else ("momentum_buffer",)
    params = [
        torch.nn.Parameter(raw.view(dtypes[dt]).clone().to(cuda))
        for raw, dt in zip(case["initial"], case["dtypes"])
    ]
    param_groups, at = [], 0
    for group in case["groups"]:
        count = len(group["sizes"])
        fmt = {n: StateFormat(short[f.split("/")[0]], f.split("/")[1]) for n, f in zip(names, group["formats"])}
        entry = {"params": params[at : at + count], "state_format": fmt, "sr_seed": group["sr_seed"]}
        if "lr" in group:
            entry["lr"] = group["lr"]
        param_groups.append(entry)
        at += count
    cls = sr_states.AdamWHip if kind == "adamw" else sr_states.SGDMHip
    opt = cls(param_groups, **case["hyper"])
    for group in opt.param_groups:
        group["sr_step"] = case["initial_sr_step"]
    previous = None
    for step, record in enumerate(case["steps"], start=1):
        if previous is not None:
            # Each step starts from the reference's own bytes of the step
            # before, so per-step differences cannot accumulate.
            with torch.no_grad():
                for p, want_p, want_state in zip(params, previous["params"], previous["states"]):
                    p.copy_(want_p.view(p.dtype).to(cuda))
                    for state_name, value in want_state.items():
                        if state_name in names:
                            stored = opt.state[p][state_name]
                            stored.copy_(value.view(stored.dtype).to(cuda))
        for p, grad in zip(params, record["grads"]):
            p.grad = None if grad is None else grad.view(p.dtype).clone().to(cuda)
        opt.step()
        assert [g["sr_step"] for g in opt.param_groups] == record["sr_step"]
        for index, (p, want_p, want_state) in enumerate(zip(params, record["params"], record["states"])):
            want = want_p.view(p.dtype)
            # The reference's CPU square root is not always correctly rounded:
            # FP32 parameters within 1 ulp; BF16 parameters, rounded from
            # them, equal.
            bound = 1 if p.dtype == torch.float32 else 0
            distance = int(ulp_distance(p.detach().float(), want.float()).max())
            assert distance <= bound, (name, step, index, distance)
            for state_name in names:
                if state_name not in want_state:
                    assert state_name not in opt.state[p]
                    continue
                got = opt.state[p][state_name]
                assert_bits_or_nan(got, want_state[state_name].view(got.dtype), f"{name} step {step}")
            if "step" in want_state:
                assert opt.state[p]["step"] == want_state["step"]


@pytest.mark.parametrize("kind", ["adamw", "sgd"])
def test_one_launch_per_bucket_and_no_launch_on_validation_error(cuda, kind, monkeypatch):
    """tests/test_triton_multi_tensor.py:184-228."""
    import sr_states

    module = importlib.import_module(f"sr_states.hip.{kind}")
    cls = sr_states.AdamWHip if kind == "adamw" else sr_states.SGDMHip
    launch = module._launch
    tiles = []

    def count(tables, *args):
        tiles.append(tables.total_tiles)
        return launch(tables, *args)

    monkeypatch.setattr(module, "_launch", count)
    tile = DEFAULT_BLOCK_SIZE * sr_states._lib.LANE_ELEMENTS  # BF16 moments

    def parameter(n, dtype=torch.float32):
        p = torch.nn.Parameter(torch.ones(n, device=cuda, dtype=dtype))
        p.grad = torch.ones_like(p)
        return p

    p, q, r, empty, second = (parameter(1), parameter(tile + 1), parameter(3, torch.bfloat16),
                              parameter(0), parameter(31))
    opt = cls([{"params": [p, q, r, empty]}, {"params": [second]}], lr=0.01)
    opt.step()
    assert tiles == [3, 1, 1]
    tiles.clear()
    q.grad = None
    opt.step()
    q.grad = torch.ones_like(q)
    tiles.clear()
    opt.step()
    # q's AdamW step now lags p's; the reference would launch the two steps
    # separately, here they share one launch with per-row bias corrections.
    assert tiles == [3, 1, 1]

    before = p.detach().clone()
    tiles.clear()
    opt.state[r][opt._state_names[0]] = torch.zeros(4, device=cuda, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="shapes"):
        opt.step()
    assert not tiles
    assert_bytes(p.detach(), before)


@pytest.mark.parametrize("kind", ["adamw", "sgd"])
def test_tables_follow_the_launch_stream(cuda, kind):
    """tests/test_triton_multi_tensor.py:231-249."""
    import sr_states

    cls = sr_states.AdamWHip if kind == "adamw" else sr_states.SGDMHip
    p, q = [torch.nn.Parameter(torch.ones(2570, device=cuda)) for _ in range(2)]
    base = torch.cuda.current_stream()
    p.grad = q.grad = torch.full_like(p, 0.123)
    alternating, single = cls([p], lr=0.02), cls([q], lr=0.02)
    other = torch.cuda.Stream()
    for _ in range(3):
        alternating.step()
        other.wait_stream(base)
        with torch.cuda.stream(other):
            alternating.step()
        base.wait_stream(other)
        single.step()
        single.step()
    assert_bytes(p.detach(), q.detach())
    for name in alternating._state_names:
        assert_bytes(alternating.state[p][name], single.state[q][name])


@pytest.mark.parametrize("kind", ["adamw", "sgd"])
@pytest.mark.parametrize("state_dtype", [torch.float32, torch.bfloat16, torch.float8_e4m3fn])
@pytest.mark.parametrize("parameter_dtype", [torch.float32, torch.bfloat16])
def test_checkpoint_resumes_identically(cuda, kind, state_dtype, parameter_dtype):
    """tests/test_triton_states.py:165-185."""
    import sr_states

    cls = sr_states.AdamWHip if kind == "adamw" else sr_states.SGDMHip
    initial = torch.linspace(-1, 1, 1003, device=cuda, dtype=parameter_dtype)
    p = torch.nn.Parameter(initial.clone())
    opt = cls([p], lr=0.01, state_dtype=state_dtype, seed=77)
    p.grad = torch.cos(initial)
    opt.step()
    q = torch.nn.Parameter(p.detach().clone())
    resumed = cls([q], lr=0.1, seed=12)
    resumed.load_state_dict(copy.deepcopy(opt.state_dict()))
    for step in range(1, 6):
        p.grad = torch.sin(initial * step)
        q.grad = p.grad.clone()
        opt.step()
        resumed.step()
        assert torch.equal(p, q)
        for name in opt._state_names:
            assert opt.state[p][name].dtype == state_dtype
            assert_bytes(opt.state[p][name], resumed.state[q][name])


@pytest.mark.parametrize("kind", ["adamw", "sgd"])
def test_fp32_states_match_torch_optim(cuda, kind):
    """tests/test_triton_states.py:237-258."""
    import sr_states

    p = torch.nn.Parameter(torch.linspace(-1, 1, 1003, device=cuda))
    q = torch.nn.Parameter(p.detach().clone())
    if kind == "adamw":
        options = {"lr": 0.01, "betas": (0.8, 0.95), "eps": 1e-6, "weight_decay": 0.1}
        opt = sr_states.AdamWHip([p], state_dtype=torch.float32, **options)
        native = torch.optim.AdamW([q], foreach=False, **options)
    else:
        options = {"lr": 0.01, "momentum": 0.8}
        opt = sr_states.SGDMHip([p], state_dtype=torch.float32, **options)
        native = torch.optim.SGD([q], foreach=False, **options)
    for step in range(1, 21):
        p.grad = torch.sin(torch.arange(1003, device=cuda) * 0.001 + step)
        q.grad = p.grad.clone()
        opt.step()
        native.step()
        torch.testing.assert_close(p, q, rtol=1e-5, atol=1e-6)
        for name in opt._state_names:
            torch.testing.assert_close(opt.state[p][name], native.state[q][name], rtol=1e-5, atol=1e-6)


def test_rows_at_different_steps_share_one_launch(cuda, monkeypatch):
    """Parameters whose AdamW steps diverge update exactly as separate functional steps."""
    import sr_states

    module = importlib.import_module("sr_states.hip.adamw")
    launch = module._launch
    calls = []

    def count(tables, *args):
        calls.append(tables.nrows)
        return launch(tables, *args)

    monkeypatch.setattr(module, "_launch", count)
    sizes = (1003, 4096 + 7, 77)
    params = [torch.nn.Parameter(torch.linspace(-1, 1, n, device=cuda)) for n in sizes]
    expected = [p.detach().clone() for p in params]
    states = [[torch.zeros(n, device=cuda, dtype=torch.bfloat16) for _ in range(2)] for n in sizes]
    opt = sr_states.AdamWHip(params, lr=0.05, seed=9)
    generator = torch.Generator(device=cuda).manual_seed(3)
    steps = [0, 0, 0]
    for t in range(1, 7):
        skip = t % 3 if t > 1 else None  # one parameter without a gradient per step
        for k, p in enumerate(params):
            p.grad = None if k == skip else torch.randn(p.shape, device=cuda, generator=generator) * 0.1
        calls.clear()
        opt.step()
        assert calls == [len(params) - (skip is not None)]
        for k, p in enumerate(params):
            if k == skip:
                continue
            steps[k] += 1
            sr_states.hip_adamw_step_(expected[k], p.grad, *states[k], lr=0.05, beta1=0.9, beta2=0.999,
                                      eps=1e-8, weight_decay=1e-2, step=steps[k],
                                      seed=sr_states.update_key(9, t, k))
        for k, p in enumerate(params):
            assert opt.state[p]["step"] == steps[k] if steps[k] else p not in opt.state
            assert_bytes(p.detach(), expected[k])
            if steps[k]:
                assert_bytes(opt.state[p]["exp_avg"], states[k][0])
                assert_bytes(opt.state[p]["exp_avg_sq"], states[k][1])
    assert len(set(steps)) > 1


@pytest.mark.parametrize("kind", ["adamw", "sgd"])
@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")  # nothing was launched: the point
def test_graph_capture_is_refused_before_any_launch(cuda, kind):
    """Replaying a captured step would repeat its scalars; the optimizers refuse capture."""
    import sr_states

    cls = sr_states.AdamWHip if kind == "adamw" else sr_states.SGDMHip
    p = torch.nn.Parameter(torch.ones(1000, device=cuda))
    p.grad = torch.full_like(p, 0.5)
    opt = cls([p], lr=0.01)
    opt.step()
    before = p.detach().clone()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="cannot be captured"):
        with torch.cuda.graph(graph):
            opt.step()
    torch.cuda.synchronize()
    assert_bytes(p.detach(), before)
    opt.step()  # eager steps still work after the refused capture
    torch.cuda.synchronize()
    assert not torch.equal(p.detach(), before)
