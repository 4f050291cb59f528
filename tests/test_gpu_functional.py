"""The functional updates and per-parameter optimizers under the reference's names, on the GPU.

``sr_states.reference.adamw_step``/``adamw_step_``/``sgdm_step``/``sgdm_step_``
(reference/adamw.py:12-127, reference/sgd.py:12-84) and
``AdamWReferenceSR/RN``, ``SGDMReferenceSR/RN`` (optim/adamw.py:21-79,
optim/sgd.py:19-69), checked

- against the C oracle (correctly rounded FP32 operations in the eager
  order), parameter and state bytes identical;
- against the torch-CPU oracle, which reads inputs of any dtype through
  ``.float()`` as the reference does: state bytes identical;
- against the fused multi-tensor optimizers, all bytes identical.

Mirrors tests/test_reference_optimizers.py, tests/test_rng_streams.py:122-177
and tests/test_triton_states.py:85-113 of the reference.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from conftest import assert_bits_or_nan, raw_bits

import sr_states
import sr_states.reference as functional
from oracle import c_oracle, sr_oracle
from sr_states import StateFormat, register_rounding, update_key

pytestmark = pytest.mark.gpu

ADAMW = {"lr": 1e-3, "beta1": 0.9, "beta2": 0.999, "eps": 1e-8, "weight_decay": 1e-2, "step": 7}
SGDM = {"lr": 1e-3, "momentum_factor": 0.9}
FORMAT_SETS = [
    ((torch.bfloat16, "stochastic"), (torch.bfloat16, "stochastic")),
    ((torch.float8_e4m3fn, "stochastic"), (torch.bfloat16, "stochastic")),
    ((torch.float16, "nearest"), (torch.float32, "stochastic")),
    ((torch.float8_e5m2, "nearest"), (torch.float8_e4m3fn, "stochastic")),
]
FORMAT_IDS = ["-".join(f"{str(d)[6:]}/{r[0]}" for d, r in f) for f in FORMAT_SETS]
KEY = update_key(11, 3, 2)
OFFSET = 4097


def _inputs(n, p_dtype, g_dtype, state_dtypes, seed=5):
    gen = torch.Generator().manual_seed(seed)
    p = torch.randn(n, generator=gen).to(p_dtype)
    g = (torch.randn(n, generator=gen) * 0.1).to(g_dtype)
    states = [(torch.randn(n, generator=gen) * 0.01).to(state_dtypes[0])]
    if len(state_dtypes) > 1:
        states.append((torch.rand(n, generator=gen) * 0.01 + 1e-4).to(state_dtypes[1]))
    return p, g, states


def _fmts(formats):
    return tuple(StateFormat(d, r) for d, r in formats)


def _c_adamw(p, g, m, v, formats):
    p, g, m, v = (t.clone() for t in (p, g, m, v))
    c_oracle.adamw_step_(p, g, m, v, formats=formats, seed=KEY, offset=OFFSET, **ADAMW)
    return p, m, v


def _c_sgdm(p, g, u, formats):
    p, g, u = (t.clone() for t in (p, g, u))
    c_oracle.sgdm_step_(p, g, u, formats=formats, seed=KEY, offset=OFFSET, **SGDM)
    return p, u


def _assert_all(actual, expected, what):
    for a, e, name in zip(actual, expected, ("parameter", "state 0", "state 1")):
        assert_bits_or_nan(a.cpu(), e, f"{what}: {name}")


@pytest.mark.parametrize("p_dtype,g_dtype", [(torch.float32, torch.float32),
                                             (torch.bfloat16, torch.bfloat16),
                                             (torch.float32, torch.bfloat16)])
@pytest.mark.parametrize("formats", FORMAT_SETS, ids=FORMAT_IDS)
def test_adamw_step_returns_the_oracle_update_and_keeps_its_inputs(cuda, p_dtype, g_dtype, formats):
    p, g, (m, v) = _inputs(1003, p_dtype, g_dtype, [f[0] for f in formats])
    inputs = [t.to(cuda) for t in (p, g, m, v)]
    before = [raw_bits(t.cpu()).clone() for t in inputs]
    result = functional.adamw_step(*inputs, formats=_fmts(formats), seed=KEY, offset=OFFSET, **ADAMW)
    assert [t.dtype for t in result] == [p_dtype, formats[0][0], formats[1][0]]
    _assert_all(result, _c_adamw(p, g, m, v, formats), "adamw_step")
    for t, bits in zip(inputs, before):
        assert torch.equal(raw_bits(t.cpu()), bits), "adamw_step modified an input"


@pytest.mark.parametrize("formats", FORMAT_SETS, ids=FORMAT_IDS)
def test_adamw_step_in_place_updates_without_copies(cuda, formats):
    """Contiguous inputs in their formats go straight to the fused launch."""
    p, g, (m, v) = _inputs(8 * 512 + 3, torch.float32, torch.float32, [f[0] for f in formats])
    tensors = [t.to(cuda) for t in (p, g, m, v)]
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats(cuda)
    resident = torch.cuda.memory_allocated(cuda)
    functional.adamw_step_(*tensors, formats=_fmts(formats), seed=KEY, offset=OFFSET, **ADAMW)
    torch.cuda.synchronize()
    assert torch.cuda.max_memory_allocated(cuda) == resident
    _assert_all((tensors[0], tensors[2], tensors[3]), _c_adamw(p, g, m, v, formats), "adamw_step_")


@pytest.mark.parametrize("formats", FORMAT_SETS, ids=FORMAT_IDS)
def test_adamw_step_reads_states_of_any_dtype_as_the_reference_does(cuda, formats):
    """FP32 states with narrower formats: read exactly, stored through each format.

    States: the torch-CPU oracle, which follows the reference's
    ``.float()``/``cast`` composition, byte for byte.  Parameter: the C
    oracle on FP32 moments (the parameter update uses the unrounded moments,
    so the storage formats do not enter it).
    """
    identity = ((torch.float32, "nearest"),) * 2
    p, g, (m, v) = _inputs(2051, torch.float32, torch.bfloat16, [torch.float32] * 2, seed=9)
    new_p, new_m, new_v = functional.adamw_step(
        *(t.to(cuda) for t in (p, g, m, v)), formats=_fmts(formats), seed=KEY, offset=OFFSET, **ADAMW
    )
    _, torch_m, torch_v = sr_oracle.adamw_step(
        p, g, m, v, formats=tuple(sr_oracle.Fmt(d, r) for d, r in formats), seed=KEY, offset=OFFSET, **ADAMW
    )
    assert_bits_or_nan(new_m.cpu(), torch_m, "exp_avg")
    assert_bits_or_nan(new_v.cpu(), torch_v, "exp_avg_sq")
    c_p, _, _ = _c_adamw(p, g, m, v, identity)
    assert_bits_or_nan(new_p.cpu(), c_p, "parameter")


def test_adamw_step_states_read_either_way_give_the_same_bytes(cuda):
    """States held in their formats, or widened to FP32, give one update."""
    formats = FORMAT_SETS[1]
    p, g, (m, v) = _inputs(3000, torch.bfloat16, torch.bfloat16, [f[0] for f in formats], seed=2)
    args = dict(formats=_fmts(formats), seed=KEY, offset=OFFSET, **ADAMW)
    narrow = functional.adamw_step(*(t.to(cuda) for t in (p, g, m, v)), **args)
    wide = functional.adamw_step(*(t.to(cuda) for t in (p, g)), m.float().to(cuda), v.float().to(cuda), **args)
    _assert_all(wide, [t.cpu() for t in narrow], "widened states")


def test_adamw_step_fp16_parameter_and_gradient(cuda):
    """Parameters outside FP32/BF16 are updated in FP32 and rounded back to nearest."""
    formats = FORMAT_SETS[0]
    p, g, (m, v) = _inputs(1500, torch.float16, torch.float16, [f[0] for f in formats], seed=4)
    result = functional.adamw_step(*(t.to(cuda) for t in (p, g, m, v)), formats=_fmts(formats),
                                   seed=KEY, offset=OFFSET, **ADAMW)
    assert result[0].dtype == torch.float16
    _assert_all(result, _c_adamw(p, g, m, v, formats), "fp16 parameter")


def test_adamw_step_in_place_on_strided_views(cuda):
    """Non-contiguous tensors are updated out of place and written back."""
    formats = FORMAT_SETS[1]
    rows, cols = 37, 53
    p, g, (m, v) = _inputs(rows * cols, torch.float32, torch.float32, [f[0] for f in formats], seed=8)
    views = [t.reshape(cols, rows).to(cuda).t() for t in (p, g, m, v)]
    assert not any(t.is_contiguous() for t in views)
    functional.adamw_step_(*views, formats=_fmts(formats), seed=KEY, offset=OFFSET, **ADAMW)
    contiguous = [t.reshape(cols, rows).t().contiguous().flatten() for t in (p, g, m, v)]
    expected = _c_adamw(*contiguous, formats)
    _assert_all([views[0].flatten(), views[2].flatten(), views[3].flatten()], expected, "strided")


def test_adamw_step_default_formats_are_bf16_stochastic(cuda):
    p, g, (m, v) = _inputs(777, torch.float32, torch.float32, [torch.bfloat16] * 2, seed=6)
    result = functional.adamw_step(*(t.to(cuda) for t in (p, g, m, v)), seed=KEY, offset=OFFSET, **ADAMW)
    expected = _c_adamw(p, g, m, v, ((torch.bfloat16, "stochastic"),) * 2)
    _assert_all(result, expected, "defaults")


@pytest.mark.parametrize("p_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("fmt", [(torch.bfloat16, "stochastic"), (torch.float8_e4m3fn, "stochastic"),
                                 (torch.float16, "nearest"), (torch.float32, "nearest")],
                         ids=lambda f: f"{str(f[0])[6:]}/{f[1][0]}")
def test_sgdm_step_matches_the_oracle_out_of_place_and_in_place(cuda, p_dtype, fmt):
    p, g, (u,) = _inputs(2049, p_dtype, p_dtype, [fmt[0]], seed=12)
    expected = _c_sgdm(p, g, u, (fmt,))
    inputs = [t.to(cuda) for t in (p, g, u)]
    result = functional.sgdm_step(*inputs, formats=_fmts((fmt,)), seed=KEY, offset=OFFSET, **SGDM)
    _assert_all(result, expected, "sgdm_step")
    assert torch.equal(raw_bits(inputs[2].cpu()), raw_bits(u)), "sgdm_step modified the momentum"
    functional.sgdm_step_(*inputs, formats=_fmts((fmt,)), seed=KEY, offset=OFFSET, **SGDM)
    _assert_all((inputs[0], inputs[2]), expected, "sgdm_step_")


def test_sgdm_step_fp8_tie_stores_the_even_neighbour(cuda):
    """u' = RN(RN(0.9 u) + g) = 5.5/512 exactly, stored as 6/512 (tests/test_triton_states.py:85-113)."""
    n = 1003
    signs = (1 - 2 * (torch.arange(n, device=cuda) % 2)).float()
    p = torch.ones(n, device=cuda)
    g = -signs * (8 / 512)
    u = (signs * (15 / 512)).to(torch.float8_e4m3fn)
    functional.sgdm_step_(p, g, u, lr=1e-3, momentum_factor=0.9, seed=0,
                          formats=(StateFormat(torch.float8_e4m3fn, "nearest"),))
    assert torch.equal(u.float(), signs * (6 / 512))


def test_stochastic_round_bf16_is_the_hip_cast(cuda):
    x = torch.randn(10_000, generator=torch.Generator().manual_seed(1))
    got = functional.stochastic_round_bf16(x.to(cuda), seed=KEY, offset=OFFSET)
    assert_bits_or_nan(got.cpu(), c_oracle.cast(x, dtype=torch.bfloat16, seed=KEY, offset=OFFSET), "cast")


# -- per-parameter optimizers --------------------------------------------------

def _model(device, seed=0):
    gen = torch.Generator().manual_seed(seed)
    shapes = [(33, 17), (1000,), (5,), (4, 4, 4)]
    return [torch.nn.Parameter(torch.randn(s, generator=gen).to(device)) for s in shapes]


def _gradients(params, step):
    gen = torch.Generator().manual_seed(100 + step)
    for i, param in enumerate(params):
        # The third parameter never has a gradient: it keeps its index.
        param.grad = None if i == 2 else (torch.randn(param.shape, generator=gen) * 0.1).to(param.device)


def _run(optimizer_type, steps, device, fused_route=True, **options):
    params = _model(device)
    optimizer = optimizer_type([{"params": params[:2]}, {"params": params[2:], "lr": 3e-3}], **options)
    if not fused_route:
        optimizer._fused_route = False
    for step in range(steps):
        _gradients(params, step)
        optimizer.step()
    return params, optimizer


def _assert_same_run(a, b):
    params_a, opt_a = a
    params_b, opt_b = b
    for x, y in zip(params_a, params_b):
        assert_bits_or_nan(x.detach().cpu(), y.detach().cpu(), "parameter")
        state_a, state_b = opt_a.state.get(x, {}), opt_b.state.get(y, {})
        assert set(state_a) == set(state_b)
        for name in state_a:
            if isinstance(state_a[name], torch.Tensor):
                assert_bits_or_nan(state_a[name].cpu(), state_b[name].cpu(), name)
            else:
                assert state_a[name] == state_b[name]


@pytest.mark.parametrize("eager,fused,options", [
    (sr_states.AdamWReferenceSR, sr_states.AdamWHip,
     {"state_format": {"exp_avg": StateFormat(torch.float8_e4m3fn), "exp_avg_sq": StateFormat(torch.bfloat16)},
      "seed": 9}),
    (sr_states.AdamWReferenceRN, sr_states.AdamWHipRN, {"state_dtype": torch.float16}),
    (sr_states.SGDMReferenceSR, sr_states.SGDMHip, {"lr": 1e-2, "state_dtype": torch.float8_e5m2, "seed": 4}),
    (sr_states.SGDMReferenceRN, sr_states.SGDMHipRN, {"lr": 1e-2}),
], ids=["adamw_sr", "adamw_rn", "sgdm_sr", "sgdm_rn"])
def test_per_parameter_optimizers_equal_the_fused_ones(cuda, eager, fused, options):
    """The reference-named optimizers, one parameter at a time, equal the fused ones; so does
    their own fused route."""
    eager_run = _run(eager, 3, cuda, fused_route=False, **options)
    _assert_same_run(eager_run, _run(fused, 3, cuda, **options))
    _assert_same_run(eager_run, _run(eager, 3, cuda, **options))
    # The checkpoint layout is shared: the fused optimizer resumes the eager one.
    params, optimizer = eager_run
    resumed_params = [torch.nn.Parameter(p.detach().clone()) for p in params]
    resumed = fused([{"params": resumed_params[:2]}, {"params": resumed_params[2:], "lr": 3e-3}], **options)
    resumed.load_state_dict(optimizer.state_dict())
    _gradients(params, 3)
    _gradients(resumed_params, 3)
    optimizer.step()
    resumed.step()
    _assert_same_run((params, optimizer), (resumed_params, resumed))


def test_adamw_reference_sr_matches_the_c_oracle_replay(cuda):
    """Keys from (seed, rng step, parameter index) and per-parameter steps."""
    params, _ = _run(sr_states.AdamWReferenceSR, 2, cuda, seed=21)
    replay = [p.detach().cpu().clone() for p in _model("cpu")]
    states = [[torch.zeros_like(p, dtype=torch.bfloat16) for _ in range(2)] for p in replay]
    hyper = {"beta1": 0.9, "beta2": 0.999, "eps": 1e-8, "weight_decay": 1e-2}
    for rng_step in (1, 2):
        _gradients(replay, rng_step - 1)
        for index, (p, (m, v)) in enumerate(zip(replay, states)):
            if p.grad is None:
                continue
            c_oracle.adamw_step_(p, p.grad, m, v, lr=1e-3 if index < 2 else 3e-3, step=rng_step,
                                 formats=((torch.bfloat16, "stochastic"),) * 2,
                                 seed=update_key(21, rng_step, index), **hyper)
    for got, want in zip(params, replay):
        assert_bits_or_nan(got.detach().cpu(), want, "parameter")


ROUND_DOWN = "sr_states_test_toward_zero"


def _toward_zero(x, *, dtype, seed, offset):
    return (x.view(torch.int32) & -65536).view(torch.float32).to(dtype)


def test_registered_rules_are_applied_by_the_functional_and_eager_updates(cuda):
    """A rule without a HIP implementation: FP32 moments, then the registered routine."""
    try:
        register_rounding(ROUND_DOWN, torch.bfloat16, reference=_toward_zero)
    except ValueError:
        pass  # registered by an earlier run in this process
    fmt = StateFormat(torch.bfloat16, ROUND_DOWN)
    p, g, (m, v) = _inputs(1111, torch.float32, torch.float32, [torch.bfloat16] * 2, seed=13)
    new_p, new_m, new_v = functional.adamw_step(*(t.to(cuda) for t in (p, g, m, v)), formats=(fmt, fmt),
                                                seed=KEY, offset=OFFSET, **ADAMW)
    c_p, c_m, c_v = _c_adamw(p, g, m.float(), v.float(), ((torch.float32, "nearest"),) * 2)
    assert_bits_or_nan(new_p.cpu(), c_p, "parameter")
    assert_bits_or_nan(new_m.cpu(), _toward_zero(c_m, dtype=torch.bfloat16, seed=0, offset=0), "exp_avg")
    assert_bits_or_nan(new_v.cpu(), _toward_zero(c_v, dtype=torch.bfloat16, seed=0, offset=0), "exp_avg_sq")
    with pytest.raises(ValueError, match="no HIP implementation"):
        sr_states.AdamWHip(_model(cuda), state_format=fmt)
    # The eager optimizer's first step on parameter 0 (zero moments, key of index 0).
    params, optimizer = _run(sr_states.AdamWReferenceSR, 1, cuda, state_format=fmt)
    p0 = _model("cpu")[0].detach()
    _gradients([p0], 0)
    zeros = torch.zeros_like(p0)
    c_p, c_m, c_v = (t.clone() for t in (p0, zeros, zeros))
    c_oracle.adamw_step_(c_p, p0.grad, c_m, c_v, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8,
                         weight_decay=1e-2, step=1, formats=((torch.float32, "nearest"),) * 2,
                         seed=update_key(0, 1, 0))
    state = optimizer.state[params[0]]
    assert_bits_or_nan(params[0].detach().cpu(), c_p, "eager parameter")
    assert_bits_or_nan(state["exp_avg"].cpu(), _toward_zero(c_m, dtype=torch.bfloat16, seed=0, offset=0), "m")
    assert_bits_or_nan(state["exp_avg_sq"].cpu(), _toward_zero(c_v, dtype=torch.bfloat16, seed=0, offset=0), "v")


@pytest.mark.parametrize("hyper", [
    {"lr": -1e-3},
    {"weight_decay": -0.05},
    {"eps": -1e-3},
    {"beta1": 1.25, "beta2": 0.0},
    {"beta1": -0.5, "lr": 2.0, "weight_decay": 3.0},
], ids=lambda h: ",".join(f"{k}={v}" for k, v in h.items()))
def test_reference_adamw_takes_any_hyperparameters_as_the_reference_does(cuda, hyper):
    """reference/adamw.py:54-105 checks no hyperparameter; nor does sr_states.reference.

    Values the optimizers refuse (a negative learning rate, epsilon or
    weight decay; betas outside [0, 1)) update as the C oracle does, byte
    for byte; a negative epsilon makes some denominators negative.
    """
    formats = FORMAT_SETS[1]
    options = {**ADAMW, **hyper}
    p, g, (m, v) = _inputs(3001, torch.float32, torch.float32, [f[0] for f in formats], seed=21)
    want = [t.clone() for t in (p, g, m, v)]
    c_oracle.adamw_step_(*want, formats=formats, seed=KEY, offset=OFFSET, **options)
    got = [t.to(cuda) for t in (p, g, m, v)]
    functional.adamw_step_(*got, formats=_fmts(formats), seed=KEY, offset=OFFSET, **options)
    _assert_all([got[0], got[2], got[3]], [want[0], want[2], want[3]], f"adamw_step_ {hyper}")
    out = functional.adamw_step(*(t.to(cuda) for t in (p, g, m, v)), formats=_fmts(formats), seed=KEY,
                                offset=OFFSET, **options)
    _assert_all(out, [want[0], want[2], want[3]], f"adamw_step {hyper}")
    with pytest.raises(ValueError, match="invalid"):
        sr_states.hip_adamw_step_(*got, formats=_fmts(formats), seed=KEY, offset=OFFSET, **options)


@pytest.mark.parametrize("step", [np.int64(7), 7.0, 2.5, np.float32(3.0), True], ids=repr)
def test_reference_adamw_takes_any_real_step_as_the_reference_does(cuda, step):
    """reference/adamw.py:73-84 checks only step >= 1 and uses it in the bias corrections."""
    formats = FORMAT_SETS[0]
    options = {**ADAMW, "step": step}
    p, g, (m, v) = _inputs(2003, torch.float32, torch.float32, [f[0] for f in formats], seed=19)
    want = [t.clone() for t in (p, g, m, v)]
    c_oracle.adamw_step_(*want, formats=formats, seed=KEY, offset=OFFSET, **options)
    out = functional.adamw_step(*(t.to(cuda) for t in (p, g, m, v)), formats=_fmts(formats), seed=KEY,
                                offset=OFFSET, **options)
    _assert_all(out, [want[0], want[2], want[3]], f"step {step!r}")


def test_reference_adamw_reads_integer_and_boolean_tensors_through_float(cuda):
    """reference/adamw.py:79-89 reads every input with ``.float()``, returns the parameter
    through ``.to(parameter.dtype)`` (truncation for integers) and each moment through its
    format; the in-place update copies them back into the tensors' own dtypes."""
    formats = FORMAT_SETS[0]
    gen = torch.Generator().manual_seed(13)
    n = 1999
    p = torch.randint(-60, 60, (n,), generator=gen, dtype=torch.int32)
    g = torch.randint(0, 2, (n,), generator=gen).bool()
    m = torch.randint(-2, 3, (n,), generator=gen, dtype=torch.int16)
    v = torch.randint(0, 4, (n,), generator=gen, dtype=torch.int64)
    new_p, new_m, new_v = functional.adamw_step(*(t.to(cuda) for t in (p, g, m, v)), formats=_fmts(formats),
                                                seed=KEY, offset=OFFSET, **ADAMW)
    p32, g32, m32, v32 = (t.float() for t in (p, g, m, v))
    c_oracle.adamw_step_(p32, g32, m32, v32, formats=((torch.float32, "nearest"),) * 2, seed=KEY, offset=OFFSET,
                         **ADAMW)
    assert new_p.dtype == torch.int32 and torch.equal(new_p.cpu(), p32.to(torch.int32))
    for k, (got, wide, (dtype, rule)) in enumerate(zip((new_m, new_v), (m32, v32), formats)):
        want = c_oracle.cast(wide, dtype=dtype, rounding=rule, seed=sr_oracle.state_key(KEY, k), offset=OFFSET)
        assert_bits_or_nan(got.cpu(), want, f"state {k}")
    tensors = [t.to(cuda) for t in (p, g, m, v)]
    functional.adamw_step_(*tensors, formats=_fmts(formats), seed=KEY, offset=OFFSET, **ADAMW)
    assert torch.equal(tensors[0].cpu(), new_p.cpu())
    assert torch.equal(tensors[2].cpu(), new_m.cpu().to(torch.int16))
    assert torch.equal(tensors[3].cpu(), new_v.cpu().to(torch.int64))


def test_reference_adamw_refuses_only_what_the_launch_cannot_divide_by(cuda):
    p, g, (m, v) = _inputs(64, torch.float32, torch.float32, [torch.bfloat16] * 2)
    p, g, m, v = (t.to(cuda) for t in (p, g, m, v))
    for beta2 in (1.0, 1.5, -3.0):
        with pytest.raises(ValueError, match=r"sqrt\(1 - beta2\*\*step\)"):
            functional.adamw_step_(p, g, m, v, **{**ADAMW, "beta2": beta2, "step": 1})
    with pytest.raises(ZeroDivisionError):  # 1 - beta1**step == 0, as in the reference
        functional.adamw_step_(p, g, m, v, **{**ADAMW, "beta1": 1.0})


@pytest.mark.parametrize("hyper", [{"lr": -0.01}, {"momentum_factor": 1.0}, {"momentum_factor": -0.9, "lr": 3.0},
                                   {"momentum_factor": 1.5}],
                         ids=lambda h: ",".join(f"{k}={v}" for k, v in h.items()))
def test_reference_sgdm_takes_any_hyperparameters_as_the_reference_does(cuda, hyper):
    """reference/sgd.py:44-72 checks no hyperparameter; nor does sr_states.reference."""
    formats = ((torch.float8_e4m3fn, "stochastic"),)
    options = {**SGDM, **hyper}
    p, g, (u,) = _inputs(3001, torch.bfloat16, torch.float32, [formats[0][0]], seed=22)
    want = [t.clone() for t in (p, g, u)]
    c_oracle.sgdm_step_(*want, formats=formats, seed=KEY, offset=OFFSET, **options)
    got = [t.to(cuda) for t in (p, g, u)]
    functional.sgdm_step_(*got, formats=_fmts(formats), seed=KEY, offset=OFFSET, **options)
    _assert_all([got[0], got[2]], [want[0], want[2]], f"sgdm_step_ {hyper}")
    with pytest.raises(ValueError, match="invalid"):
        sr_states.hip_sgdm_step_(*got, formats=_fmts(formats), seed=KEY, offset=OFFSET, **options)


def _route_counter(monkeypatch):
    """Counts the groups the reference-named optimizers run on the fused launch."""
    from sr_states.optim import eager as eager_module

    counts = {"fused": 0}
    original = eager_module._FusedGroups._fused_prepare

    def counting(self, group, formats, items):
        prepared = original(self, group, formats, items)
        counts["fused"] += prepared is not None
        return prepared

    monkeypatch.setattr(eager_module._FusedGroups, "_fused_prepare", counting)
    return counts


@pytest.mark.parametrize("cls", [sr_states.AdamWReferenceSR, sr_states.SGDMReferenceSR], ids=lambda c: c.__name__)
def test_reference_named_optimizers_fall_back_per_parameter_where_the_fused_launch_refuses(cuda, cls,
                                                                                            monkeypatch):
    """Groups the fused launch refuses update one parameter at a time, as before.

    Each case runs both routes from the same start and compares every byte:
    a strided parameter, two parameters sharing storage (updated in order,
    the second reading what the first wrote) and a learning rate set below
    zero after construction.  (Registered rules without a HIP kernel run per
    parameter too: test_registered_rules_are_applied_by_the_functional_and_
    eager_updates.)
    """
    counts = _route_counter(monkeypatch)
    lr = 1e-2

    def run(make_params, fused_route):
        params = make_params()
        optimizer = cls(params, lr=lr, seed=5)
        optimizer._fused_route = fused_route
        for step in range(3):
            _gradients(params, step)
            optimizer.step()
        return params, optimizer

    def plain():
        return _model(cuda, seed=1)

    def strided():
        params = _model(cuda, seed=1)
        gen = torch.Generator().manual_seed(3)
        params[0] = torch.nn.Parameter(torch.randn(17, 33, generator=gen).to(cuda).t())
        return params

    def shared():
        base = torch.randn(2000, generator=torch.Generator().manual_seed(4)).to(cuda)
        return [torch.nn.Parameter(base[:1000]), torch.nn.Parameter(base[500:1500])]

    counts["fused"] = 0
    _assert_same_run(run(plain, True), run(plain, False))
    assert counts["fused"] == 3  # three steps, one group, all on the fused launch
    for make in (strided, shared):
        counts["fused"] = 0
        _assert_same_run(run(make, True), run(make, False))
        assert counts["fused"] == 0, make.__name__
    # A negative learning rate set after construction: the reference computes with it.
    routes = []
    for fused_route in (True, False):
        params = _model(cuda, seed=2)
        optimizer = cls(params, lr=lr, seed=5)
        optimizer._fused_route = fused_route
        optimizer.param_groups[0]["lr"] = -lr
        counts["fused"] = 0
        for step in range(2):
            _gradients(params, step)
            optimizer.step()
        assert counts["fused"] == 0
        routes.append((params, optimizer))
    _assert_same_run(*routes)
