"""Pinning the optimizer oracles (CPU).

* The C oracle (correctly rounded FP32 ops) and the torch oracle (the
  reference's eager operations) agree: state bytes identical, FP32
  parameters within 1 ulp (torch's CPU square root is not always correctly
  rounded).
* Closed forms: dyadic gradients make proposals exact (tests/test_rng_streams.py:86-119),
  zero gradients give pure decay, the FP8 tie case rounds to even.
* FP32-state trajectories agree with torch.optim.AdamW / SGD, an independent
  implementation (tests/test_reference_optimizers.py:8-40).
* Golden trajectories written by the reference itself
  (tests/golden/reference_trajectories.pt) and the reference's RNG-free v0.1
  fixture (tests/golden/optimizer_v01.pt) are reproduced by the torch
  oracle's optimizer composition.
"""

from __future__ import annotations

from pathlib import Path

import pytest
import torch
from _cases import dyadic_gradient
from conftest import POLICIES, assert_bits_or_nan, ulp_distance

from oracle import c_oracle, sr_oracle

GOLDEN = Path(__file__).parent / "golden"
ADAMW = {"lr": 1e-3, "beta1": 0.9, "beta2": 0.999, "eps": 1e-8, "weight_decay": 1e-2, "step": 100}
SGDM = {"lr": 1e-3, "momentum_factor": 0.9}


def _inputs(kind, n, p_dtype, formats, seed=3):
    gen = torch.Generator().manual_seed(seed)
    p = torch.randn(n, generator=gen).to(p_dtype)
    g = (torch.randn(n, generator=gen) * 0.1).to(p_dtype)
    m = (torch.randn(n, generator=gen) * 0.01).to(formats[0][0])
    if kind == "sgdm":
        return [p, g, m]
    return [p, g, m, (torch.rand(n, generator=gen) * 0.01 + 1e-4).to(formats[1][0])]


@pytest.mark.parametrize("kind", ["adamw", "sgdm"])
@pytest.mark.parametrize("p_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("policy", list(POLICIES))
def test_c_oracle_matches_torch_oracle(kind, p_dtype, policy):
    formats = [POLICIES[policy]] * (2 if kind == "adamw" else 1)
    options = ADAMW if kind == "adamw" else SGDM
    initial = _inputs(kind, 20_011, p_dtype, formats)
    key, offset = 0x1234567, 2**32 - 5
    fmts = tuple(sr_oracle.Fmt(d, r) for d, r in formats)
    if kind == "adamw":
        reference = sr_oracle.adamw_step(*initial, formats=fmts, seed=key, offset=offset, **options)
    else:
        reference = sr_oracle.sgdm_step(*initial, formats=fmts, seed=key, offset=offset, **options)
    ours = [t.clone() for t in initial]
    step = c_oracle.adamw_step_ if kind == "adamw" else c_oracle.sgdm_step_
    step(*ours, formats=formats, seed=key, offset=offset, **options)
    for state, ref in zip(ours[2:], reference[1:]):
        assert_bits_or_nan(state, ref)
    if kind == "sgdm":
        assert_bits_or_nan(ours[0], reference[0])  # no square root: identical
    elif p_dtype == torch.float32:
        assert ulp_distance(ours[0], reference[0]).max() <= 1
    else:
        assert ulp_distance(ours[0].float(), reference[0].float()).max() <= 1 << 16


@pytest.mark.parametrize("kind", ["adamw", "sgdm"])
@pytest.mark.parametrize("policy", ["bf16_sr", "fp16_sr", "fp8e4_sr", "fp8e5_sr"])
def test_dyadic_proposals_are_exact(kind, policy):
    """lr=0 and dyadic gradients: stored states are casts of g/2 and g^2/2 (or g)."""
    dtype, _ = POLICIES[policy]
    g = dyadic_gradient()
    states = [torch.zeros_like(g, dtype=dtype) for _ in range(2 if kind == "adamw" else 1)]
    tensors = [torch.ones_like(g), g, *states]
    options = ({"beta1": 0.5, "beta2": 0.5, "eps": 0.125, "weight_decay": 0.0, "step": 1}
               if kind == "adamw" else {"momentum_factor": 0.5})
    key = sr_oracle.update_key(0xFEDCBA9876543210, (1 << 32) + 1, 7)
    formats = [(dtype, "stochastic")] * len(states)
    step = c_oracle.adamw_step_ if kind == "adamw" else c_oracle.sgdm_step_
    step(*tensors, lr=0.0, formats=formats, seed=key, offset=2**32 - 211, **options)
    proposals = [g * 0.5, g.square() * 0.5] if kind == "adamw" else [g]
    for index, (state, proposal) in enumerate(zip(tensors[2:], proposals)):
        expected = sr_oracle.cast(proposal, dtype=dtype, seed=sr_oracle.state_key(key, index),
                                  offset=2**32 - 211)
        assert_bits_or_nan(state, expected)
    assert torch.equal(tensors[0], torch.ones_like(g))


def test_zero_gradient_is_pure_decay():
    p = torch.linspace(-1, 1, 1003)
    tensors = [p.clone(), torch.zeros_like(p), torch.zeros_like(p, dtype=torch.bfloat16),
               torch.zeros_like(p, dtype=torch.bfloat16)]
    c_oracle.adamw_step_(*tensors, lr=0.01, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.1,
                         step=1, formats=[(torch.bfloat16, "stochastic")] * 2, seed=7)
    assert torch.equal(tensors[0], p * (1.0 - 0.01 * 0.1))
    assert torch.count_nonzero(tensors[2]) == 0 and torch.count_nonzero(tensors[3]) == 0


@pytest.mark.parametrize("n", [1, 1003])
def test_fp8_tie_rounds_to_even_without_fusion(n):
    """tests/test_triton_states.py:85-113: u = 0.9*15/512 - 8/512 lands on 5.5/512 -> 6/512."""
    signs = (1 - 2 * (torch.arange(n) % 2)).float()
    tensors = [torch.ones(n), -signs * (8 / 512), (signs * (15 / 512)).to(torch.float8_e4m3fn)]
    reference = sr_oracle.sgdm_step(*[t.clone() for t in tensors], lr=1e-3, momentum_factor=0.9,
                                    formats=(sr_oracle.Fmt(torch.float8_e4m3fn, "nearest"),), seed=0)
    assert torch.equal(reference[1].float(), signs * (6 / 512))
    c_oracle.sgdm_step_(*tensors, lr=1e-3, momentum_factor=0.9,
                        formats=[(torch.float8_e4m3fn, "nearest")], seed=0)
    assert torch.equal(tensors[2].float(), signs * (6 / 512))


def test_adamw_fp8_first_moment_tie_rounds_to_even():
    """AdamW's analogue of the FP8 tie: m = 2^-9, g = 331/512, beta1 = 0.9.

    The eager order fma(g, 1 - beta1, RN(m beta1)) is exactly the E4M3 tie
    0.06640625 and stores the even 0.0625; the other association and the
    unfused sum lie just above the tie and would store 0.0703125, so the
    case tells the orders apart.
    """
    signs = torch.tensor([1.0, -1.0, 1.0])
    m = (signs * 2.0**-9).to(torch.float8_e4m3fn)
    g = signs * (331 / 512)
    beta1 = torch.tensor(0.9, dtype=torch.float32)
    one_minus = torch.tensor(1.0 - 0.9, dtype=torch.float32)
    scaled = m.float() * beta1
    eager = (g.double() * one_minus.double() + scaled.double()).float()  # one rounding: the FMA
    assert torch.equal(eager, signs * 0.06640625)
    other = (m.float().double() * beta1.double() + (g * one_minus).double()).float()
    unfused = scaled + g * one_minus
    for value in (other, unfused):
        assert not torch.equal(value, eager)
        assert torch.equal(value.to(torch.float8_e4m3fn).float(), signs * 0.0703125)
    options = {"lr": 1e-3, "beta1": 0.9, "beta2": 0.999, "eps": 1e-8, "weight_decay": 0.0, "step": 3}
    formats = ((torch.float8_e4m3fn, "nearest"), (torch.bfloat16, "nearest"))
    tensors = [torch.ones(3), g.clone(), m.clone(), torch.zeros(3, dtype=torch.bfloat16)]
    reference = sr_oracle.adamw_step(*[t.clone() for t in tensors],
                                     formats=tuple(sr_oracle.Fmt(*f) for f in formats), seed=9, **options)
    assert torch.equal(reference[1].float(), signs * 0.0625)
    c_oracle.adamw_step_(*tensors, formats=formats, seed=9, **options)
    assert torch.equal(tensors[2].float(), signs * 0.0625)


@pytest.mark.parametrize("kind", ["adamw", "sgdm"])
def test_fp32_states_match_torch_optim(kind):
    initial = torch.linspace(-1, 1, 257)
    ours = initial.clone()
    theirs = torch.nn.Parameter(initial.clone())
    fmt = (sr_oracle.Fmt(torch.float32, "nearest"),) * (2 if kind == "adamw" else 1)
    if kind == "adamw":
        options = {"lr": 3e-3, "betas": (0.8, 0.95), "eps": 1e-6, "weight_decay": 0.1}
        group = {"params": [ours], "grads": [None], "formats": fmt, "sr_seed": 0, **options}
        opt, native = sr_oracle.AdamWOracle([group]), torch.optim.AdamW([theirs], foreach=False, **options)
    else:
        options = {"lr": 0.03, "momentum": 0.8}
        group = {"params": [ours], "grads": [None], "formats": fmt, "sr_seed": 0, **options}
        opt, native = sr_oracle.SGDMOracle([group]), torch.optim.SGD([theirs], **options)
    for step in range(5):
        gradient = torch.cos(initial * (step + 1))
        group["grads"] = [gradient.clone()]
        theirs.grad = gradient.clone()
        opt.step()
        native.step()
    torch.testing.assert_close(ours, theirs.detach(), rtol=2e-6, atol=2e-7)


def _replay(case):
    """Run the torch oracle's optimizer over a reference trajectory record."""
    dtypes = {"torch.float32": torch.float32, "torch.bfloat16": torch.bfloat16}
    short = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16,
             "e4m3": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}
    params = [raw.view(dtypes[dt]).clone() for raw, dt in zip(case["initial"], case["dtypes"])]
    groups, at = [], 0
    for group in case["groups"]:
        count = len(group["sizes"])
        fmts = tuple(sr_oracle.Fmt(short[f.split("/")[0]], f.split("/")[1]) for f in group["formats"])
        hyper = dict(case["hyper"])
        if "lr" in group:
            hyper["lr"] = group["lr"]
        groups.append({"params": params[at: at + count], "grads": [None] * count, "formats": fmts,
                       "sr_seed": group["sr_seed"], "sr_step": case["initial_sr_step"], **hyper})
        at += count
    cls = sr_oracle.AdamWOracle if case["kind"] == "adamw" else sr_oracle.SGDMOracle
    opt = cls(groups)
    names = cls.state_names
    for step, record in enumerate(case["steps"], start=1):
        flat = iter(record["grads"])
        for group in groups:
            group["grads"] = [None if (g := next(flat)) is None else g.view(p.dtype).clone()
                              for p in group["params"]]
        opt.step()
        assert [g["sr_step"] for g in groups] == record["sr_step"]
        yield step, params, opt, record, names


@pytest.mark.parametrize("name", ["adamw_mixed", "adamw_minifloat", "sgdm_mixed"])
def test_torch_oracle_reproduces_reference_trajectories(name):
    fixture = torch.load(GOLDEN / "reference_trajectories.pt", weights_only=True)
    case = fixture["cases"][name]
    same_platform = fixture["torch"] == torch.__version__ and fixture["cpu_capability"] == torch.backends.cpu.get_cpu_capability()
    for step, params, opt, record, names in _replay(case):
        for p, want_p, want_state in zip(params, record["params"], record["states"]):
            want = want_p.view(p.dtype)
            if same_platform:
                assert torch.equal(p.view(torch.uint8), want.view(torch.uint8)), (name, step)
            else:
                assert ulp_distance(p.float(), want.float()).max() <= (4 if p.dtype == torch.float32 else 1 << 16) * step
            state = opt.state.get(id(p), {})
            for state_name in names:
                if state_name in want_state:
                    assert_bits_or_nan(state[state_name], want_state[state_name].view(state[state_name].dtype))
                else:
                    assert state_name not in state
            if "step" in want_state:
                assert state["step"] == want_state["step"]


def test_torch_oracle_reproduces_the_v01_rng_free_fixture():
    """tests/golden/optimizer_v01.pt (reference data): FP32 and BF16-nearest states.

    Captured from the v0.1 baseline on another platform (macOS ARM, torch
    2.13) whose FP32 kernels round some products differently, so values are
    compared within a few ulps of their own format (the reference replays
    this fixture in-environment for the same reason,
    tests/test_state_formats.py:53-88).  Step counters must match exactly.
    """
    golden = torch.load(GOLDEN / "optimizer_v01.pt", weights_only=True)
    for key, expected in golden["cases"].items():
        cls_name, policy, pdtype_name = key.split("/")
        if policy == "bf16_sr" or "Compiled" in cls_name:
            continue
        pdtype = torch.float32 if pdtype_name == "torch.float32" else torch.bfloat16
        dtype = torch.float32 if policy == "fp32" else torch.bfloat16
        adamw = cls_name.startswith("AdamW")
        params = [torch.linspace(-1, 1, n).to(pdtype) for n in (17, 9, 5)]
        fmt = (sr_oracle.Fmt(dtype, "nearest"),) * (2 if adamw else 1)
        hyper = ({"betas": (0.9, 0.999), "eps": 1e-8, "weight_decay": 1e-2} if adamw else {"momentum": 0.9})
        groups = [
            {"params": params[:2], "grads": [None, None], "formats": fmt, "sr_seed": 2**32 - 13, "lr": 0.01, **hyper},
            {"params": params[2:], "grads": [None], "formats": fmt, "sr_seed": 2**32 - 13, "lr": 0.03, **hyper},
        ]
        opt = (sr_oracle.AdamWOracle if adamw else sr_oracle.SGDMOracle)(groups)
        for step in range(7):
            grads = [None if (step + i) % 4 == 0 else
                     torch.sin(torch.arange(p.numel()).float() * 0.137 + step + i).to(pdtype)
                     for i, p in enumerate(params)]
            groups[0]["grads"], groups[1]["grads"] = grads[:2], grads[2:]
            opt.step()
        for p, want_p, want_state in zip(params, expected["parameters"], expected["states"]):
            want = want_p.view(pdtype)
            limit = 8 if pdtype == torch.float32 else 1 << 16
            assert ulp_distance(p.float(), want.float()).max() <= limit, key
            state = opt.state.get(id(p), {})
            for name in (("exp_avg", "exp_avg_sq") if adamw else ("momentum_buffer",)):
                got = state[name]
                want_state_value = want_state[name].view(got.dtype)
                limit = 8 if got.dtype == torch.float32 else 1 << 16
                assert ulp_distance(got.float(), want_state_value.float()).max() <= limit, (key, name)
            if adamw:
                assert state["step"] == want_state["step"]
