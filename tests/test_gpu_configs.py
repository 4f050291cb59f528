"""The benchmark configurations (C1-C5 and the north star) at their full sizes on the GPU.

Every element's update depends only on its own inputs, its flat index and the
update key (sr_states/_hash.py:31-50; triton/adamw.py:102-157), so the C
oracle run on a contiguous chunk of a tensor, with ``offset`` set to the
chunk's first index, must reproduce the GPU's bytes for that chunk exactly.
Each test runs the full-size workload through the multi-tensor optimizer (or
the cast), then replays sampled chunks (first and last elements of the
tensor, aligned and unaligned interior starts) through the oracle for the same
steps and compares parameters and stored states bit for bit.  Whole-tensor
properties cover what sampling cannot: E4M3 saturation never produces a
non-finite moment, and stored steps and RNG steps advance once per step.

The inputs are bench.py's workload definitions, including C4's saturating and
infinite gradients and C5's zero and subnormal-magnitude gradients.
"""

from __future__ import annotations

import gc
import math
import random

import pytest
import torch
from conftest import assert_bits_or_nan

import bench
from oracle import c_oracle, sr_oracle

pytestmark = pytest.mark.gpu

CHUNK = 4099  # odd, so chunk boundaries fall inside vector groups


def _chunks(numel: int, count: int, seed: int) -> list[tuple[int, int]]:
    """(start, length) of `count` chunks: the head, the tail and random interior starts."""
    rng = random.Random(seed)
    starts = {0, max(0, numel - CHUNK)}
    while len(starts) < min(count, max(1, numel // CHUNK)):
        starts.add(rng.randrange(0, max(1, numel - CHUNK)))
    return [(s, min(CHUNK, numel - s)) for s in sorted(starts)]


def _sample_tensors(count: int, total: int, seed: int) -> list[int]:
    rng = random.Random(seed)
    picks = {0, total - 1}
    while len(picks) < min(count, total):
        picks.add(rng.randrange(total))
    return sorted(picks)


def _run_optimizer_config(cuda, workload, steps, *, tensors, chunks):
    spec = bench.WORKLOADS[workload]
    params, opt = bench.make_optimizer(spec, cuda)
    names = opt._state_names
    formats = tuple(tuple(f) for f in spec["formats"])
    hp = spec["hparams"]
    adamw = spec["optimizer"] == "adamw"
    # The first step allocates the states (zeros); snapshot sampled chunks
    # before it, with zero states.
    samples = []
    for index in _sample_tensors(tensors, len(params), seed=len(params) * steps):
        p = params[index]
        flat_p, flat_g = p.detach().view(-1), p.grad.view(-1)
        for start, length in _chunks(p.numel(), chunks, seed=index):
            sl = slice(start, start + length)
            p0 = flat_p[sl].cpu().clone()
            g0 = flat_g[sl].cpu().clone()
            states = [torch.zeros(length, dtype=dtype) for dtype, _ in formats]
            samples.append((index, start, length, p0, g0, states))
    for _ in range(steps):
        opt.step()
    torch.cuda.synchronize()

    for index, start, length, p_ref, g_ref, states in samples:
        for t in range(1, steps + 1):
            key = sr_oracle.update_key(spec["seed"], t, index)
            if adamw:
                beta1, beta2 = hp["betas"]
                c_oracle.adamw_step_(p_ref, g_ref, *states, lr=hp["lr"], beta1=beta1, beta2=beta2,
                                     eps=hp["eps"], weight_decay=hp["weight_decay"], step=t,
                                     formats=formats, seed=key, offset=start)
            else:
                c_oracle.sgdm_step_(p_ref, g_ref, *states, lr=hp["lr"],
                                    momentum_factor=hp["momentum"], formats=formats, seed=key,
                                    offset=start)
        p = params[index]
        sl = slice(start, start + length)
        what = f"{workload} tensor {index} [{start}, {start + length})"
        assert_bits_or_nan(p.detach().view(-1)[sl].cpu(), p_ref, f"{what} parameter")
        for name, expected in zip(names, states):
            got = opt.state[p][name].view(-1)[sl].cpu()
            assert_bits_or_nan(got, expected, f"{what} {name}")
        if adamw:
            assert opt.state[p]["step"] == steps
    assert opt._rng_step() == steps
    return params, opt, samples


@pytest.fixture(autouse=True)
def _release_device_memory():
    """Return the full-size workloads' memory before the next test allocates."""
    yield
    gc.collect()
    if torch.cuda.is_available():
        torch.cuda.empty_cache()


@pytest.mark.parametrize("rounding", ["stochastic", "nearest"])
def test_c1_cast_full_size(cuda, rounding):
    """Config 1: 2^24 N(0,1) values from CPU seed 0, seed 7, every output byte."""
    import sr_states

    x = torch.randn(1 << 24, generator=torch.Generator().manual_seed(0))
    got = sr_states.cast(x.to(cuda), dtype=torch.bfloat16, rounding=rounding, seed=7).cpu()
    expected = c_oracle.cast(x, dtype=torch.bfloat16, rounding=rounding, seed=7)
    assert_bits_or_nan(got, expected, f"C1 {rounding}")
    if rounding == "nearest":
        assert_bits_or_nan(got, x.to(torch.bfloat16), "C1 nearest vs torch RNE")
    else:
        # Every output is one of the input's two BF16 neighbours (finite inputs).
        lo, hi = sr_oracle.bf16_neighbors(x)
        assert bool(((got.float() == lo.float()) | (got.float() == hi.float())).all())


def test_c2_single_tensor_ten_steps(cuda):
    """Config 2: one 2^26-element tensor, BF16-SR moments, 10 steps."""
    _run_optimizer_config(cuda, "c2_single_2e26", 10, tensors=1, chunks=24)


def test_c3_gpt2_shapes_bf16_gradients(cuda):
    """Config 3: 148 GPT-2-small tensors in one launch, FP32 parameters, BF16 gradients."""
    params, opt, samples = _run_optimizer_config(cuda, "c3_gpt2", 3, tensors=12, chunks=4)
    assert len(params) == 148 and sum(p.numel() for p in params) == 124_439_808
    assert len({index for index, *_ in samples}) == 12


def test_c4_mixed_fp8_saturation(cuda):
    """Config 4 (1.55 G elements): E4M3-SR first moment saturates at +-448, never Inf/NaN."""
    params, opt, samples = _run_optimizer_config(cuda, "c4_fp8_mixed", 2, tensors=6, chunks=4)
    saturated = 0
    for p in params:
        m = opt.state[p]["exp_avg"].view(torch.uint8)
        # E4M3fn: exponent and mantissa all ones (0x7F / 0xFF) is NaN.
        assert not bool(((m & 0x7F) == 0x7F).any()), "E4M3 moment holds NaN"
        saturated += int(((m & 0x7F) == 0x7E).sum())
    assert saturated > 0, "no first-moment element reached the E4M3 maximum"
    # Sampled chunks contain injected +-5000 gradients.
    assert any(bool((g.abs() == 5000).any()) for _, _, _, _, g, _ in samples)


def test_north_star_full_size(cuda):
    """The headline workload bench.py times: BF16-SR m and v over the 1.55 G-element set, 2 steps."""
    spec = bench.WORKLOADS["north_star"]
    assert sum(math.prod(s) for s in spec["shapes"]) == 1_547_698_176
    assert tuple(tuple(f) for f in spec["formats"]) == ((torch.bfloat16, "stochastic"),) * 2
    params, opt, samples = _run_optimizer_config(cuda, "north_star", 2, tensors=6, chunks=4)
    assert len(params) == 50 and len({index for index, *_ in samples}) == 6
    for p in params:
        for name in ("exp_avg", "exp_avg_sq"):
            assert opt.state[p][name].dtype == torch.bfloat16


def test_c4_literal_24_blocks(cuda):
    """Config 4 at its literal size: 4.99 G elements over 169 tensors, one step."""
    spec = bench.WORKLOADS["c4_fp8_24block"]
    assert sum(math.prod(s) for s in spec["shapes"]) == 4_988_076_032
    params, opt, _ = _run_optimizer_config(cuda, "c4_fp8_24block", 1, tensors=8, chunks=3)
    assert len(params) == 169


def test_c5_sgdm_fp16_twenty_steps(cuda):
    """Config 5: 256 x 2048^2 SGDM, FP16-SR momentum, zero and subnormal gradients, 20 steps."""
    params, opt, samples = _run_optimizer_config(cuda, "c5_sgdm_fp16", 20, tensors=6, chunks=4)
    grads = torch.cat([g for _, _, _, _, g, _ in samples])
    assert 0.03 < float((grads == 0).float().mean()) < 0.07
    # 1% injected below 2^-14, plus the N(0, 1e-2) draws that land there
    # (P(|N(0, 1e-2)| < 2^-14) = 0.49%, times the remaining 94%): 1.46%.
    tiny = (grads != 0) & (grads.abs() < 2.0**-14)
    assert 0.011 < float(tiny.float().mean()) < 0.018


@pytest.mark.parametrize("workload", ["bf16_params_e4m3_bf16sr", "bf16_params_fp16sr"])
def test_bf16_parameter_launches_full_size(cuda, workload):
    """The arithmetic-heaviest launches at the north star's size, 3 steps.

    BF16 parameters and gradients with an E4M3-SR first moment, or FP16-SR
    moments: every element goes through the short square root and division
    (with their library fallbacks where the moments or quotients are tiny)
    and, for E4M3, the single-form FP8 encoder, at 3 M tiles.
    """
    spec = bench.WORKLOADS[workload]
    assert spec["p_dtype"] == torch.bfloat16 and spec["g_dtype"] == torch.bfloat16
    params, opt, samples = _run_optimizer_config(cuda, workload, 3, tensors=6, chunks=4)
    assert len({index for index, *_ in samples}) == 6
