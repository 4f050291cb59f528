"""Fused AdamW / SGDM parity on the GPU.

Bars (from the path's contract):
  * against the C oracle (correctly rounded FP32 ops in the eager order):
    parameter and state bytes identical;
  * against the torch-CPU oracle (the reference's eager operations, whose
    CPU square root is not always correctly rounded): state bytes identical,
    FP32 parameters within 1 ulp (BF16 parameters within 1 BF16 ulp).
Mirrors tests/test_triton_states.py and tests/test_triton_sgdm.py.
"""

from __future__ import annotations

import pytest
import torch
from _cases import dyadic_gradient
from conftest import POLICIES, assert_bits_or_nan, ulp_distance

from oracle import c_oracle, sr_oracle

pytestmark = pytest.mark.gpu

ADAMW = {"lr": 1e-3, "beta1": 0.9, "beta2": 0.999, "eps": 1e-8, "weight_decay": 1e-2, "step": 100}
SGDM = {"lr": 1e-3, "momentum_factor": 0.9}


def _inputs(kind, n, p_dtype, g_dtype, formats, seed=3):
    """Inputs like benchmarks/bench_states.py:87-97, states in their formats."""
    gen = torch.Generator().manual_seed(seed)
    p = torch.randn(n, generator=gen).to(p_dtype)
    g = (torch.randn(n, generator=gen) * 0.1).to(g_dtype)
    m = (torch.randn(n, generator=gen) * 0.01).to(formats[0][0])
    if kind == "sgdm":
        return [p, g, m]
    v = (torch.rand(n, generator=gen) * 0.01 + 1e-4).to(formats[1][0])
    return [p, g, m, v]


def _run_hip(kind, tensors, formats, key, offset, options, block_size=256):
    import sr_states
    from sr_states import StateFormat

    fmts = tuple(StateFormat(d, r) for d, r in formats)
    if kind == "adamw":
        sr_states.hip_adamw_step_(*tensors, seed=key, offset=offset, formats=fmts,
                                  block_size=block_size, **options)
    else:
        sr_states.hip_sgdm_step_(*tensors, seed=key, offset=offset, formats=fmts,
                                 block_size=block_size, **options)


def _run_c(kind, tensors, formats, key, offset, options):
    if kind == "adamw":
        c_oracle.adamw_step_(*tensors, formats=formats, seed=key, offset=offset, **options)
    else:
        c_oracle.sgdm_step_(*tensors, formats=formats, seed=key, offset=offset, **options)


def _run_torch(kind, tensors, formats, key, offset, options):
    fmts = tuple(sr_oracle.Fmt(d, r) for d, r in formats)
    if kind == "adamw":
        return sr_oracle.adamw_step(*tensors, formats=fmts, seed=key, offset=offset, **options)
    return sr_oracle.sgdm_step(*tensors, formats=fmts, seed=key, offset=offset, **options)


FORMAT_SETS = [(POLICIES[name],) * 2 for name in POLICIES] + [
    ((torch.float8_e4m3fn, "stochastic"), (torch.bfloat16, "stochastic")),
    ((torch.float8_e4m3fn, "stochastic"), (torch.float8_e5m2, "nearest")),
    ((torch.float16, "nearest"), (torch.float32, "stochastic")),
]


@pytest.mark.parametrize("kind", ["adamw", "sgdm"])
@pytest.mark.parametrize("p_dtype,g_dtype", [(torch.float32, torch.float32),
                                             (torch.bfloat16, torch.bfloat16),
                                             (torch.float32, torch.bfloat16)])
@pytest.mark.parametrize("formats", FORMAT_SETS, ids=lambda f: "-".join(f"{d}/{r}" for d, r in f))
@pytest.mark.parametrize("n", [1, 1003, 8 * 256 * 3 + 5])
def test_single_tensor_matches_oracles(cuda, kind, p_dtype, g_dtype, formats, n):
    formats = formats[: 2 if kind == "adamw" else 1]
    options = ADAMW if kind == "adamw" else SGDM
    key, offset = 0x9E3779B9, 2**32 - 211
    initial = _inputs(kind, n, p_dtype, g_dtype, formats)

    expected = [t.clone() for t in initial]
    _run_c(kind, expected, formats, key, offset, options)
    actual = [t.to(cuda) for t in initial]
    _run_hip(kind, actual, formats, key, offset, options)
    for index, (a, e) in enumerate(zip(actual, expected)):
        assert_bits_or_nan(a, e, f"tensor {index} vs C oracle")

    reference = _run_torch(kind, initial, formats, key, offset, options)
    for state, ref in zip(actual[2:], reference[1:]):
        assert_bits_or_nan(state, ref, "state vs torch oracle")
    if p_dtype == torch.float32:
        assert ulp_distance(actual[0], reference[0]).max() <= 1
    else:
        assert ulp_distance(actual[0].float(), reference[0].float()).max() <= 1 << 16


@pytest.mark.parametrize("kind", ["adamw", "sgdm"])
@pytest.mark.parametrize("policy", ["bf16_sr", "fp16_sr", "fp8e4_sr", "fp8e5_sr"])
def test_rng_state_bytes_follow_spec_and_flat_shards(cuda, kind, policy):
    """tests/test_triton_states.py:37-67: exact dyadic proposals, stream spec, shards."""
    import sr_states

    dtype, _ = POLICIES[policy]
    g = dyadic_gradient()
    states = [torch.zeros_like(g, dtype=dtype) for _ in range(2 if kind == "adamw" else 1)]
    initial = [torch.ones_like(g), g, *states]
    options = (
        {"beta1": 0.5, "beta2": 0.5, "eps": 0.125, "weight_decay": 0.0, "step": 1}
        if kind == "adamw" else {"momentum_factor": 0.5}
    )
    options["lr"] = 0.0
    key = sr_oracle.update_key(0xFEDCBA9876543210, (1 << 32) + 1, 7)
    offset = (1 << 32) - 211
    formats = [(dtype, "stochastic")] * len(states)

    full = [t.to(cuda) for t in initial]
    _run_hip(kind, full, formats, key, offset, options)
    proposals = [g * 0.5, g.square() * 0.5] if kind == "adamw" else [g]
    for index, (state, proposal) in enumerate(zip(full[2:], proposals)):
        expected = sr_oracle.cast(proposal, dtype=dtype, seed=sr_oracle.state_key(key, index), offset=offset)
        assert_bits_or_nan(state, expected)

    sharded = [t.to(cuda) for t in initial]
    for lo, hi in ((0, 11), (11, 227), (227, 728), (728, g.numel())):
        _run_hip(kind, [t[lo:hi] for t in sharded], formats, key, offset + lo, options)
    for a, b in zip(sharded, full):
        assert torch.equal(a.view(torch.uint8), b.view(torch.uint8))
    assert sr_states.update_key(0xFEDCBA9876543210, (1 << 32) + 1, 7) == key


@pytest.mark.parametrize("kind", ["adamw", "sgdm"])
@pytest.mark.parametrize("block_size", [128, 512, 1024])
def test_block_size_invariance(cuda, kind, block_size):
    formats = [(torch.bfloat16, "stochastic")] * (2 if kind == "adamw" else 1)
    options = ADAMW if kind == "adamw" else SGDM
    initial = _inputs(kind, 40_009, torch.float32, torch.float32, formats)
    base = [t.to(cuda) for t in initial]
    _run_hip(kind, base, formats, 991, 17, options, block_size=256)
    other = [t.to(cuda) for t in initial]
    _run_hip(kind, other, formats, 991, 17, options, block_size=block_size)
    for a, b in zip(base, other):
        assert torch.equal(a.view(torch.uint8), b.view(torch.uint8))


@pytest.mark.parametrize("betas", [(0.0, 0.0), (0.9, 0.999)])
def test_adamw_zero_gradient_and_decay(cuda, betas):
    """tests/test_triton_states.py:261-283."""
    import sr_states

    p = torch.linspace(-1, 1, 1003, device=cuda)
    expected = p * (1.0 - 0.01 * 0.1)
    g = torch.zeros_like(p)
    m = torch.zeros_like(p, dtype=torch.bfloat16)
    v = torch.zeros_like(m)
    sr_states.hip_adamw_step_(p, g, m, v, lr=0.01, beta1=betas[0], beta2=betas[1], eps=1e-8,
                              weight_decay=0.1, step=1, seed=7)
    torch.testing.assert_close(p, expected, rtol=0, atol=0)
    assert torch.count_nonzero(m) == 0 and torch.count_nonzero(v) == 0


def test_round_to_nearest_variants_store_deterministic_bf16_state(cuda):
    """tests/test_reference_optimizers.py:90-103 on the device.

    The RN classes store BF16 states rounded to nearest even: the first
    momentum equals the gradient converted by torch, and neither class's
    states depend on the seed.
    """
    import sr_states

    runs = []
    for seed in (0, 12345):
        q = torch.nn.Parameter(torch.linspace(-1, 1, 1027, device=cuda))
        q.grad = torch.cos(q.detach())
        sgd = sr_states.SGDMHipRN([q], lr=0.01, seed=seed)
        sgd.step()
        assert torch.equal(sgd.state[q]["momentum_buffer"], q.grad.float().to(torch.bfloat16))
        p = torch.nn.Parameter(torch.linspace(-1, 1, 1027, device=cuda))
        p.grad = torch.sin(p.detach())
        adam = sr_states.AdamWHipRN([p], lr=0.01, seed=seed)
        adam.step()
        adam.step()
        states = [adam.state[p][name] for name in ("exp_avg", "exp_avg_sq")]
        assert all(s.dtype == torch.bfloat16 for s in states)
        runs.append((p.detach().clone(), *states))
    for a, b in zip(*runs):
        assert_bits_or_nan(a, b)


@pytest.mark.parametrize("kind", ["adamw", "sgdm"])
def test_validation_and_disjoint_buffers(cuda, kind):
    """tests/test_triton_states.py:213-234."""
    import sr_states
    from sr_states import StateFormat

    formats = [(torch.float32, "nearest")] * (2 if kind == "adamw" else 1)
    tensors = [t.to(cuda) for t in _inputs(kind, 257, torch.float32, torch.float32, formats)]
    function = sr_states.hip_adamw_step_ if kind == "adamw" else sr_states.hip_sgdm_step_
    options = ({**ADAMW, "step": 1} if kind == "adamw" else SGDM) | {"seed": 0}
    with pytest.raises(ValueError, match="overlap"):
        function(tensors[0], tensors[0], *tensors[2:], **options)
    with pytest.raises(ValueError, match="identical shapes"):
        function(tensors[0][:-1], *tensors[1:], **options)
    strided = [torch.zeros(514, device=cuda)[::2] for _ in tensors]
    with pytest.raises(ValueError, match="contiguous"):
        function(*strided, **options)
    if kind == "adamw":
        with pytest.raises(ValueError, match="positive integer"):
            function(*tensors, **{**options, "step": 0})
        with pytest.raises(ValueError, match="state dtype"):
            function(*tensors[:-1], tensors[-1].bfloat16(),
                     formats=(StateFormat(torch.float32), StateFormat(torch.float32)), **options)


@pytest.mark.parametrize("kind", ["adamw", "sgdm"])
def test_refused_updates_launch_nothing_and_keys_wrap_modulo_2_32(cuda, kind):
    """The update entries' tensor checks (triton/_optimizer.py:24-60) refuse before any launch.

    A written tensor sharing a byte with any other operand is refused, a
    gradient only next to the parameter is not; a tensor on another device
    and an FP16 parameter are refused; empty tensors launch nothing.  Keys
    and offsets are taken modulo 2^32, as the ctypes path took them.
    """
    import sr_states

    formats = [(torch.bfloat16, "stochastic")] * (2 if kind == "adamw" else 1)
    function = sr_states.hip_adamw_step_ if kind == "adamw" else sr_states.hip_sgdm_step_
    options = {**ADAMW} if kind == "adamw" else {**SGDM}
    fmts = tuple(sr_states.StateFormat(d, r) for d, r in formats)
    n = 257
    host = _inputs(kind, n, torch.float32, torch.float32, formats)

    def fresh():
        return [t.to(cuda) for t in host]

    def nbytes(t):
        return t.numel() * t.element_size()

    # Every (written, other) pair carved from one byte buffer, the other
    # starting a few bytes before the written one ends.
    for written in [0] + list(range(2, len(host))):
        for other in range(len(host)):
            if other == written:
                continue
            tensors = fresh()
            start = (nbytes(host[written]) - 4) & ~3
            shared = torch.zeros(start + nbytes(host[other]), dtype=torch.uint8, device=cuda)
            for role, begin in ((written, 0), (other, start)):
                tensors[role] = shared[begin:begin + nbytes(host[role])].view(host[role].dtype)
                tensors[role].copy_(host[role])
            before = [t.clone() for t in tensors]
            with pytest.raises(ValueError, match="must not overlap optimizer writes"):
                function(*tensors, seed=5, formats=fmts, **options)
            assert all(torch.equal(a.view(torch.uint8), b.view(torch.uint8)) for a, b in zip(tensors, before))
    # A gradient only adjacent to the parameter is accepted and gives the usual update.
    buffer = torch.empty(2 * n, device=cuda)
    adjacent = fresh()
    buffer[:n].copy_(adjacent[0])
    buffer[n:].copy_(adjacent[1])
    adjacent[0], adjacent[1] = buffer[:n], buffer[n:]
    separate = fresh()
    function(*adjacent, seed=5, formats=fmts, **options)
    function(*separate, seed=5, formats=fmts, **options)
    for a, b in zip(adjacent, separate):
        assert torch.equal(a.view(torch.uint8), b.view(torch.uint8))

    tensors = fresh()
    with pytest.raises(ValueError, match="same GPU device"):
        function(*tensors[:-1], tensors[-1].cpu(), seed=5, formats=fmts, **options)
    with pytest.raises(TypeError, match="FP32 or BF16"):
        function(tensors[0].half(), *tensors[1:], seed=5, formats=fmts, **options)
    empty = [t[:0] for t in tensors]
    function(*empty, seed=5, formats=fmts, **options)

    wrapped, plain = fresh(), fresh()
    function(*wrapped, seed=5 + 3 * 2**32, offset=-2**32 + 11, formats=fmts, **options)
    function(*plain, seed=5, offset=11, formats=fmts, **options)
    for a, b in zip(wrapped, plain):
        assert torch.equal(a.view(torch.uint8), b.view(torch.uint8))
