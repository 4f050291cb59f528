"""HIP cast parity: bit-exact against both oracles (NaN payload excluded).

Mirrors the reference's GPU cast tests (tests/test_triton_casts.py,
tests/test_minifloat_gpu.py:38-50, tests/test_triton_sr_cast.py).
"""

from __future__ import annotations

import pytest
import torch
from _cases import boundary_inputs, cast_cases, random_words, rn_midpoint_words
from conftest import RULES, STATE_DTYPES, assert_bits_or_nan

from oracle import c_oracle, sr_oracle

pytestmark = pytest.mark.gpu

MINIFLOATS = (torch.float16, torch.float8_e4m3fn, torch.float8_e5m2)


def _inputs(dtype):
    parts = [random_words(10007, 541), torch.randn(4099, generator=torch.Generator().manual_seed(5)) * 300]
    if dtype in MINIFLOATS:
        parts.append(boundary_inputs(dtype))
    return torch.cat(parts)


@pytest.mark.parametrize("dtype", STATE_DTYPES)
@pytest.mark.parametrize("rounding", RULES)
def test_cast_matches_both_oracles(cuda, dtype, rounding):
    import sr_states

    x = _inputs(dtype)
    options = {"dtype": dtype, "rounding": rounding, "seed": 2**32 - 7, "offset": 2**32 - 93}
    expected = sr_oracle.cast(x, **options)
    assert_bits_or_nan(c_oracle.cast(x, **options), expected, "C oracle vs torch oracle")
    actual = sr_states.cast(x.to(cuda), **options)
    assert actual.device == x.to(cuda).device
    assert_bits_or_nan(actual, expected, f"HIP {dtype} {rounding}")


@pytest.mark.parametrize("dtype", STATE_DTYPES)
@pytest.mark.parametrize("rounding", RULES)
@pytest.mark.parametrize("block_size,num_warps", [(128, 1), (256, 4), (1024, 8), (4096, 2)])
def test_cast_launch_shapes_do_not_change_results(cuda, dtype, rounding, block_size, num_warps):
    from sr_states.hip import cast

    x = _inputs(dtype)
    options = {"dtype": dtype, "rounding": rounding, "seed": 77, "offset": 2**32 - 19}
    expected = c_oracle.cast(x, **options)
    actual = cast(x.to(cuda), block_size=block_size, num_warps=num_warps, **options)
    assert_bits_or_nan(actual, expected)


def test_bf16_cast_contract_cases(cuda):
    """benchmarks/cast_checks.py:70-80: fresh outputs, input untouched, exact bits."""
    from sr_states.hip import rn_cast_bf16, sr_cast_bf16

    for x, seed, offset in cast_cases():
        xd = x.to(cuda)
        original = xd.view(torch.int32).clone()
        expected = sr_oracle.stochastic_round_bf16(x, seed=seed, offset=offset)
        for store_mode in ("convert", "bits"):
            first = sr_cast_bf16(xd, seed=seed, offset=offset, store_mode=store_mode)
            second = sr_cast_bf16(xd, seed=seed, offset=offset, store_mode=store_mode)
            assert_bits_or_nan(first, expected)
            assert_bits_or_nan(second, expected)
            if x.numel():
                assert first.data_ptr() != second.data_ptr()
                assert first.data_ptr() != xd.data_ptr()
        assert torch.equal(xd.view(torch.int32), original)
        assert_bits_or_nan(rn_cast_bf16(xd), x.to(torch.bfloat16))
    x = rn_midpoint_words()
    assert_bits_or_nan(rn_cast_bf16(x.to(cuda)), x.to(torch.bfloat16))


@pytest.mark.parametrize("dtype", STATE_DTYPES)
def test_stream_partition_invariance(cuda, dtype):
    import sr_states

    x = torch.linspace(-3, 7, 10003).to(cuda)
    seed, offset, split = 77, 2**32 - 19, 4101
    whole = sr_states.cast(x, dtype=dtype, seed=seed, offset=offset)
    parts = torch.cat(
        [
            sr_states.cast(x[:split], dtype=dtype, seed=seed, offset=offset),
            sr_states.cast(x[split:], dtype=dtype, seed=seed, offset=offset + split),
        ]
    )
    assert_bits_or_nan(parts, whole)


@pytest.mark.parametrize("dtype,ulp", [(torch.bfloat16, 2.0**-7), (torch.float16, 2.0**-10),
                                       (torch.float8_e4m3fn, 2.0**-3), (torch.float8_e5m2, 2.0**-2)])
def test_seed_reproducibility_and_counter_periodicity(cuda, dtype, ulp):
    """tests/test_seed_reproducibility.py:6-36 on the device, per stochastic format.

    The same seed and offset reproduce the output; another seed changes the
    choices of inexact values; seed and offset act modulo 2^32, for negative
    and very large Python integers too.
    """
    import sr_states

    x = torch.linspace(-10, 10, 10003, device=cuda)
    first = sr_states.cast(x, dtype=dtype, seed=1234, offset=77)
    assert_bits_or_nan(sr_states.cast(x, dtype=dtype, seed=1234, offset=77), first)
    inexact = torch.full((4096,), 1.0 + ulp / 4, device=cuda)
    assert not torch.equal(sr_states.cast(inexact, dtype=dtype, seed=1).float(),
                           sr_states.cast(inexact, dtype=dtype, seed=2).float())
    y = torch.linspace(-1, 1, 1003, device=cuda)
    expected = sr_states.cast(y, dtype=dtype, seed=7, offset=31)
    for periods in (-(2**60), -1, 1, 2**60):
        actual = sr_states.cast(y, dtype=dtype, seed=7 + periods * 2**32, offset=31 + periods * 2**32)
        assert_bits_or_nan(actual, expected, f"{periods} periods")


def test_unaligned_noncontiguous_and_empty_inputs(cuda):
    import sr_states

    base = torch.linspace(-1, 1, 4101, device=cuda)
    unaligned = base[1:]  # 4-byte offset: takes the scalar path
    expected = c_oracle.cast(unaligned.cpu(), dtype=torch.bfloat16, seed=3, offset=5)
    assert_bits_or_nan(sr_states.cast(unaligned, dtype=torch.bfloat16, seed=3, offset=5), expected)
    strided = torch.linspace(-1, 1, 35, device=cuda).reshape(5, 7).T
    for dtype in STATE_DTYPES:
        got = sr_states.cast(strided, dtype=dtype, seed=7)
        assert got.shape == strided.shape
        assert_bits_or_nan(got, sr_states.cast(strided.contiguous(), dtype=dtype, seed=7))
        empty = sr_states.cast(torch.empty(0, 3, device=cuda), dtype=dtype)
        assert empty.shape == (0, 3) and empty.dtype == dtype


def test_cast_rejects_invalid_inputs(cuda):
    from sr_states.hip import cast, rn_cast_bf16, sr_cast_bf16

    with pytest.raises(TypeError, match="float32"):
        rn_cast_bf16(torch.ones(4, device=cuda, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="contiguous"):
        rn_cast_bf16(torch.ones(8, device=cuda)[::2])
    with pytest.raises(ValueError, match="block_size"):
        sr_cast_bf16(torch.ones(4, device=cuda), seed=1, block_size=3)
    with pytest.raises(ValueError, match="num_warps"):
        cast(torch.ones(4, device=cuda), dtype=torch.bfloat16, num_warps=3)
    with pytest.raises(ValueError, match="store_mode"):
        sr_cast_bf16(torch.ones(4, device=cuda), seed=1, store_mode="invalid")


def test_cast_into_an_output_buffer(cuda):
    """native_cast(out=...) writes the oracle's bytes into a given buffer and
    refuses, without writing, outputs on another device, of another shape or
    dtype, strided, or sharing a byte with the input."""
    from sr_states import _lib
    from sr_states.hip.cast import native_cast

    x = _inputs(torch.bfloat16).to(cuda)
    sr = _lib.RULE_CODES["stochastic"]
    expected = sr_oracle.cast(x.cpu(), dtype=torch.bfloat16, rounding="stochastic", seed=9, offset=4)
    out = torch.full(x.shape, 7.0, device=cuda, dtype=torch.bfloat16)
    assert native_cast(x, dtype=torch.bfloat16, rule=sr, seed=9, offset=4, out=out) is out
    assert_bits_or_nan(out, expected, "into out")
    bad = [torch.empty(x.shape, dtype=torch.bfloat16),  # host memory
           torch.empty(x.numel() - 1, device=cuda, dtype=torch.bfloat16),
           torch.empty(x.shape, device=cuda, dtype=torch.float16),
           torch.empty(2 * x.numel(), device=cuda, dtype=torch.bfloat16)[::2]]
    for candidate in bad:
        before = candidate.clone()
        with pytest.raises(ValueError, match="contiguous tensor of the requested dtype, shape and device"):
            native_cast(x, dtype=torch.bfloat16, rule=sr, seed=9, out=candidate)
        assert torch.equal(candidate.contiguous().view(torch.uint8), before.contiguous().view(torch.uint8))
    storage = torch.zeros(2 * x.numel(), device=cuda)
    inside = storage[: x.numel()]
    inside.copy_(x)
    overlapping = storage[x.numel() // 2:].view(torch.bfloat16)[: x.numel()]
    before = storage.clone()
    with pytest.raises(ValueError, match="overlap"):
        native_cast(inside, dtype=torch.bfloat16, rule=sr, seed=9, out=overlapping)
    assert torch.equal(storage.view(torch.int32), before.view(torch.int32))  # bits: x holds NaNs


def test_casts_and_updates_from_several_threads(cuda):
    """The native entries release the GIL while launching: four threads, each on
    its own stream, cast and update their own tensors; every result equals the
    oracle's."""
    import threading

    import sr_states

    x = _inputs(torch.bfloat16)
    options = {"dtype": torch.bfloat16, "rounding": "stochastic"}
    gen = torch.Generator().manual_seed(17)
    p, g = torch.randn(3001, generator=gen), torch.randn(3001, generator=gen) * 1e-2
    m = (torch.randn(3001, generator=gen) * 1e-3).bfloat16()
    results, errors = {}, []

    def work(k):
        try:
            stream = torch.cuda.Stream(device=cuda)
            with torch.cuda.stream(stream):
                xs, ps, gs, ms = (t.to(cuda, non_blocking=False) for t in (x, p, g, m))
                for _ in range(25):
                    cast = sr_states.cast(xs, seed=k, **options)
                sr_states.hip_sgdm_step_(ps, gs, ms, lr=1e-3, momentum_factor=0.9, seed=k)
            stream.synchronize()
            results[k] = (cast.cpu(), ps.cpu(), ms.cpu())
        except Exception as error:  # reported below, in the test's thread
            errors.append(error)

    threads = [threading.Thread(target=work, args=(k,)) for k in range(4)]
    for thread in threads:
        thread.start()
    for thread in threads:
        thread.join(timeout=60)
    assert not errors and len(results) == 4, errors
    for k, (cast, ps, ms) in results.items():
        assert_bits_or_nan(cast, sr_oracle.cast(x, seed=k, **options), f"thread {k} cast")
        want_p, want_m = p.clone(), m.clone()
        c_oracle.sgdm_step_(want_p, g, want_m, formats=((torch.bfloat16, "stochastic"),), seed=k,
                            lr=1e-3, momentum_factor=0.9)
        assert_bits_or_nan(ps, want_p, f"thread {k} parameter")
        assert_bits_or_nan(ms, want_m, f"thread {k} momentum")
