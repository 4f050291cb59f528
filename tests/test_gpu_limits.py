"""Maximum sizes on the GPU: a parameter of 2^32 elements, launches past 2^31 and 2^34.

The reference caps a parameter at 2^32 elements because its counters are
32-bit (sr_states/optim/_state.py:16-18); past 2^31 elements every index and
address computation must be 64-bit.  These tests run one update (or cast) at
those sizes and replay chunks at the head, around 2^31 and at the tail
through the C oracle with the chunk start as the element offset, so that the
counters' wrap modulo 2^32 is checked too.  Each test needs up to 86 GB of
device memory.
"""

from __future__ import annotations

import gc

import pytest
import torch
from conftest import assert_bits_or_nan

from oracle import c_oracle, sr_oracle

pytestmark = pytest.mark.gpu

CHUNK = 4099


@pytest.fixture(autouse=True)
def _release_device_memory():
    yield
    gc.collect()
    if torch.cuda.is_available():
        torch.cuda.empty_cache()


def _starts(n):
    half = 1 << 31
    return [0, half - CHUNK // 2, half + 3, n - CHUNK]


def test_adamw_parameter_of_2_32_elements(cuda):
    import sr_states

    n = 1 << 32
    gen = torch.Generator(device=cuda).manual_seed(3)
    p = torch.nn.Parameter(torch.empty(n, device=cuda).normal_(std=0.02, generator=gen))
    p.grad = torch.empty(n, device=cuda).normal_(std=1e-3, generator=gen)
    before = {s: (p.detach()[s:s + CHUNK].cpu(), p.grad[s:s + CHUNK].cpu()) for s in _starts(n)}
    opt = sr_states.AdamWHip([p], lr=3e-4, weight_decay=0.01, seed=7)
    opt.step()
    torch.cuda.synchronize()
    key = sr_oracle.update_key(7, 1, 0)
    formats = ((torch.bfloat16, "stochastic"),) * 2
    for start, (p_ref, g_ref) in before.items():
        m_ref, v_ref = (torch.zeros(CHUNK, dtype=torch.bfloat16) for _ in range(2))
        c_oracle.adamw_step_(p_ref, g_ref, m_ref, v_ref, lr=3e-4, beta1=0.9, beta2=0.999, eps=1e-8,
                             weight_decay=0.01, step=1, formats=formats, seed=key, offset=start)
        sl = slice(start, start + CHUNK)
        assert_bits_or_nan(p.detach()[sl].cpu(), p_ref, f"p at {start}")
        assert_bits_or_nan(opt.state[p]["exp_avg"][sl].cpu(), m_ref, f"exp_avg at {start}")
        assert_bits_or_nan(opt.state[p]["exp_avg_sq"][sl].cpu(), v_ref, f"exp_avg_sq at {start}")


def test_sgdm_past_2_31_elements(cuda):
    import sr_states
    from sr_states import StateFormat

    n = (1 << 31) + 12_345
    gen = torch.Generator(device=cuda).manual_seed(4)
    p = torch.nn.Parameter(torch.empty(n, device=cuda).normal_(std=0.02, generator=gen))
    p.grad = torch.empty(n, device=cuda).normal_(std=1e-2, generator=gen)
    before = {s: (p.detach()[s:s + CHUNK].cpu(), p.grad[s:s + CHUNK].cpu()) for s in _starts(n)}
    opt = sr_states.SGDMHip([p], lr=0.1, momentum=0.9, seed=11,
                            state_format=StateFormat(torch.float16))
    opt.step()
    torch.cuda.synchronize()
    key = sr_oracle.update_key(11, 1, 0)
    for start, (p_ref, g_ref) in before.items():
        u_ref = torch.zeros(CHUNK, dtype=torch.float16)
        c_oracle.sgdm_step_(p_ref, g_ref, u_ref, lr=0.1, momentum_factor=0.9,
                            formats=((torch.float16, "stochastic"),), seed=key, offset=start)
        sl = slice(start, start + CHUNK)
        assert_bits_or_nan(p.detach()[sl].cpu(), p_ref, f"p at {start}")
        assert_bits_or_nan(opt.state[p]["momentum_buffer"][sl].cpu(), u_ref, f"momentum at {start}")


def test_sgdm_bucket_past_2_34_elements(cuda):
    """One launch over more work-items than a grid dimension holds.

    A dispatch carries fewer than 2^32 work-items per dimension, and at four
    elements per lane that is 2^34 elements.  Four parameters of 2^32
    elements and one of 2^20 (BF16 parameters and gradients, E4M3 momentum:
    86 GB) form one bucket of 2^25 + 2^11 tiles, launched as two rows of
    workgroups; the last 8192 workgroups, in the second row, cover the tail
    of parameter 3 and all of parameter 4.
    """
    import sr_states
    from sr_states import StateFormat

    sizes = [1 << 32] * 4 + [1 << 20]
    # One work-item per lane, LANE_ELEMENTS elements each: past 2^32 - 1.
    assert sum(sizes) // sr_states._lib.LANE_ELEMENTS >= 1 << 32
    gen = torch.Generator(device=cuda).manual_seed(8)
    params = []
    for n in sizes:
        p = torch.nn.Parameter(torch.empty(n, device=cuda, dtype=torch.bfloat16).normal_(std=0.02, generator=gen))
        p.grad = torch.empty(n, device=cuda, dtype=torch.bfloat16).normal_(std=1e-2, generator=gen)
        params.append(p)
    samples = {}
    for index, p in enumerate(params):
        n = p.numel()
        starts = [0, n - CHUNK] if n < 1 << 31 else _starts(n)
        samples[index] = {s: (p.detach()[s:s + CHUNK].cpu(), p.grad[s:s + CHUNK].cpu()) for s in starts}
    fmt = ((torch.float8_e4m3fn, "stochastic"),)
    opt = sr_states.SGDMHip(params, lr=0.1, momentum=0.9, seed=13,
                            state_format=StateFormat(torch.float8_e4m3fn))
    opt.step()
    torch.cuda.synchronize()
    for index, chunks in samples.items():
        p = params[index]
        key = sr_oracle.update_key(13, 1, index)
        for start, (p_ref, g_ref) in chunks.items():
            u_ref = torch.zeros(CHUNK, dtype=torch.float8_e4m3fn)
            c_oracle.sgdm_step_(p_ref, g_ref, u_ref, lr=0.1, momentum_factor=0.9, formats=fmt, seed=key,
                                offset=start)
            sl = slice(start, start + CHUNK)
            what = f"parameter {index} at {start}"
            assert_bits_or_nan(p.detach()[sl].cpu(), p_ref, f"p of {what}")
            assert_bits_or_nan(opt.state[p]["momentum_buffer"][sl].cpu(), u_ref, f"momentum of {what}")


@pytest.mark.parametrize("dtype", [torch.float8_e4m3fn, torch.bfloat16])
def test_cast_past_2_31_elements(cuda, dtype):
    import sr_states

    n = (1 << 31) + 7
    x = torch.empty(n, device=cuda).normal_(generator=torch.Generator(device=cuda).manual_seed(5))
    # The seed and offset put the counters of the last elements past 2^32.
    seed, offset = 0xFFFF0000, 0x00F00000
    y = sr_states.cast(x, dtype=dtype, seed=seed, offset=offset)
    for start in _starts(n):
        chunk = x[start:start + CHUNK].cpu()
        expected = c_oracle.cast(chunk, dtype=dtype, seed=seed, offset=(offset + start) & 0xFFFFFFFF)
        assert_bits_or_nan(y[start:start + CHUNK].cpu(), expected, f"{dtype} at {start}")
