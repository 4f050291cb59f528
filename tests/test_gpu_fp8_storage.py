"""FP8 optimizer states in training and checkpoints on the device.

Mirrors tests/test_fp8_storage.py for the HIP optimizers: the README's FP8
first moment with a BF16 second moment keeps training on small gradients
(no denominator collapse), and a mixed E4M3-SR / E5M2-nearest state survives
torch.save / torch.load(weights_only=True) and resumes bit for bit.  The
capability check of that file (sm_89) is replaced by the gfx950 check,
tested on the CPU in tests/test_host_api.py; per-state format dispatch is
tested in tests/test_tables.py.
"""

from __future__ import annotations

import io

import pytest
import torch
from conftest import raw_bits

pytestmark = pytest.mark.gpu


def test_bf16_second_moment_preserves_small_gradient_training(cuda):
    """tests/test_fp8_storage.py:22-48 with AdamWHip."""
    import sr_states
    from sr_states import StateFormat

    p = torch.nn.Parameter(torch.zeros(1024, device=cuda))
    opt = sr_states.AdamWHip(
        [p],
        lr=3e-4,
        state_format={"exp_avg": StateFormat(torch.float8_e4m3fn), "exp_avg_sq": StateFormat(torch.bfloat16)},
        seed=7,
    )
    for _ in range(10):
        p.grad = torch.full_like(p, 1e-3)
        opt.step()
        second_moment = opt.state[p]["exp_avg_sq"]
        assert second_moment.dtype == torch.bfloat16
        assert bool((second_moment.float() > 0).all())
        assert bool(torch.isfinite(p).all())
    # Denominator collapse would blow the update up; FP8 first moments need
    # not follow the FP32 trajectory.
    assert p.abs().max().item() < 0.05


def test_mixed_fp8_checkpoint_and_resume(cuda):
    """tests/test_fp8_storage.py:57-85 with AdamWHip and BF16 parameters."""
    import sr_states
    from sr_states import StateFormat

    mixed = {"exp_avg": StateFormat(torch.float8_e4m3fn),
             "exp_avg_sq": StateFormat(torch.float8_e5m2, "nearest")}
    arange = torch.arange(31, device=cuda)
    p = torch.nn.Parameter(torch.linspace(-1, 1, 31, device=cuda).bfloat16())
    opt = sr_states.AdamWHip([p], lr=0.001, state_format=mixed, seed=194)
    for step in range(3):
        p.grad = torch.sin(arange + step).bfloat16()
        opt.step()
    assert opt.state[p]["exp_avg"].nbytes + opt.state[p]["exp_avg_sq"].nbytes == 62
    stream = io.BytesIO()
    torch.save(opt.state_dict(), stream)
    stream.seek(0)
    checkpoint = torch.load(stream, weights_only=True)
    q = torch.nn.Parameter(p.detach().clone())
    resumed = sr_states.AdamWHip([q])
    resumed.load_state_dict(checkpoint)
    for name, fmt in mixed.items():
        assert resumed.state[q][name].dtype == fmt.dtype
        assert torch.equal(raw_bits(opt.state[p][name]), raw_bits(resumed.state[q][name]))
    for step in range(4):
        p.grad = torch.sin(arange * 0.1 + step).bfloat16()
        q.grad = p.grad.clone()
        opt.step()
        resumed.step()
        assert torch.equal(p, q)
        for name in mixed:
            assert torch.equal(raw_bits(opt.state[p][name]), raw_bits(resumed.state[q][name]))
    assert opt._rng_step() == resumed._rng_step() == 7
