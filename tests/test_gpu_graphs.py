"""The functional updates and the casts inside a captured HIP graph.

hip_adamw_step_, hip_sgdm_step_ and cast take every scalar (learning rate,
step, key, offset) from the caller and launch on the current stream, so a
graph captured around them replays the same launches.  Each replay here is
preceded by eager work that resets the inputs, then synchronised and
compared bit for bit with the eager result.  The fused optimizers' step()
keeps per-step scalars and is refused under capture (see
tests/test_gpu_multi_tensor.py).
"""

from __future__ import annotations

import pytest
import torch
from conftest import assert_bits_or_nan

from oracle import sr_oracle

pytestmark = pytest.mark.gpu

N = 10007  # odd: full vector tiles and a scalar tail


def test_functional_steps_and_cast_replay_in_a_hip_graph(cuda):
    import sr_states
    from sr_states import StateFormat

    gen = torch.Generator(device=cuda).manual_seed(31)
    p0 = torch.randn(N, device=cuda, generator=gen) * 0.02
    g = torch.randn(N, device=cuda, generator=gen) * 1e-3
    x = torch.randn(N, device=cuda, generator=gen)
    key = sr_oracle.update_key(7, 3, 5)
    adamw = {"lr": 3e-4, "beta1": 0.9, "beta2": 0.999, "eps": 1e-8, "weight_decay": 0.01, "step": 3,
             "seed": key, "offset": 11}
    formats = (StateFormat(torch.float8_e4m3fn), StateFormat(torch.bfloat16))
    sgdm = {"lr": 0.1, "momentum_factor": 0.9, "seed": key ^ 0x5A5A, "offset": 2**32 - 5}

    def inputs():
        return (p0.clone(), torch.full((N,), 0.01, device=cuda).to(torch.float8_e4m3fn),
                torch.full((N,), 1e-6, device=cuda).to(torch.bfloat16), p0.clone(),
                torch.full((N,), 0.003, device=cuda).to(torch.float16))

    def run(p, m, v, q, u):
        sr_states.hip_adamw_step_(p, g, m, v, formats=formats, **adamw)
        sr_states.hip_sgdm_step_(q, g, u, **sgdm)
        return sr_states.cast(x, dtype=torch.bfloat16, seed=7, offset=3)

    expected = inputs()
    expected_cast = run(*expected)
    torch.cuda.synchronize()

    static = inputs()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run(*inputs())  # warm-up launch off the capture, as torch recommends
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured_cast = run(*static)
    for replay in range(3):
        # Eager work between replays: reset the captured inputs.
        for tensor, fresh in zip(static, inputs()):
            tensor.copy_(fresh)
        graph.replay()
        torch.cuda.synchronize()
        for name, got, want in zip(("p", "m", "v", "q", "u"), static, expected):
            assert_bits_or_nan(got, want, f"replay {replay}: {name}")
        assert_bits_or_nan(captured_cast, expected_cast, f"replay {replay}: cast")
