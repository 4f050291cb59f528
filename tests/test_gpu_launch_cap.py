"""The resident-workgroup cap of large optimizer launches.

Large FP32-parameter launches reserve LDS they never use so that only
sr::resident_cap workgroups stay resident per CU: 72-96 KiB of tiles in
flight per CU by launch family, where 16 workgroups fit.
tests/native/stream_ceiling.hip's sr_launch_cap_sweep times the library's
fused AdamW kernel (FP32 parameter and gradient, BF16 stochastic moments)
on one tensor of 2^28 elements (5.4 GB) with the rule's cap and with none,
interleaved over three rounds: the occupancy calculator must report the
rule's 8 workgroups per CU, and the capped kernel must not be slower than
the uncapped one by more than 2%.  How much faster it is depends on the
machine: 3-4% on most MI355X boxes measured, level on one.  The single-tensor entries, AdamW
with two stochastic FP16 or FP8 moments (96 KiB in flight) and the
optimizers at 256-, 512- and 1024-lane workgroups, capped past 2^16 tiles,
are held to the C oracle.  SR_STATES_RESIDENT_CAP, which replaces the
rule for a process, changes the time of a launch and none of its bytes.
"""

from __future__ import annotations

import ctypes
import json
import os
import statistics
import subprocess
import sys
from pathlib import Path

import pytest
import torch

pytestmark = pytest.mark.gpu

LIBRARY = Path(__file__).resolve().parent / "native" / "libstream_ceiling.so"
N = 1 << 28


def test_capped_fused_kernel_holds_the_cap_and_is_not_slower(cuda):
    assert LIBRARY.exists(), f"{LIBRARY} is not built (tests/native/build_checks.py)"
    lib = ctypes.CDLL(str(LIBRARY))
    lib.sr_launch_cap_sweep.restype = ctypes.c_int
    lib.sr_launch_cap_sweep.argtypes = [ctypes.c_uint64, ctypes.c_int, ctypes.POINTER(ctypes.c_int), ctypes.c_int,
                                        ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_float),
                                        ctypes.POINTER(ctypes.c_int)]
    caps = (ctypes.c_int * 2)(-1, 0)
    capped, uncapped = [], []
    for _ in range(3):
        trivial, fused, resident = (ctypes.c_float * 2)(), (ctypes.c_float * 2)(), (ctypes.c_int * 2)()
        assert lib.sr_launch_cap_sweep(N, 40, caps, 2, trivial, fused, resident) == 0
        assert resident[0] == 8 and resident[1] == 16, list(resident)
        capped.append(fused[0])
        uncapped.append(fused[1])
    rate = lambda ms: 20 * N / ms / 1e6  # noqa: E731  (GB/s)
    capped_ms, uncapped_ms = statistics.median(capped), statistics.median(uncapped)
    print(f"capped {rate(capped_ms):.0f} GB/s, uncapped {rate(uncapped_ms):.0f} GB/s")
    assert capped_ms <= 1.02 * uncapped_ms, (
        f"capped {rate(capped_ms):.0f} GB/s against uncapped {rate(uncapped_ms):.0f} GB/s")


CHUNK = 4099


@pytest.mark.parametrize("kind", ["adamw", "sgdm"])
def test_capped_single_tensor_launches_equal_the_oracle(cuda, kind):
    """The single-tensor entries past 2^16 tiles (capped) against the C oracle, sampled chunks.

    2^25 + 5 elements make 65537 tiles of 512: the launch reserves its LDS.
    Chunks at the head, inside and at the tail (a partial last tile) must
    equal the oracle's replay of the same elements with the chunk start as
    the counter offset, parameters and states byte for byte.
    """
    import sr_states
    from conftest import assert_bits_or_nan

    from oracle import c_oracle

    n = (1 << 25) + 5
    key, offset = 0xA5A5F00D, 12_345
    gen = torch.Generator(device=cuda).manual_seed(23)
    p = torch.empty(n, device=cuda).normal_(std=0.02, generator=gen)
    g = torch.empty(n, device=cuda).normal_(std=1e-3, generator=gen)
    starts = [0, (n // 3) * 2 + 7, n - CHUNK]
    before = {s: (p[s:s + CHUNK].cpu(), g[s:s + CHUNK].cpu()) for s in starts}
    if kind == "adamw":
        formats = ((torch.float8_e4m3fn, "stochastic"), (torch.bfloat16, "stochastic"))
        states = [torch.zeros(n, device=cuda, dtype=d) for d, _ in formats]
        hyper = dict(lr=3e-4, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01, step=3)
        sr_states.hip_adamw_step_(p, g, *states, seed=key, offset=offset,
                                  formats=tuple(sr_states.StateFormat(d, r) for d, r in formats), **hyper)
    else:
        formats = ((torch.float16, "stochastic"),)
        states = [torch.zeros(n, device=cuda, dtype=torch.float16)]
        hyper = dict(lr=0.1, momentum_factor=0.9)
        sr_states.hip_sgdm_step_(p, g, *states, seed=key, offset=offset,
                                 formats=(sr_states.StateFormat(torch.float16, "stochastic"),), **hyper)
    torch.cuda.synchronize()
    for start, (p_ref, g_ref) in before.items():
        refs = [torch.zeros(CHUNK, dtype=d) for d, _ in formats]
        if kind == "adamw":
            c_oracle.adamw_step_(p_ref, g_ref, *refs, formats=formats, seed=key, offset=offset + start, **hyper)
        else:
            c_oracle.sgdm_step_(p_ref, g_ref, *refs, formats=formats, seed=key, offset=offset + start, **hyper)
        sl = slice(start, start + CHUNK)
        assert_bits_or_nan(p[sl].cpu(), p_ref, f"{kind} parameter at {start}")
        for k, (state, ref) in enumerate(zip(states, refs)):
            assert_bits_or_nan(state[sl].cpu(), ref, f"{kind} state {k} at {start}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.float8_e4m3fn, torch.float8_e5m2],
                         ids=lambda d: str(d).replace("torch.", ""))
def test_capped_launches_with_two_minifloat_sr_moments_equal_the_oracle(cuda, dtype):
    """AdamW with both moments stochastic FP16 or FP8 keeps 96 KiB in flight (10 or 12 workgroups
    per CU); past 2^16 tiles, sampled chunks against the C oracle."""
    import sr_states
    from conftest import assert_bits_or_nan

    from oracle import c_oracle, sr_oracle

    n = (1 << 25) + 517
    gen = torch.Generator(device=cuda).manual_seed(29)
    p = torch.nn.Parameter(torch.empty(n, device=cuda).normal_(std=0.02, generator=gen))
    p.grad = torch.empty(n, device=cuda).normal_(std=1e-3, generator=gen)
    starts = [0, n // 2 + 5, n - CHUNK]
    before = {s: (p.detach()[s:s + CHUNK].cpu(), p.grad[s:s + CHUNK].cpu()) for s in starts}
    formats = ((dtype, "stochastic"),) * 2
    opt = sr_states.AdamWHip([p], lr=3e-4, weight_decay=0.01, seed=13,
                             state_format=sr_states.StateFormat(dtype, "stochastic"))
    opt.step()
    torch.cuda.synchronize()
    key = sr_oracle.update_key(13, 1, 0)
    for start, (p_ref, g_ref) in before.items():
        refs = [torch.zeros(CHUNK, dtype=dtype) for _ in range(2)]
        c_oracle.adamw_step_(p_ref, g_ref, *refs, lr=3e-4, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01,
                             step=1, formats=formats, seed=key, offset=start)
        sl = slice(start, start + CHUNK)
        assert_bits_or_nan(p.detach()[sl].cpu(), p_ref, f"{dtype} parameter at {start}")
        for name, ref in zip(("exp_avg", "exp_avg_sq"), refs):
            assert_bits_or_nan(opt.state[p][name][sl].cpu(), ref, f"{dtype} {name} at {start}")


@pytest.mark.parametrize("kind, block_size", [("adamw", 256), ("adamw", 1024), ("sgdm", 512)])
def test_capped_launches_of_other_workgroup_sizes_equal_the_oracle(cuda, kind, block_size):
    """The optimizers with a non-default workgroup size, past 2^16 tiles (so capped: 4 workgroups
    of 256 lanes and 1 of 1024 for AdamW, 2 of 512 for SGDM with FP16-SR momentum per CU),
    against the C oracle on sampled chunks."""
    import sr_states
    from conftest import assert_bits_or_nan

    from oracle import c_oracle, sr_oracle

    n = (1 << 16) * block_size * 4 + 9
    gen = torch.Generator(device=cuda).manual_seed(block_size)
    p = torch.nn.Parameter(torch.empty(n, device=cuda).normal_(std=0.02, generator=gen))
    p.grad = torch.empty(n, device=cuda).normal_(std=1e-3, generator=gen)
    starts = [0, n // 2 + 11, n - CHUNK]
    before = {s: (p.detach()[s:s + CHUNK].cpu(), p.grad[s:s + CHUNK].cpu()) for s in starts}
    if kind == "adamw":
        formats = ((torch.bfloat16, "stochastic"),) * 2
        opt = sr_states.AdamWHip([p], lr=3e-4, weight_decay=0.01, seed=5, block_size=block_size)
        names = ("exp_avg", "exp_avg_sq")
    else:
        formats = ((torch.float16, "stochastic"),)
        opt = sr_states.SGDMHip([p], lr=0.1, momentum=0.9, seed=5, block_size=block_size,
                                state_format=sr_states.StateFormat(torch.float16))
        names = ("momentum_buffer",)
    opt.step()
    torch.cuda.synchronize()
    key = sr_oracle.update_key(5, 1, 0)
    for start, (p_ref, g_ref) in before.items():
        refs = [torch.zeros(CHUNK, dtype=d) for d, _ in formats]
        if kind == "adamw":
            c_oracle.adamw_step_(p_ref, g_ref, *refs, lr=3e-4, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01,
                                 step=1, formats=formats, seed=key, offset=start)
        else:
            c_oracle.sgdm_step_(p_ref, g_ref, *refs, lr=0.1, momentum_factor=0.9, formats=formats, seed=key,
                                offset=start)
        sl = slice(start, start + CHUNK)
        assert_bits_or_nan(p.detach()[sl].cpu(), p_ref, f"{kind}/{block_size} parameter at {start}")
        for name, ref in zip(names, refs):
            assert_bits_or_nan(opt.state[p][name][sl].cpu(), ref, f"{kind}/{block_size} {name} at {start}")


# One process per setting of SR_STATES_RESIDENT_CAP (the library reads it
# once): two AdamW steps on 2^25 + 3 elements (65537 tiles, so capped), a
# digest of the parameter and moments, then the mean time of 30 launches.
_OVERRIDE_CHILD = """
import hashlib, json, torch
import sr_states
dev = torch.device("cuda", 0)
n = (1 << 25) + 3
gen = torch.Generator(device=dev).manual_seed(31)
p = torch.empty(n, device=dev).normal_(std=0.02, generator=gen)
g = torch.empty(n, device=dev).normal_(std=1e-3, generator=gen)
m = torch.zeros(n, device=dev, dtype=torch.bfloat16)
v = torch.zeros(n, device=dev, dtype=torch.bfloat16)
fmt = (sr_states.StateFormat(torch.bfloat16, "stochastic"),) * 2
hyper = dict(lr=3e-4, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01, seed=0x5EED, formats=fmt)
for step in (1, 2):
    sr_states.hip_adamw_step_(p, g, m, v, step=step, **hyper)
torch.cuda.synchronize()
digest = hashlib.sha256()
for t in (p, m, v):
    digest.update(t.view(torch.uint8).cpu().numpy().tobytes())
for _ in range(5):
    sr_states.hip_adamw_step_(p, g, m, v, step=3, **hyper)
a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
a.record()
for _ in range(30):
    sr_states.hip_adamw_step_(p, g, m, v, step=3, **hyper)
b.record()
b.synchronize()
print(json.dumps({"digest": digest.hexdigest(), "ms": a.elapsed_time(b) / 30}), flush=True)
"""


def test_resident_cap_override_changes_time_not_bytes(cuda):
    """SR_STATES_RESIDENT_CAP=0 (uncapped) and =1 give the same bytes as the rule's cap of 8, and
    cap 1 (two waves per CU) is far slower, so the variable does reach the launches."""
    root = Path(__file__).resolve().parents[1]
    env = dict(os.environ)
    env["PYTHONPATH"] = os.pathsep.join(
        [str(root), str(root / "stochastic-rounding-pytorch_amd"), env.get("PYTHONPATH", "")])
    runs = {}
    for setting in ("rule", "0", "1"):
        if setting == "rule":
            env.pop("SR_STATES_RESIDENT_CAP", None)
        else:
            env["SR_STATES_RESIDENT_CAP"] = setting
        print(f"child with SR_STATES_RESIDENT_CAP={setting}", flush=True)
        done = subprocess.run([sys.executable, "-c", _OVERRIDE_CHILD], env=env, capture_output=True, text=True,
                              timeout=100)
        assert done.returncode == 0, f"{setting}: exit {done.returncode}\n{done.stderr[-2000:]}"
        runs[setting] = json.loads(done.stdout.strip().splitlines()[-1])
    assert runs["0"]["digest"] == runs["rule"]["digest"]
    assert runs["1"]["digest"] == runs["rule"]["digest"]
    times = {k: round(r["ms"], 4) for k, r in runs.items()}
    assert runs["1"]["ms"] > 1.5 * runs["rule"]["ms"], times
