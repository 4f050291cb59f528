"""bench.py's contract on the CPU: workloads, byte accounting, arguments, validation.

The timed run needs a GPU (the round-end driver runs it); here the
workload table, the algorithmic bytes per element (the reference's traffic
model, benchmarks/bench_states.py:65-70, extended to mixed widths), the
refusal of more than one GPU and of empty workloads, and the validation
leg's byte comparison (clean runs pass, planted mistakes are caught; the
reference's tests/test_state_benchmark.py:34-76) are checked without one.
"""

from __future__ import annotations

import math
import subprocess
import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
import bench  # noqa: E402


@pytest.mark.parametrize(
    "name,expected",
    [("north_star", 20), ("c1_cast_bf16", 6), ("c2_single_2e26", 20), ("c3_gpt2", 18), ("c4_fp8_mixed", 18),
     ("c5_sgdm_fp16", 16), ("bf16_params_bf16sr", 14), ("bf16_params_e4m3_bf16sr", 12),
     ("bf16_params_fp16sr", 14), ("cast_2e26_e4m3", 5), ("cast_2e26_fp16", 6)],
)
def test_bytes_per_element_follow_the_traffic_model(name, expected):
    assert bench.bytes_per_element(bench.WORKLOADS[name]) == expected


def test_north_star_is_the_default_and_has_the_stated_size():
    spec = bench.WORKLOADS["north_star"]
    assert sum(math.prod(s) for s in spec["shapes"]) == 1_547_698_176
    assert len(spec["shapes"]) == 50
    assert spec["p_dtype"] == spec["g_dtype"] == torch.float32
    assert spec.get("warmup", 25) == 25 and spec.get("steps", 100) == 100


def test_llama_workload_has_the_reference_benchmark_shapes():
    """benchmarks/bench_optimizer_steps.py:54-69: 146 tensors, 1.24 G elements."""
    spec = bench.WORKLOADS["llama32_1b"]
    assert len(spec["shapes"]) == 146
    assert sum(math.prod(s) for s in spec["shapes"]) == 1_235_814_400
    assert spec["hparams"] == dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-2)


def test_torch_baseline_applies_only_where_torch_fused_can_run():
    """Casts, the copy and mixed-dtype gradients (C3's BF16 gradients on FP32 parameters) get none."""
    for name in ("c1_cast_bf16", "cast_2e26_e4m3", "copy_calibration", "c3_gpt2"):
        assert bench.torch_fused_baseline(bench.WORKLOADS[name], work=None, steps=1, warmup=0) is None
    for name in ("north_star", "c5_sgdm_fp16", "copy_calibration"):
        assert bench.torch_cast_baseline(bench.WORKLOADS[name], work=None, steps=1, warmup=0) is None


def test_short_launches_warm_up_for_the_clock_ramp():
    """Each cast or sub-millisecond workload's default warmup spans at least ~0.3 s of GPU work."""
    rough_ms = {"c1_cast_bf16": 0.0165, "c2_single_2e26": 0.208, "c3_gpt2": 0.353, "cast_2e26_bf16": 0.061}
    for name, ms in rough_ms.items():
        assert bench.WORKLOADS[name]["warmup"] * ms >= 300, name


def test_more_than_one_gpu_is_refused_with_a_reason():
    result = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True,
                            text=True, timeout=300)
    assert result.returncode != 0
    assert "one GPU" in result.stderr or "one GPU" in result.stdout


@pytest.mark.parametrize("value", ["float8_e4m3fn/sideways", "float9/stochastic", "bfloat16"])
def test_state_format_override_is_validated_before_anything_runs(value):
    result = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--state-format", value],
                            capture_output=True, text=True, timeout=300)
    assert result.returncode != 0 and "--state-format" in result.stderr


def test_ceiling_helpers_refuse_bad_arguments_before_any_device_work():
    """The pattern ceilings check their arguments first (no GPU here)."""
    import ctypes

    lib = ctypes.CDLL(str(bench.CEILING_LIBRARY))
    lib.sr_stream_ceiling_p.restype = ctypes.c_int
    lib.sr_stream_ceiling_p.argtypes = [ctypes.c_uint64, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                        ctypes.c_int, ctypes.POINTER(ctypes.c_float)]
    lib.sr_cast_ceiling.restype = ctypes.c_int
    lib.sr_cast_ceiling.argtypes = [ctypes.c_uint64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                    ctypes.POINTER(ctypes.c_float)]
    ms = ctypes.c_float()
    n = 512 * 1000
    assert lib.sr_stream_ceiling_p(n, 2, 4, 2, 2, 1, ctypes.byref(ms)) == 1  # no such pattern
    assert lib.sr_stream_ceiling_p(n, 4, 4, 3, 2, 1, ctypes.byref(ms)) == 1
    assert lib.sr_stream_ceiling_p(0, 4, 4, 2, 2, 1, ctypes.byref(ms)) == 1
    assert lib.sr_stream_ceiling_p(n + 1, 4, 4, 2, 2, 1, ctypes.byref(ms)) == 1  # not whole tiles
    assert lib.sr_stream_ceiling_p(n, 4, 4, 2, 2, 0, ctypes.byref(ms)) == 1  # no repetitions
    assert lib.sr_cast_ceiling(2048 * 10, 3, 8, 1, ctypes.byref(ms)) == 1  # 3-byte output
    assert lib.sr_cast_ceiling(2048 * 10, 2, 17, 1, ctypes.byref(ms)) == 1  # too many buffers
    assert lib.sr_cast_ceiling(2048 * 10 + 1, 2, 8, 1, ctypes.byref(ms)) == 1
    lib.sr_launch_cap_sweep.restype = ctypes.c_int
    lib.sr_launch_cap_sweep.argtypes = [ctypes.c_uint64, ctypes.c_int, ctypes.POINTER(ctypes.c_int), ctypes.c_int,
                                        ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_float),
                                        ctypes.POINTER(ctypes.c_int)]
    out = [(ctypes.c_float * 2)(), (ctypes.c_float * 2)(), (ctypes.c_int * 2)()]

    def sweep(n, caps, reps=1):
        return lib.sr_launch_cap_sweep(n, reps, (ctypes.c_int * max(len(caps), 1))(*caps), len(caps), *out)

    assert sweep(n, [-2]) == 1  # below -1 (the rule)
    assert sweep(n, [17]) == 1  # above the largest cap
    assert sweep(n, []) == 1
    assert sweep(n + 1, [0]) == 1  # not whole tiles
    assert sweep(n, [0], reps=0) == 1


@pytest.mark.parametrize("value,ok", [("1", True), ("1024", True), ("0", False), ("-1", False)])
def test_positive_int(value, ok):
    """benchmarks/bench_sgdm.py's argument types (tests/test_benchmark_helpers.py:14-31)."""
    import argparse

    if ok:
        assert bench.positive_int(value) == int(value)
    else:
        with pytest.raises(argparse.ArgumentTypeError, match="positive"):
            bench.positive_int(value)
    assert bench.nonnegative_int("0") == 0
    with pytest.raises(argparse.ArgumentTypeError, match="nonnegative"):
        bench.nonnegative_int("-1")


@pytest.mark.parametrize("option", ["--steps=0", "--warmup=-1", "--gpus=0", "--cpu-seconds=0", "--cpu-seconds=inf"])
def test_nonpositive_workloads_are_refused(option):
    """tests/test_state_benchmark.py:138-141: zero sizes and counts are refused before anything runs."""
    result = subprocess.run([sys.executable, str(ROOT / "bench.py"), option], capture_output=True, text=True,
                            timeout=300)
    assert result.returncode == 2 and option.split("=")[0] in result.stderr


@pytest.mark.parametrize(
    "optimizer,p_dtype,state_dtype,expected",
    [("sgdm", torch.float32, torch.bfloat16, 16), ("sgdm", torch.float32, torch.float32, 20),
     ("adamw", torch.float32, torch.bfloat16, 20), ("adamw", torch.float32, torch.float32, 28),
     ("sgdm", torch.bfloat16, torch.bfloat16, 10), ("sgdm", torch.bfloat16, torch.float32, 14),
     ("adamw", torch.float32, torch.float8_e4m3fn, 16)],
)
def test_bytes_per_element_of_every_state_policy(optimizer, p_dtype, state_dtype, expected):
    """tests/test_state_benchmark.py:125-135 and tests/test_benchmark_helpers.py:9-11."""
    count = 2 if optimizer == "adamw" else 1
    spec = {"optimizer": optimizer, "p_dtype": p_dtype, "g_dtype": p_dtype,
            "formats": ((state_dtype, "stochastic"),) * count}
    assert bench.bytes_per_element(spec) == expected


# -- the validation leg ---------------------------------------------------------
# validate() replays sampled chunks with the C oracle.  Here the "device" bytes
# come from the torch restatement of the reference (oracle/sr_oracle.py), an
# independent formulation, so a clean run checks the two against each other
# and the planted mistakes check that the comparison sees them.

SGDM_POLICIES = {
    "bf16_sr": (torch.bfloat16, "stochastic"),
    "fp16_sr": (torch.float16, "stochastic"),
    "fp8e4_nr": (torch.float8_e4m3fn, "nearest"),
    "fp8e4_sr": (torch.float8_e4m3fn, "stochastic"),
    "fp8e5_nr": (torch.float8_e5m2, "nearest"),
    "fp8e5_sr": (torch.float8_e5m2, "stochastic"),
}
FP8_POLICIES = ["fp8e4_nr", "fp8e4_sr", "fp8e5_nr", "fp8e5_sr"]


def _sgdm_case(policy, steps=3):
    from oracle import sr_oracle

    spec = {"optimizer": "sgdm", "formats": (SGDM_POLICIES[policy],), "seed": 11,
            "hparams": {"lr": 0.1, "momentum": 0.9}}
    gen = torch.Generator().manual_seed(4)
    samples, finals = [], []
    for index, start, length in ((0, 0, 4099), (3, 8192 + 5, 1001)):
        p0 = torch.randn(length, generator=gen)
        g = torch.randn(length, generator=gen) * 0.05
        samples.append((index, start, length, [p0, g]))
        p, u = p0.clone(), torch.zeros(length, dtype=SGDM_POLICIES[policy][0])
        for t in range(1, steps + 1):
            key = sr_oracle.update_key(spec["seed"], t, index)
            p, u = sr_oracle.sgdm_step(p, g, u, lr=0.1, momentum_factor=0.9,
                                       formats=(sr_oracle.Fmt(*SGDM_POLICIES[policy]),), seed=key, offset=start)
        finals.append([p, u])
    return spec, samples, finals


@pytest.mark.parametrize("policy", list(SGDM_POLICIES))
def test_validation_accepts_the_reference_update(policy):
    spec, samples, finals = _sgdm_case(policy)
    result = bench.validate(spec, samples, finals, steps=3)
    assert result["mismatches"] == 0
    assert result["elements_checked"] == 2 * (4099 + 1001) and result["chunks"] == 2


@pytest.mark.parametrize("policy", FP8_POLICIES)
def test_validation_rejects_wrong_storage_with_correct_recurrence(policy):
    """tests/test_state_benchmark.py:48-61: one storage step off is caught."""
    spec, samples, finals = _sgdm_case(policy)
    u = finals[0][1]
    finals[0][1] = (u.float() + torch.finfo(u.dtype).eps).to(u.dtype)
    assert bench.validate(spec, samples, finals, steps=3)["mismatches"] > 0


@pytest.mark.parametrize("policy", FP8_POLICIES)
def test_validation_rejects_wrong_fp32_recurrence(policy):
    """tests/test_state_benchmark.py:63-76."""
    spec, samples, finals = _sgdm_case(policy)
    u = finals[1][1]
    finals[1][1] = (u.float() + 0.0625).to(u.dtype)
    assert bench.validate(spec, samples, finals, steps=3)["mismatches"] > 0


def test_validation_counts_single_changes_and_step_counts():
    spec, samples, finals = _sgdm_case("bf16_sr")
    p = finals[1][0]
    p.view(torch.int32)[:7] += 1  # seven parameters one ulp off
    assert bench.validate(spec, samples, finals, steps=3)["mismatches"] == 7
    spec, samples, finals = _sgdm_case("bf16_sr", steps=2)
    assert bench.validate(spec, samples, finals, steps=3)["mismatches"] > 0


@pytest.mark.parametrize("dtype,rule", [(torch.bfloat16, "stochastic"), (torch.float8_e4m3fn, "stochastic"),
                                        (torch.float16, "nearest")])
def test_validation_of_casts(dtype, rule):
    from oracle import sr_oracle

    spec = {"optimizer": "cast", "formats": ((dtype, rule),), "seed": 7}
    x = torch.randn(3001, generator=torch.Generator().manual_seed(2)) * 50
    samples = [(0, 5, 3001, [x])]
    finals = [[sr_oracle.cast(x, dtype=dtype, rounding=rule, seed=7, offset=5)]]
    assert bench.validate(spec, samples, finals, steps=1)["mismatches"] == 0
    finals = [[sr_oracle.cast(x, dtype=dtype, rounding=rule, seed=7, offset=6)]]
    if rule == "stochastic":  # another counter base draws other bits
        assert bench.validate(spec, samples, finals, steps=1)["mismatches"] > 0


def test_traffic_comes_with_its_source():
    """The bench line's HBM traffic is read from a committed summary, which it names with its build."""
    traffic, source = bench.load_traffic("north_star")
    assert traffic is not None and traffic > 30e9
    assert source["profile"] == "profiles/adamw_kernel_north_star_hbm_traffic.md"
    assert source["build_commit"] and len(source["build_commit"]) >= 7
    assert (ROOT / source["profile"]).exists()
    assert bench.load_traffic("no_such_workload") == (None, None)
