"""Shared pytest setup: import paths, markers, helpers.

``-m gpu`` tests need an MI355X (gfx950) and fail, rather than skip, when no
GPU is visible, so a silent skip can never pass for a GPU run.  The CPU
suite (``-m "not gpu"``) covers the oracles against golden vectors and
closed forms, the host logic, and the C ABI's exported surface.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
PACKAGE_DIR = ROOT / "stochastic-rounding-pytorch_amd"
for path in (ROOT, PACKAGE_DIR):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config):
    # Markers are registered in pytest.ini.
    built = (PACKAGE_DIR / "sr_states").glob("_group_walk*.so")
    library = PACKAGE_DIR / "sr_states" / "libsr_states_hip.so"
    checks = [ROOT / "tests" / "native" / name
              for name in ("libbf16_sr_check.so", "libstream_ceiling.so", "libminifloat_check.so",
                         "libdivsqrt_check.so", "abi_c_host")]
    if not all(check.exists() for check in checks) and not torch.cuda.is_available():
        import importlib.util

        spec = importlib.util.spec_from_file_location("sr_checks", ROOT / "tests" / "native" / "build_checks.py")
        module = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(module)
        module.build()
    if (not library.exists() or not any(built)) and not torch.cuda.is_available():
        # Only a CPU checkout builds here; GPU runs use the prebuilt library.
        import importlib.util

        spec = importlib.util.spec_from_file_location("sr_build", PACKAGE_DIR / "build.py")
        module = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(module)
        module.build()


@pytest.fixture
def cuda():
    """The GPU device; fails loudly when the run has no GPU."""
    assert torch.cuda.is_available(), "gpu-marked test ran without a visible GPU"
    return torch.device("cuda", 0)


STATE_DTYPES = (torch.float32, torch.bfloat16, torch.float16, torch.float8_e4m3fn, torch.float8_e5m2)
RULES = ("nearest", "stochastic")
# The reference's nine built-in storage policies (benchmarks/bench_states.py:21-31).
POLICIES = {
    "bf16_sr": (torch.bfloat16, "stochastic"),
    "bf16_nr": (torch.bfloat16, "nearest"),
    "fp32": (torch.float32, "nearest"),
    "fp8e4_sr": (torch.float8_e4m3fn, "stochastic"),
    "fp8e4_nr": (torch.float8_e4m3fn, "nearest"),
    "fp8e5_sr": (torch.float8_e5m2, "stochastic"),
    "fp8e5_nr": (torch.float8_e5m2, "nearest"),
    "fp16_sr": (torch.float16, "stochastic"),
    "fp16_nr": (torch.float16, "nearest"),
}


def raw_bits(t: torch.Tensor) -> torch.Tensor:
    """Integer view of a tensor's storage words (same shape)."""
    t = t.detach().cpu().contiguous()
    view = {4: torch.int32, 2: torch.int16, 1: torch.uint8}[t.element_size()]
    return t.view(view)


def assert_bits_or_nan(actual: torch.Tensor, expected: torch.Tensor, what: str = "") -> None:
    """Equal storage bits, except that NaN payload and sign are not compared."""
    assert actual.dtype == expected.dtype, (actual.dtype, expected.dtype)
    assert actual.shape == expected.shape, (actual.shape, expected.shape)
    a, e = actual.detach().cpu().float(), expected.detach().cpu().float()
    nan_a, nan_e = torch.isnan(a), torch.isnan(e)
    assert torch.equal(nan_a, nan_e), f"{what}: NaN positions differ"
    keep = ~nan_e
    ra, re = raw_bits(actual)[keep], raw_bits(expected)[keep]
    if not torch.equal(ra, re):
        bad = (ra != re).nonzero().flatten()
        first = bad[:5].tolist()
        raise AssertionError(
            f"{what}: {bad.numel()} of {ra.numel()} elements differ; first {first}: "
            f"actual {[hex(int(v)) for v in ra[first]]} expected {[hex(int(v)) for v in re[first]]}"
        )


def ulp_distance(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """|a - b| in units in the last place of FP32 (ordered-integer distance)."""
    def ordered(x):
        i = x.detach().cpu().float().contiguous().view(torch.int32).to(torch.int64)
        return torch.where(i < 0, -(i & 0x7FFFFFFF), i)

    return (ordered(a) - ordered(b)).abs()
