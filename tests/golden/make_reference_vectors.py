"""Write reference optimizer trajectories to tests/golden/reference_trajectories.pt.

Runs the reference package in THIS container only (PYTHONPATH pointing at the
read-only reference checkout, default /root/reference); the GPU box never
sees the reference, only the fixture this script writes.

Why an import: the multi-step composition -- torch CPU's exact FP32 operation
sequence in the eager recurrences together with the optimizer's RNG-step,
parameter-index, missing-gradient and group plumbing -- is fixed by no
closed form or known-answer test of the reference.  Everything else (hash,
keys, encoders) is pinned by closed forms in the CPU tests.

Usage:  python tests/golden/make_reference_vectors.py [--reference PATH] [--force]
"""

from __future__ import annotations

import argparse
import sys
from pathlib import Path

import torch

OUTPUT = Path(__file__).with_name("reference_trajectories.pt")


def bits(t: torch.Tensor) -> torch.Tensor:
    return t.detach().contiguous().view(torch.uint8).clone()


def gradient(n, step, index, dtype, scale):
    x = torch.arange(n, dtype=torch.float32)
    return (torch.sin(x * 0.37 + 1.7 * step + index) * scale).to(dtype)


CASES = {
    # name: (optimizer, groups, hyperparameters, steps, initial sr_step)
    "adamw_mixed": (
        "adamw",
        [
            {"sizes": [(1031, "f32"), (3, "f32")], "formats": ("bf16/stochastic", "bf16/stochastic"),
             "sr_seed": 0xFEDCBA9876543210},
            {"sizes": [(515, "bf16"), (257, "f32")],
             "formats": ("e4m3/stochastic", "bf16/stochastic"), "sr_seed": -(2**48) - 1, "lr": 3e-3},
        ],
        {"lr": 1e-3, "betas": (0.9, 0.999), "eps": 1e-8, "weight_decay": 0.01},
        6,
        2**32 - 2,
    ),
    "adamw_minifloat": (
        "adamw",
        [
            {"sizes": [(2053, "f32")], "formats": ("f16/stochastic", "e5m2/nearest"), "sr_seed": 7},
            {"sizes": [(129, "f32"), (700, "bf16")], "formats": ("e5m2/stochastic", "f16/nearest"),
             "sr_seed": 2**70 + 5},
        ],
        {"lr": 3e-4, "betas": (0.8, 0.95), "eps": 1e-6, "weight_decay": 0.1},
        5,
        0,
    ),
    "sgdm_mixed": (
        "sgdm",
        [
            {"sizes": [(1031, "f32"), (64, "bf16")], "formats": ("f16/stochastic",), "sr_seed": 11},
            {"sizes": [(333, "f32")], "formats": ("e4m3/stochastic",), "sr_seed": -5},
            {"sizes": [(257, "f32")], "formats": ("bf16/nearest",), "sr_seed": 2**40},
        ],
        {"lr": 0.1, "momentum": 0.9},
        6,
        2**32 - 3,
    ),
}

DTYPES = {
    "f32": torch.float32,
    "bf16": torch.bfloat16,
    "f16": torch.float16,
    "e4m3": torch.float8_e4m3fn,
    "e5m2": torch.float8_e5m2,
}


def run_case(name, spec, sr):
    kind, groups, hyper, steps, sr_step = spec
    names = ("exp_avg", "exp_avg_sq") if kind == "adamw" else ("momentum_buffer",)
    params, param_groups = [], []
    for gi, group in enumerate(groups):
        plist = []
        for pi, (n, dt) in enumerate(group["sizes"]):
            p = torch.nn.Parameter((torch.linspace(-0.8, 0.7, n) * (1 + gi + pi)).to(DTYPES[dt]))
            plist.append(p)
            params.append(p)
        fmt = {
            state: sr.StateFormat(DTYPES[f.split("/")[0]], f.split("/")[1])
            for state, f in zip(names, group["formats"])
        }
        entry = {"params": plist, "state_format": fmt, "sr_seed": group["sr_seed"]}
        if "lr" in group:
            entry["lr"] = group["lr"]
        param_groups.append(entry)
    cls = sr.AdamWReferenceSR if kind == "adamw" else sr.SGDMReferenceSR
    optimizer = cls(param_groups, **hyper)
    for group in optimizer.param_groups:
        group["sr_step"] = sr_step
    record = {
        "kind": kind,
        "groups": groups,
        "hyper": hyper,
        "initial_sr_step": sr_step,
        "initial": [bits(p) for p in params],
        "dtypes": [str(p.dtype) for p in params],
        "steps": [],
    }
    for step in range(steps):
        grads = []
        for index, p in enumerate(params):
            missing = (step + index) % 5 == 3
            scale = 1e-3 if kind == "adamw" else 1e-2
            p.grad = None if missing else gradient(p.numel(), step, index, p.dtype, scale)
            grads.append(None if missing else bits(p.grad))
        optimizer.step()
        record["steps"].append(
            {
                "grads": grads,
                "params": [bits(p) for p in params],
                "states": [
                    {k: bits(v) if isinstance(v, torch.Tensor) else v for k, v in optimizer.state[p].items()}
                    for p in params
                ],
                "sr_step": [g["sr_step"] for g in optimizer.param_groups],
            }
        )
    record["state_dict"] = optimizer.state_dict()
    return record


def main():
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--reference", default="/root/reference")
    parser.add_argument("--force", action="store_true")
    args = parser.parse_args()
    if OUTPUT.exists() and not args.force:
        raise SystemExit(f"refusing to overwrite {OUTPUT}")
    sys.path.insert(0, args.reference)
    import sr_states as sr

    fixture = {
        "torch": str(torch.__version__),
        "cpu_capability": torch.backends.cpu.get_cpu_capability(),
        "cases": {name: run_case(name, spec, sr) for name, spec in CASES.items()},
    }
    torch.save(fixture, OUTPUT)
    print(f"wrote {OUTPUT} ({OUTPUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
