"""Benchmark of the fused stochastic-rounding AdamW step on one MI355X.

``python bench.py [--steps K] [--warmup W] [--workload NAME]`` times K
optimizer steps (one ``AdamWHip.step()`` = one pass of the fused kernel over
every parameter) after W untimed warmup steps, and prints ONE JSON line.
K and W default to the workload's own values (100 and 25 for the north
star; more for short launches, so that the warmup spans the few hundred
milliseconds in which the GPU raises its clocks).

Default workload ``north_star``: AdamW with stochastically rounded BF16
moments over the 1.55 G-element multi-tensor set of the mixed-FP8 config's
shapes (7 blocks of 4x 4096x4096 + 3x 4096x11008, plus a 32000x4096
embedding; FP32 parameters and gradients), lr=3e-4, betas=(0.9, 0.999),
eps=1e-8, weight_decay=0.01, seed=7.  Inputs are synthetic (seeded normal
draws generated on the GPU), resident in HBM before timing starts.

Roofline: the kernel is HBM-bound.  Algorithmic bytes per element are the
minimum reads+writes: parameter read+write, gradient read, each moment
read+write, at their storage widths (20 B for FP32 p/g and BF16 moments).
``achieved`` = bytes per launch / mean kernel time: two HIP events on the
launch stream bracket the K back-to-back steps (one launch per step).  A
second pass of K steps, each started on an idle GPU between its own two
events, gives ``step_ms_median`` (and min, max; the events add about 2 us
per step), ``host_ms_submit`` (median host time until step() returns) and
``host_ms_wall`` (median host time until the step's work has finished).
``traffic`` comes from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE
measurement of the same workload, scaled by a copy-kernel calibration, when
present; ``traffic_source`` names that summary and the build it measured.
``pattern_ceiling`` is the rate of a trivial-math kernel that moves exactly
the same streams (widths, tile shape and order, non-temporal accesses) over
the same number of elements (tests/native/stream_ceiling.hip), timed in the
same process after the workload's tensors are freed, also over
back-to-back launches, at the best of four stream placements and three
resident-workgroup caps (none, that of an 80 KiB budget, half of it): what the memory
system gives this access pattern at this footprint.  ``frac`` there is the
fused kernel's rate over it.

``--workload footprint_sweep`` times the fused AdamW kernel and the trivial
kernel with the north star's streams on one tensor at six footprints from
1.34 to 31 GB, each with the library's resident-workgroup cap and without.

``torch_fused``: torch's own ``torch.optim.AdamW`` / ``SGD`` with
``fused=True`` (states in the parameters' dtype), timed the same way on the same parameters
and gradients after the fused SR steps (the vendor baseline the reference's
step benchmark reports its speedup against); ``speedup`` is its time per
step over the fused SR step's.  For casts, ``torch_cast`` times torch's own
conversion (``Tensor.copy_`` into the output dtype, round to nearest) on the
same buffers.

cpu_baseline: the reference's eager CPU path (restated in oracle/sr_oracle.py
with the same torch operations) timed on this host on a bounded sample of
the same workload.  ``validation``, in the same leg: sampled chunks of the
timed workload's tensors, read before the first step and after the last,
replayed through every step (warmup and both timed passes) by the C oracle
and compared byte for byte; the run fails if any byte differs.

``--separate-states`` gives every optimizer state an allocation of its own,
as the reference does, instead of the optimizers' default of one allocation
per state name for the states a step creates together;
``config.state_allocation`` says which ran.

``config.resident_cap`` is the resident-workgroup cap the library's large
optimizer launches ran with: "rule" (its own choice per launch), or the value
of ``SR_STATES_RESIDENT_CAP`` when that environment variable replaces it.

``--workload cast_sizes`` times the reference cast benchmark's size sweep
(2^10 to 2^24): this backend's stochastic and nearest BF16 casts and torch's
conversion, per size.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "stochastic-rounding-pytorch_amd"))

import torch  # noqa: E402

HBM_PEAK_GBPS = 8000.0

C4_BLOCK = [(4096, 4096)] * 4 + [(4096, 11008)] * 3
WORKLOADS = {
    # name: (optimizer, shapes, param dtype, grad dtype, state formats, hyperparameters)
    "north_star": dict(
        optimizer="adamw",
        shapes=C4_BLOCK * 7 + [(32000, 4096)],
        p_dtype=torch.float32,
        g_dtype=torch.float32,
        formats=((torch.bfloat16, "stochastic"), (torch.bfloat16, "stochastic")),
        grad_std=1e-3,
        hparams=dict(lr=3e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01),
        seed=7,
    ),
    # Config 1: standalone SR cast of 2^24 FP32 values to BF16 (seed 7).  Eight
    # input/output buffer pairs rotate so that 640 MB of traffic passes through
    # the 256 MB last-level cache between reuses of a buffer.
    "c1_cast_bf16": dict(
        warmup=20000,
        steps=5000,
        optimizer="cast",
        shapes=[(1 << 24,)],
        p_dtype=torch.float32,
        g_dtype=torch.float32,
        formats=((torch.bfloat16, "stochastic"),),
        grad_std=1.0,
        hparams={},
        seed=7,
    ),
    "c2_single_2e26": dict(
        warmup=1500,
        steps=500,
        optimizer="adamw",
        shapes=[(1 << 26,)],
        p_dtype=torch.float32,
        g_dtype=torch.float32,
        formats=((torch.bfloat16, "stochastic"), (torch.bfloat16, "stochastic")),
        grad_std=1e-3,
        hparams=dict(lr=3e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01),
        seed=7,
    ),
    # Config 3: GPT-2 small shapes (148 tensors, 124,439,808 elements), FP32
    # parameters with BF16 gradients, BF16-SR moments
    # (benchmarks/bench_optimizer_steps.py:33-53).
    "c3_gpt2": dict(
        warmup=1000,
        steps=300,
        optimizer="adamw",
        shapes=[(50257, 768), (1024, 768)]
        + [(768,), (768,), (768, 2304), (2304,), (768, 768), (768,), (768,), (768,),
           (768, 3072), (3072,), (3072, 768), (768,)] * 12
        + [(768,), (768,)],
        p_dtype=torch.float32,
        g_dtype=torch.bfloat16,
        formats=((torch.bfloat16, "stochastic"), (torch.bfloat16, "stochastic")),
        grad_std=1e-3,
        hparams=dict(lr=3e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01),
        seed=7,
    ),
    # Llama 3.2 1B shapes, the reference benchmark's other model
    # (benchmarks/bench_optimizer_steps.py:54-69): 146 tensors, 1,235,814,400
    # elements, FP32 parameters and gradients, BF16-SR moments, with that
    # benchmark's hyperparameters (bench_optimizer_steps.py:200-203).
    "llama32_1b": dict(
        optimizer="adamw",
        shapes=[(128256, 2048)]
        + [(2048,), (2048, 2048), (512, 2048), (512, 2048), (2048, 2048), (2048,),
           (8192, 2048), (8192, 2048), (2048, 8192)] * 16
        + [(2048,)],
        p_dtype=torch.float32,
        g_dtype=torch.float32,
        formats=((torch.bfloat16, "stochastic"), (torch.bfloat16, "stochastic")),
        grad_std=1e-3,
        hparams=dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-2),
        seed=7,
    ),
    # Config 4: E4M3-SR first moment, BF16-SR second moment over the 1.5 G
    # element set; gradients carry values beyond +-448/(1-beta1) and +-Inf so
    # that the saturating E4M3 encoder is exercised.
    "c4_fp8_mixed": dict(
        optimizer="adamw",
        shapes=C4_BLOCK * 7 + [(32000, 4096)],
        p_dtype=torch.float32,
        g_dtype=torch.float32,
        formats=((torch.float8_e4m3fn, "stochastic"), (torch.bfloat16, "stochastic")),
        grad_std=1e-3,
        special="saturate",
        hparams=dict(lr=3e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01),
        seed=7,
    ),
    # Config 4 at its literal size: 24 blocks plus the embedding, 4.99 G
    # elements (55 GB of parameters, gradients and moments).
    "c4_fp8_24block": dict(
        optimizer="adamw",
        shapes=C4_BLOCK * 24 + [(32000, 4096)],
        p_dtype=torch.float32,
        g_dtype=torch.float32,
        formats=((torch.float8_e4m3fn, "stochastic"), (torch.bfloat16, "stochastic")),
        grad_std=1e-3,
        special="saturate",
        hparams=dict(lr=3e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01),
        seed=7,
    ),
    # The north star's shapes with BF16 parameters and gradients, for three
    # state formats: the launches where the FP32 update's arithmetic, not
    # memory, sets the rate.
    "bf16_params_bf16sr": dict(
        optimizer="adamw",
        shapes=C4_BLOCK * 7 + [(32000, 4096)],
        p_dtype=torch.bfloat16,
        g_dtype=torch.bfloat16,
        formats=((torch.bfloat16, "stochastic"), (torch.bfloat16, "stochastic")),
        grad_std=1e-3,
        hparams=dict(lr=3e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01),
        seed=7,
    ),
    "bf16_params_e4m3_bf16sr": dict(
        optimizer="adamw",
        shapes=C4_BLOCK * 7 + [(32000, 4096)],
        p_dtype=torch.bfloat16,
        g_dtype=torch.bfloat16,
        formats=((torch.float8_e4m3fn, "stochastic"), (torch.bfloat16, "stochastic")),
        grad_std=1e-3,
        hparams=dict(lr=3e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01),
        seed=7,
    ),
    "bf16_params_fp16sr": dict(
        optimizer="adamw",
        shapes=C4_BLOCK * 7 + [(32000, 4096)],
        p_dtype=torch.bfloat16,
        g_dtype=torch.bfloat16,
        formats=((torch.float16, "stochastic"), (torch.float16, "stochastic")),
        grad_std=1e-3,
        hparams=dict(lr=3e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01),
        seed=7,
    ),
    # Stochastic casts of 2^26 values, eight rotating buffer pairs, per output format.
    **{
        f"cast_2e26_{name}": dict(
            warmup=5000,
            steps=2000,
            optimizer="cast",
            shapes=[(1 << 26,)],
            p_dtype=torch.float32,
            g_dtype=torch.float32,
            formats=((dtype, "stochastic"),),
            grad_std=1.0,
            hparams={},
            seed=7,
        )
        for name, dtype in (("bf16", torch.bfloat16), ("fp16", torch.float16),
                            ("e4m3", torch.float8_e4m3fn), ("e5m2", torch.float8_e5m2))
    },
    # A plain device copy of known size (4 GiB read + 4 GiB written per step);
    # its rocprofv3 FETCH_SIZE / WRITE_SIZE readings calibrate the counters.
    "copy_calibration": dict(
        optimizer="copy",
        shapes=[(1 << 30,)],
        p_dtype=torch.float32,
        g_dtype=torch.float32,
        formats=(),
        grad_std=1.0,
        hparams={},
        seed=0,
    ),
    # The north star's streams (FP32 p/g, BF16-SR m/v) on one tensor at six
    # footprints from 1.34 to 31 GB: the fused kernel and the trivial kernel
    # with the same streams, each with the library's resident-workgroup cap
    # and without one (tests/native/stream_ceiling.hip, sr_launch_cap_sweep).
    # steps = launches per measurement, warmup = interleaved rounds.
    "footprint_sweep": dict(
        optimizer="footprint",
        shapes=[(1547698176,)],
        p_dtype=torch.float32,
        g_dtype=torch.float32,
        formats=((torch.bfloat16, "stochastic"), (torch.bfloat16, "stochastic")),
        grad_std=1e-3,
        hparams={},
        seed=0,
        steps=100,
        warmup=2,
    ),
    # The reference cast benchmark's size sweep (benchmarks/bench_sr_cast.py:
    # 25-27: 2^10 to 2^24 in steps of 4x) of FP32 -> BF16: this backend's
    # stochastic and nearest casts beside torch's conversion, per size.
    "cast_sizes": dict(
        optimizer="cast_sweep",
        shapes=[(1 << k,) for k in range(10, 25, 2)],
        p_dtype=torch.float32,
        g_dtype=torch.float32,
        formats=((torch.bfloat16, "stochastic"),),
        grad_std=1.0,
        hparams={},
        seed=7,
        steps=2000,
        warmup=5000,
    ),
    # Host time per call of the single-tensor entries (1024 elements, BF16-SR
    # states) and per step of the optimizers on GPT-2's shapes, beside
    # torch's fused AdamW and conversion: not an optimizer step.
    "host_costs": dict(
        optimizer="host",
        shapes=[(1024,)],
        p_dtype=torch.float32,
        g_dtype=torch.float32,
        formats=((torch.bfloat16, "stochastic"), (torch.bfloat16, "stochastic")),
        grad_std=1e-3,
        hparams=dict(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=1e-2),
        seed=7,
        steps=2000,
        warmup=200,
    ),
    # Config 5: gradients with 5% exact zeros, 1% of magnitude below 2^-14
    # (FP16 subnormal range) and the rest N(0, 1e-2).
    "c5_sgdm_fp16": dict(
        optimizer="sgdm",
        shapes=[(2048, 2048)] * 256,
        p_dtype=torch.float32,
        g_dtype=torch.float32,
        formats=((torch.float16, "stochastic"),),
        grad_std=1e-2,
        special="zeros_subnormal",
        hparams=dict(lr=0.1, momentum=0.9),
        seed=11,
    ),
}


def bytes_per_element(spec) -> int:
    size = lambda dt: torch.empty((), dtype=dt).element_size()  # noqa: E731
    if spec["optimizer"] == "copy":
        return 2 * size(spec["p_dtype"])
    if spec["optimizer"] == "cast":
        return size(spec["p_dtype"]) + size(spec["formats"][0][0])
    states = sum(2 * size(dt) for dt, _ in spec["formats"])
    return 2 * size(spec["p_dtype"]) + size(spec["g_dtype"]) + states


class _Param(torch.nn.Parameter):
    """Parameter whose gradient may have another dtype (BF16 grads of FP32 params)."""

    @property
    def grad(self):
        return getattr(self, "_gradient", None)

    @grad.setter
    def grad(self, value):
        self._gradient = value


def make_gradient(shape, spec, gen, device):
    """FP32 gradient of one tensor of a workload, with the config's special values."""
    g = torch.empty(shape, device=device, dtype=torch.float32).normal_(
        std=spec["grad_std"], generator=gen
    )
    flat = g.view(-1)
    special = spec.get("special")
    if special == "saturate":
        # |g| = 5000 makes |m'| = 500 > 448 at the first step.
        flat[5::997] = 5000.0
        flat[500::1994] = -5000.0
        flat[11::1_000_003] = float("inf")
        flat[600_011::1_000_003] = float("-inf")
    elif special == "zeros_subnormal":
        u = torch.rand(flat.shape, device=device, generator=gen)
        tiny = (torch.rand(flat.shape, device=device, generator=gen) * 2 - 1) * 2.0**-14
        flat.copy_(torch.where(u < 0.05, 0.0, torch.where(u < 0.06, tiny, flat)))
    elif special is not None:
        raise ValueError(f"unknown special gradient values {special!r}")
    return g


def make_optimizer(spec, device):
    """(parameters, optimizer) of an optimizer workload, inputs resident on `device`."""
    import sr_states
    from sr_states import StateFormat

    gen = torch.Generator(device=device).manual_seed(spec["seed"])
    params = []
    for shape in spec["shapes"]:
        p = _Param(torch.empty(shape, device=device, dtype=spec["p_dtype"]))
        with torch.no_grad():
            p.normal_(std=0.02, generator=gen)
        p.grad = make_gradient(shape, spec, gen, device).to(spec["g_dtype"])
        params.append(p)
    names = ("exp_avg", "exp_avg_sq") if spec["optimizer"] == "adamw" else ("momentum_buffer",)
    formats = {n: StateFormat(d, r) for n, (d, r) in zip(names, spec["formats"])}
    cls = sr_states.AdamWHip if spec["optimizer"] == "adamw" else sr_states.SGDMHip
    return params, cls(params, state_format=formats, seed=spec["seed"], **spec["hparams"])


class Workload:
    """A built workload: its tensors, one step, and what validation reads back."""

    def __init__(self, tensors, step, optimizer=None, casts=None):
        self.tensors = tensors      # the tensors whose elements one step processes
        self.step = step
        self.optimizer = optimizer  # AdamWHip / SGDMHip of an optimizer workload
        self.casts = casts          # (inputs, outputs) of a cast workload


def build(spec, device):
    """The workload's inputs, resident on `device`, and its step."""
    import sr_states

    gen = torch.Generator(device=device).manual_seed(spec["seed"])
    if spec["optimizer"] == "copy":
        src = torch.empty(spec["shapes"][0], device=device).normal_(generator=gen)
        dst = torch.empty_like(src)
        return Workload([src], lambda: dst.copy_(src))
    if spec["optimizer"] == "cast":
        from sr_states.hip.cast import native_cast

        (dtype, rule), = spec["formats"]
        inputs = [torch.empty(spec["shapes"][0], device=device).normal_(generator=gen) for _ in range(8)]
        outputs = [torch.empty(spec["shapes"][0], device=device, dtype=dtype) for _ in range(8)]
        turn = [0]
        code = sr_states._lib.RULE_CODES[rule]

        def cast_step():
            k = turn[0] = (turn[0] + 1) % len(inputs)
            native_cast(inputs[k], dtype=dtype, rule=code, seed=spec["seed"], out=outputs[k])

        return Workload(inputs[:1], cast_step, casts=(inputs, outputs))
    params, opt = make_optimizer(spec, device)
    return Workload(params, opt.step, optimizer=opt)


# Validation samples: chunks of this many elements (odd, so that chunk edges
# fall inside the kernels' 4-element lane groups) at the head, the tail and
# random interior starts of a few tensors.
SAMPLE_CHUNK = 4099


def _sample_chunks(numel, count, rng):
    starts = {0, max(0, numel - SAMPLE_CHUNK)}
    while len(starts) < min(count, max(1, numel // SAMPLE_CHUNK)):
        starts.add(rng.randrange(0, max(1, numel - SAMPLE_CHUNK)))
    return [(s, min(SAMPLE_CHUNK, numel - s)) for s in sorted(starts)]


def snapshot_samples(spec, work, tensors=3, chunks=3):
    """Host copies of sampled chunks of the inputs, taken before the first step.

    Each entry is (tensor index, start, length, inputs): the parameter and
    gradient chunks of an optimizer workload, or the input chunk of one of
    the cast's buffer pairs.
    """
    import random

    rng = random.Random(spec["seed"])
    if spec["optimizer"] == "cast":
        inputs, _ = work.casts
        picks = [0, len(inputs) - 1]
        return [(k, s, n, [inputs[k].view(-1)[s:s + n].cpu()])
                for k in picks for s, n in _sample_chunks(inputs[k].numel(), chunks, rng)]
    if spec["optimizer"] not in ("adamw", "sgdm"):
        return None
    params = work.tensors
    picks = sorted({0, len(params) - 1, *rng.sample(range(len(params)), min(tensors, len(params)) - 1)})
    samples = []
    for index in picks:
        p = params[index]
        flat_p, flat_g = p.detach().view(-1), p.grad.view(-1)
        for start, length in _sample_chunks(p.numel(), chunks, rng):
            samples.append((index, start, length, [flat_p[start:start + length].cpu(),
                                                   flat_g[start:start + length].cpu()]))
    return samples


def read_back(spec, work, samples):
    """The device bytes of every sampled chunk after the last step."""
    if samples is None:
        return None
    if spec["optimizer"] == "cast":
        _, outputs = work.casts
        return [[outputs[k].view(-1)[s:s + n].cpu()] for k, s, n, _ in samples]
    opt, params = work.optimizer, work.tensors
    finals = []
    for index, start, length, _ in samples:
        p = params[index]
        values = [p.detach().view(-1)[start:start + length].cpu()]
        values += [opt.state[p][name].view(-1)[start:start + length].cpu() for name in opt._state_names]
        finals.append(values)
    return finals


def validate(spec, samples, finals, steps):
    """Replay every step on the sampled chunks with the C oracle; compare bytes.

    Each element's update depends only on its own inputs, its flat index and
    its parameter's update key, so the oracle run on a chunk with ``offset``
    set to the chunk's start must reproduce the device's bytes exactly (NaN
    payloads aside), after all ``steps`` optimizer steps (warmup and timed).
    """
    sys.path.insert(0, str(ROOT))
    from oracle import c_oracle, sr_oracle

    def same(actual, expected):
        a, e = actual.float(), expected.float()
        nan = torch.isnan(e)
        if not torch.equal(torch.isnan(a), nan):
            return int((torch.isnan(a) != nan).sum())
        bits = {4: torch.int32, 2: torch.int16, 1: torch.uint8}[actual.element_size()]
        return int((actual.view(bits)[~nan] != expected.view(bits)[~nan]).sum())

    mismatches = checked = 0
    started = time.perf_counter()
    for (index, start, length, inputs), final in zip(samples, finals):
        if spec["optimizer"] == "cast":
            (dtype, rule), = spec["formats"]
            expected = [c_oracle.cast(inputs[0], dtype=dtype, rounding=rule, seed=spec["seed"], offset=start)]
        else:
            p, g = inputs[0].clone(), inputs[1]
            states = [torch.zeros(length, dtype=dtype) for dtype, _ in spec["formats"]]
            hp = spec["hparams"]
            for t in range(1, steps + 1):
                key = sr_oracle.update_key(spec["seed"], t, index)
                if spec["optimizer"] == "adamw":
                    c_oracle.adamw_step_(p, g, *states, lr=hp["lr"], beta1=hp["betas"][0], beta2=hp["betas"][1],
                                         eps=hp["eps"], weight_decay=hp["weight_decay"], step=t,
                                         formats=spec["formats"], seed=key, offset=start)
                else:
                    c_oracle.sgdm_step_(p, g, *states, lr=hp["lr"], momentum_factor=hp["momentum"],
                                        formats=spec["formats"], seed=key, offset=start)
            expected = [p, *states]
        for actual, want in zip(final, expected):
            mismatches += same(actual, want)
            checked += want.numel()
    return {
        "oracle": "oracle/sr_oracle.c (C restatement, correctly rounded FP32)",
        "steps_replayed": steps if spec["optimizer"] != "cast" else 1,
        "chunks": len(samples),
        "elements_checked": checked,
        "mismatches": mismatches,
        "seconds": round(time.perf_counter() - started, 2),
    }


def torch_fused_baseline(spec, work, steps, warmup):
    """torch's own fused optimizer on the workload's tensors, or None.

    The reference's step benchmark times ``torch.optim.AdamW`` / ``SGD`` with
    ``fused=True`` beside its own optimizers and reports the speedup
    (benchmarks/bench_optimizer_steps.py:247-251, 440-449).  Here the same
    parameters and gradients (of one dtype: torch's fused kernels take
    gradients of the parameters' dtype) are stepped by torch's kernels after
    the fused SR steps are timed and read back; the time per step comes from
    two events around back-to-back steps, as for the product.  torch keeps
    its states in the parameters' dtype (FP32 for FP32 parameters).
    """
    if spec["optimizer"] not in ("adamw", "sgdm") or spec["p_dtype"] != spec["g_dtype"]:
        return None
    params = []
    for p in work.tensors:
        q = torch.nn.Parameter(p.detach())  # shares p's memory
        q.grad = p.grad
        params.append(q)
    hp = spec["hparams"]
    if spec["optimizer"] == "adamw":
        opt = torch.optim.AdamW(params, fused=True, **hp)
        name, states = "torch.optim.AdamW(fused=True)", 2
    else:
        opt = torch.optim.SGD(params, lr=hp["lr"], momentum=hp["momentum"], fused=True)
        name, states = "torch.optim.SGD(momentum, fused=True)", 1
    try:
        for _ in range(max(1, min(warmup, 25))):
            opt.step()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record()
        for _ in range(steps):
            opt.step()
        end.record()
        torch.cuda.synchronize()
    except RuntimeError as error:  # a torch build without the fused kernels
        return {"optimizer": name, "error": str(error).splitlines()[0]}
    ms = start.elapsed_time(end) / steps
    size = lambda dt: torch.empty((), dtype=dt).element_size()  # noqa: E731
    bpe = 2 * size(spec["p_dtype"]) + size(spec["g_dtype"]) + 2 * size(spec["p_dtype"]) * states
    elements = sum(p.numel() for p in params)
    del opt, params
    return {"optimizer": name, "state_dtype": str(spec["p_dtype"]).replace("torch.", ""),
            "ms_per_step": ms, "bytes_per_element": bpe,
            "achieved_gbps": bpe * elements / (ms / 1e3) / 1e9,
            "frac": bpe * elements / (ms / 1e3) / 1e9 / HBM_PEAK_GBPS}


def torch_cast_baseline(spec, work, steps, warmup):
    """torch's own conversion (``Tensor.copy_`` into the output dtype, round to nearest) on the
    cast workload's rotating buffer pairs, timed like the product's casts; None for other workloads.

    The reference's cast benchmark times ``x.to(torch.bfloat16)`` beside its
    own casts (benchmarks/bench_sr_cast.py:38-46); ``copy_`` into the
    preallocated outputs is the same conversion kernel without the
    allocation.
    """
    if spec["optimizer"] != "cast":
        return None
    inputs, outputs = work.casts
    turn = [0]

    def convert():
        k = turn[0] = (turn[0] + 1) % len(inputs)
        outputs[k].copy_(inputs[k])

    op = "Tensor.copy_ to the output dtype (round to nearest)"
    try:
        for _ in range(warmup):
            convert()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record()
        for _ in range(steps):
            convert()
        end.record()
        torch.cuda.synchronize()
    except RuntimeError as error:  # a torch build without this conversion on the device
        return {"op": op, "error": str(error).splitlines()[0]}
    ms = start.elapsed_time(end) / steps
    bpe = bytes_per_element(spec)
    elements = inputs[0].numel()
    return {"op": op, "ms_per_step": ms,
            "bytes_per_element": bpe, "achieved_gbps": bpe * elements / (ms / 1e3) / 1e9,
            "frac": bpe * elements / (ms / 1e3) / 1e9 / HBM_PEAK_GBPS}


def cast_sizes(spec, steps, warmup):
    """Per-size time of the HIP stochastic and nearest BF16 casts and of torch's conversion.

    Each size uses eight rotating input/output pairs (at least 512 MB of
    traffic between reuses of a buffer for the larger sizes) and is timed
    over back-to-back calls between two events, after ``warmup`` calls.
    """
    from sr_states import _lib
    from sr_states.hip.cast import native_cast

    device = torch.device("cuda", 0)
    gen = torch.Generator(device=device).manual_seed(spec["seed"])
    rows = []
    for (n,) in spec["shapes"]:
        inputs = [torch.empty(n, device=device).normal_(generator=gen) for _ in range(8)]
        outputs = [torch.empty(n, device=device, dtype=torch.bfloat16) for _ in range(8)]
        methods = {
            "hip_sr": lambda k: native_cast(inputs[k], dtype=torch.bfloat16, rule=_lib.RULE_CODES["stochastic"],
                                            seed=spec["seed"], out=outputs[k]),
            "hip_rn": lambda k: native_cast(inputs[k], dtype=torch.bfloat16, rule=_lib.RULE_CODES["nearest"],
                                            out=outputs[k]),
            "torch_rn": lambda k: outputs[k].copy_(inputs[k]),
        }
        row = {"elements": n}
        for name, call in methods.items():
            for i in range(warmup):
                call(i % 8)
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            start.record()
            for i in range(steps):
                call(i % 8)
            end.record()
            torch.cuda.synchronize()
            us = start.elapsed_time(end) / steps * 1e3
            row[f"{name}_us"] = us
            row[f"{name}_gbps"] = 6 * n / (us / 1e6) / 1e9
        row["hip_sr_speedup_vs_torch_rn"] = row["torch_rn_us"] / row["hip_sr_us"]
        rows.append(row)
        del inputs, outputs
    return rows


def host_costs(spec, steps, warmup):
    """Host time per call of the single-tensor entries and per optimizer step.

    Each entry runs ``warmup`` untimed calls, then ``steps`` back-to-back
    calls (a tenth as many for the GPT-2 optimizer steps) with Python's
    cyclic garbage collector paused, so that one collection over torch's
    objects (tens of milliseconds) does not land in one entry's average.
    ``host_us`` is the time for the calls to return; ``device_us`` spans the
    same calls between two events on the current stream, so it equals
    ``host_us`` when the host bounds the rate and exceeds it otherwise.
    """
    import gc

    import sr_states
    import sr_states.reference as functional
    from sr_states.hip.adamw import hip_adamw_step_
    from sr_states.hip.sgd import hip_sgdm_step_

    device = torch.device("cuda", 0)
    gen = torch.Generator(device=device).manual_seed(spec["seed"])
    (n,) = spec["shapes"][0]
    p = torch.empty(n, device=device).normal_(generator=gen)
    g = torch.empty(n, device=device).normal_(generator=gen) * spec["grad_std"]
    m = torch.zeros(n, device=device, dtype=torch.bfloat16)
    v = torch.zeros(n, device=device, dtype=torch.bfloat16)
    x = torch.empty(n, device=device).normal_(generator=gen)
    hp = {**spec["hparams"], "step": 3}
    sgd = {"lr": hp["lr"], "momentum_factor": 0.9}
    shapes = WORKLOADS["c3_gpt2"]["shapes"]

    def gpt2_params():
        params = [torch.nn.Parameter(torch.empty(s, device=device).normal_(generator=gen) * 0.02) for s in shapes]
        for q in params:
            q.grad = torch.empty_like(q).normal_(generator=gen) * spec["grad_std"]
        return params

    torch_params = gpt2_params()
    torch_adamw = torch.optim.AdamW(torch_params, lr=hp["lr"], fused=True)
    entries = {
        "hip_adamw_step_": (lambda: hip_adamw_step_(p, g, m, v, seed=7, **hp), 1),
        "hip_sgdm_step_": (lambda: hip_sgdm_step_(p, g, m, seed=7, **sgd), 1),
        "reference.adamw_step_": (lambda: functional.adamw_step_(p, g, m, v, seed=7, **hp), 1),
        "reference.sgdm_step_": (lambda: functional.sgdm_step_(p, g, m, seed=7, **sgd), 1),
        "sr_states.cast (BF16 SR)": (lambda: sr_states.cast(x, dtype=torch.bfloat16, seed=7), 1),
        "torch: x.to(bfloat16)": (lambda: x.to(torch.bfloat16), 1),
        "AdamWHip.step (GPT-2, 148 tensors)": (sr_states.AdamWHip(gpt2_params(), lr=hp["lr"]).step, 10),
        "AdamWReferenceSR.step (GPT-2, 148 tensors)": (sr_states.AdamWReferenceSR(gpt2_params(), lr=hp["lr"]).step, 10),
        "torch.optim.AdamW(fused=True).step (GPT-2, FP32 states)": (torch_adamw.step, 10),
    }
    rows = []
    for name, (call, divisor) in entries.items():
        count = max(1, steps // divisor)
        for _ in range(max(1, warmup // divisor)):
            call()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        gc.collect()
        gc.disable()
        try:
            start.record()
            began = time.perf_counter_ns()
            for _ in range(count):
                call()
            returned = time.perf_counter_ns()
            end.record()
            torch.cuda.synchronize()
        finally:
            gc.enable()
        rows.append({"entry": name, "calls": count, "host_us": (returned - began) / count / 1e3,
                     "device_us": start.elapsed_time(end) * 1e3 / count})
    return rows


def _median_step_seconds(opt, target_seconds: float, min_steps: int = 3) -> tuple[float, int]:
    opt.step()  # allocate states
    times = []
    start = time.perf_counter()
    while time.perf_counter() - start < target_seconds or len(times) < min_steps:
        t0 = time.perf_counter_ns()
        opt.step()
        times.append((time.perf_counter_ns() - t0) / 1e9)
    return sorted(times)[len(times) // 2], len(times)


def cpu_baseline(spec, target_seconds: float = 12.0):
    """Time the eager CPU path (oracle restatement) on one tensor of the workload.

    Two thirds of the budget go to torch's default thread count, the rest to
    one thread on a quarter-size sample.
    """
    sys.path.insert(0, str(ROOT))
    from oracle import sr_oracle

    shape = max(spec["shapes"], key=lambda s: math.prod(s))
    n = min(math.prod(shape), 1 << 24)

    def make(count):
        gen = torch.Generator().manual_seed(spec["seed"])
        p = (torch.randn(count, generator=gen) * 0.02).to(spec["p_dtype"])
        g = make_gradient((count,), spec, gen, "cpu").to(spec["g_dtype"])
        if spec["optimizer"] == "cast":
            (dtype, rule), = spec["formats"]

            class _Cast:
                def step(self):
                    sr_oracle.cast(p, dtype=dtype, rounding=rule, seed=spec["seed"])

            return _Cast()
        formats = tuple(sr_oracle.Fmt(d, r) for d, r in spec["formats"])
        group = {"params": [p], "grads": [g], "formats": formats, "sr_seed": spec["seed"],
                 **spec["hparams"]}
        cls = sr_oracle.AdamWOracle if spec["optimizer"] == "adamw" else sr_oracle.SGDMOracle
        return cls([group])

    threads = torch.get_num_threads()
    model = "unknown CPU"
    try:
        with open("/proc/cpuinfo") as info:
            model = next(line.split(":", 1)[1].strip() for line in info if line.startswith("model name"))
    except (OSError, StopIteration):
        pass
    median, count = _median_step_seconds(make(n), target_seconds * 2 / 3)
    n1 = max(n // 4, 1)
    torch.set_num_threads(1)
    try:
        median1, count1 = _median_step_seconds(make(n1), target_seconds / 3)
    finally:
        torch.set_num_threads(threads)
    return {
        "value": n / median,
        "unit": "params/s",
        "cores": threads,
        "kind": "port",
        "value_one_thread": n1 / median1,
        "sample": f"{count} eager steps of one {n}-element tensor of the workload at {threads} "
        f"threads (median {median * 1e3:.1f} ms) and {count1} steps of {n1} elements at 1 thread "
        f"(median {median1 * 1e3:.1f} ms); {model}, torch {torch.__version__}, "
        f"{torch.backends.cpu.get_cpu_capability()}, {os.cpu_count()} host CPUs visible",
    }


CEILING_LIBRARY = ROOT / "tests" / "native" / "libstream_ceiling.so"


def pattern_ceiling(spec, elements: int, reps: int):
    """Rate of the trivial kernel with this workload's streams, or None where none applies.

    Covers AdamW and SGDM launches whose parameter, gradient and states
    match one of the probe's patterns, and the cast with its eight rotating
    buffer pairs (tests/native/stream_ceiling.hip).
    """
    if spec["optimizer"] not in ("adamw", "sgdm", "cast"):
        return None
    if not CEILING_LIBRARY.exists():
        return None
    import ctypes

    size = lambda dt: torch.empty((), dtype=dt).element_size()  # noqa: E731
    lib = ctypes.CDLL(str(CEILING_LIBRARY))
    ms = ctypes.c_float()
    if spec["optimizer"] == "cast":
        lib.sr_cast_ceiling.restype = ctypes.c_int
        lib.sr_cast_ceiling.argtypes = [ctypes.c_uint64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                        ctypes.POINTER(ctypes.c_float)]
        n = elements // 2048 * 2048
        rc = lib.sr_cast_ceiling(n, size(spec["formats"][0][0]), 8, reps, ctypes.byref(ms))
    else:
        widths = [size(spec["g_dtype"])] + [size(dt) for dt, _ in spec["formats"]]
        if len(widths) == 2:
            widths.append(0)
        lib.sr_stream_ceiling_p.restype = ctypes.c_int
        lib.sr_stream_ceiling_p.argtypes = [ctypes.c_uint64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                            ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_float)]
        n = elements // 512 * 512
        rc = lib.sr_stream_ceiling_p(n, size(spec["p_dtype"]), *widths, reps, ctypes.byref(ms))
    if rc != 0:
        return None
    return {"achieved": bytes_per_element(spec) * n / ms.value / 1e6, "kernel_ms": ms.value,
            "elements": n, "kernel": "stream_ceiling.hip: same streams, trivial arithmetic"}


FOOTPRINTS_GB = (1.34, 2.68, 5.0, 10.0, 20.0, 30.95)


def footprint_sweep(reps: int, rounds: int):
    """Rates of the fused AdamW kernel and the trivial kernel by footprint, with and without the cap."""
    import ctypes

    if not CEILING_LIBRARY.exists():
        raise SystemExit(f"{CEILING_LIBRARY} is not built (tests/native/build_checks.py)")
    lib = ctypes.CDLL(str(CEILING_LIBRARY))
    lib.sr_launch_cap_sweep.restype = ctypes.c_int
    lib.sr_launch_cap_sweep.argtypes = [ctypes.c_uint64, ctypes.c_int, ctypes.POINTER(ctypes.c_int), ctypes.c_int,
                                        ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_float),
                                        ctypes.POINTER(ctypes.c_int)]
    caps = (ctypes.c_int * 2)(-1, 0)  # the library's rule, then none
    rows = []
    for _ in range(rounds):
        for gb in FOOTPRINTS_GB:
            n = int(gb * 1e9 / 20) >> 21 << 21  # whole 2^21-element chunk rounds
            trivial, fused, resident = (ctypes.c_float * 2)(), (ctypes.c_float * 2)(), (ctypes.c_int * 2)()
            if lib.sr_launch_cap_sweep(n, max(5, min(reps, int(300 / (n * 20 / 6e9)))), caps, 2, trivial, fused,
                                       resident) != 0:
                raise SystemExit("sr_launch_cap_sweep failed")
            rate = lambda ms: 20 * n / ms / 1e6  # noqa: E731  (GB/s)
            rows.append({"elements": n, "gb": 20 * n / 1e9,
                         "fused_capped_gbps": rate(fused[0]), "fused_uncapped_gbps": rate(fused[1]),
                         "trivial_capped_gbps": rate(trivial[0]), "trivial_uncapped_gbps": rate(trivial[1]),
                         "resident_capped": resident[0], "resident_uncapped": resident[1]})
            print(f"footprint {rows[-1]['gb']:.2f} GB: fused {rows[-1]['fused_capped_gbps']:.0f} / "
                  f"{rows[-1]['fused_uncapped_gbps']:.0f} GB/s (cap {resident[0]} / {resident[1]} per CU), trivial "
                  f"{rows[-1]['trivial_capped_gbps']:.0f} / {rows[-1]['trivial_uncapped_gbps']:.0f}",
                  file=sys.stderr, flush=True)
    return rows


def load_traffic(workload: str):
    """HBM bytes per launch from the committed rocprofv3 FETCH/WRITE summary, and where they come from.

    Returns (bytes, source) or (None, None): ``source`` names the summary
    under profiles/ and the build commit it records.  The counters are not
    collected in this run (rocprofv3 --pmc runs the program under the
    profiler, one counter per pass).
    """
    for path in sorted((ROOT / "profiles").glob(f"*_{workload}_hbm_traffic.md")):
        value, build = None, None
        for line in path.read_text().splitlines():
            if line.startswith("hbm_bytes_per_launch:"):
                value = float(line.split(":", 1)[1])
            elif line.startswith("build_commit:"):
                build = line.split(":", 1)[1].strip()
        if value is not None:
            return value, {"profile": str(path.relative_to(ROOT)), "build_commit": build,
                           "measured": "rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE, one pass each, "
                                       "scaled by a 4 GiB copy's readings"}
    return None, None


def positive_int(text: str) -> int:
    """argparse type: an integer of at least 1."""
    value = int(text)
    if value < 1:
        raise argparse.ArgumentTypeError(f"{text} is not a positive integer")
    return value


def nonnegative_int(text: str) -> int:
    """argparse type: an integer of at least 0."""
    value = int(text)
    if value < 0:
        raise argparse.ArgumentTypeError(f"{text} is not a nonnegative integer")
    return value


def positive_float(text: str) -> float:
    """argparse type: a finite number above 0."""
    value = float(text)
    if not math.isfinite(value) or value <= 0:
        raise argparse.ArgumentTypeError(f"{text} is not a positive number")
    return value


def main():
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=positive_int, default=1)
    parser.add_argument("--steps", type=positive_int, default=None,
                        help="timed steps (default: the workload's, 100 for the north star)")
    parser.add_argument("--warmup", type=nonnegative_int, default=None,
                        help="untimed warmup steps (default: the workload's, 25 for the north star)")
    parser.add_argument("--workload", choices=sorted(WORKLOADS), default="north_star")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-ceiling", action="store_true",
                        help="skip the access-pattern ceiling measurement")
    parser.add_argument("--no-torch-baseline", action="store_true",
                        help="skip timing torch's fused optimizer with FP32 states on the same tensors")
    parser.add_argument("--cpu-seconds", type=positive_float, default=12.0)
    parser.add_argument("--separate-states", action="store_true",
                        help="one allocation per optimizer state, as the reference makes them (default: the "
                             "states a step creates share one allocation per state name)")
    parser.add_argument("--state-format", default=None, metavar="DTYPE/RULE",
                        help="store every state of the workload in this format instead, e.g. "
                             "float8_e4m3fn/stochastic (the reference's nine policies: "
                             "benchmarks/bench_states.py:21-31)")
    args = parser.parse_args()
    state_formats = None
    if args.state_format:
        if WORKLOADS[args.workload]["optimizer"] not in ("adamw", "sgdm", "cast"):
            raise SystemExit(f"--state-format does not apply to {args.workload}")
        dtype_name, _, rule = args.state_format.partition("/")
        dtype = getattr(torch, dtype_name, None)
        if not isinstance(dtype, torch.dtype) or rule not in ("nearest", "stochastic"):
            raise SystemExit(f"--state-format {args.state_format!r}: expected DTYPE/nearest or DTYPE/stochastic")
        state_formats = ((dtype, rule),) * len(WORKLOADS[args.workload]["formats"])
    if args.gpus != 1:
        raise SystemExit(
            "bench.py measures one GPU: the fused update needs no collective, and each rank "
            "would run this same kernel on its own shard; run with --gpus 1"
        )
    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a GPU")
    spec = WORKLOADS[args.workload]
    if state_formats:
        spec = {**spec, "formats": state_formats}
    # Short launches need many warmup steps: the GPU raises its clocks over
    # the first few hundred milliseconds of load, and the FP8 casts at 2^26
    # measured 4.9 TB/s after 25 warmup steps (1.7 ms) against 6.4 after 3000.
    if args.warmup is None:
        args.warmup = spec.get("warmup", 25)
    if args.steps is None:
        args.steps = spec.get("steps", 100)
    device = torch.device("cuda", 0)
    if spec["optimizer"] == "footprint":
        if args.warmup < 1:
            raise SystemExit("--workload footprint_sweep takes --warmup as its number of rounds: at least 1")
        rows = footprint_sweep(args.steps, args.warmup)
        print(json.dumps({
            "metric": "fused AdamW and trivial-kernel rates by footprint, with and without the resident cap, "
                      "1 MI355X",
            "value": rows[-1]["fused_capped_gbps"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "higher_is_better": True, "vs_baseline": None, "dtype": "f32",
            "data": "synthetic (hashed uniform draws on the GPU)",
            "note": "steps = launches per measurement (fewer for large footprints), warmup = interleaved rounds; "
                    "value = the fused kernel, capped, at the largest footprint",
            "peak": HBM_PEAK_GBPS, "rows": rows}), flush=True)
        return
    if spec["optimizer"] == "cast_sweep":
        rows = cast_sizes(spec, args.steps, args.warmup)
        print(json.dumps({
            "metric": "FP32 -> BF16 cast time per call by size, 1 MI355X", "value": rows[-1]["hip_sr_gbps"],
            "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True,
            "vs_baseline": None, "dtype": "f32", "data": "synthetic (seeded normal draws on the GPU)",
            "note": "value = the stochastic cast at the largest size; rows hold every size and method",
            "peak": HBM_PEAK_GBPS, "sizes": rows}), flush=True)
        return
    if spec["optimizer"] == "host":
        rows = host_costs(spec, args.steps, args.warmup)
        print(json.dumps({
            "metric": "host time per call of the single-tensor entries and per optimizer step, 1 MI355X",
            "value": rows[0]["host_us"], "unit": "us", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "higher_is_better": False, "vs_baseline": None, "dtype": "f32",
            "data": "synthetic (seeded normal draws on the GPU)",
            "note": "value = hip_adamw_step_ on 1024 elements; rows hold every entry",
            "entries": rows}), flush=True)
        return
    work = build(spec, device)
    if args.separate_states:
        if work.optimizer is None:
            raise SystemExit(f"--separate-states does not apply to {args.workload}")
        work.optimizer._shared_state_allocations = False
    step = work.step
    elements = sum(t.numel() for t in work.tensors)
    # Inputs of the sampled chunks, read before the first step, for the
    # validation of the timed workload's bytes (cpu_baseline leg).
    samples = None if args.no_cpu_baseline else snapshot_samples(spec, work)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    total_start = torch.cuda.Event(enable_timing=True)
    total_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    total_start.record()
    for _ in range(args.steps):
        step()
    total_end.record()
    torch.cuda.synchronize()
    total_ms = total_start.elapsed_time(total_end)
    ms_per_step = total_ms / args.steps
    # One launch per step, enqueued back to back on the launch stream with the
    # host ahead of the GPU (host work per step: 4 us for the cast, 55 us for
    # C3's 148 tensors), so the time per step is the kernel's average launch
    # duration.  No events sit between the steps: on an 18 us cast they would
    # add about 2 us each.
    kernel_ms = ms_per_step
    # Single steps: a second pass of K steps, each started on an idle GPU
    # and timed three ways (benchmarks/bench_optimizer_steps.py:315-363):
    # device time between two events on the launch stream (which add about
    # 2 us), host time to submit the step (the call returning), and host wall
    # time until the step's work has finished.
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    step_ms, submit_ms, wall_ms = [], [], []
    for _ in range(args.steps):
        torch.cuda.synchronize()
        start.record()
        began = time.perf_counter_ns()
        step()
        returned = time.perf_counter_ns()
        end.record()
        end.synchronize()
        finished = time.perf_counter_ns()
        step_ms.append(start.elapsed_time(end))
        submit_ms.append((returned - began) / 1e6)
        wall_ms.append((finished - began) / 1e6)
    step_ms.sort()
    if not all(math.isfinite(v) and v > 0 for v in (*step_ms, *submit_ms, *wall_ms, total_ms)):
        raise SystemExit("nonpositive or nonfinite step timing")
    finals = read_back(spec, work, samples)
    total_steps = args.warmup + 2 * args.steps

    bpe = bytes_per_element(spec)
    bytes_per_launch = bpe * elements
    achieved = bytes_per_launch / (kernel_ms / 1e3) / 1e9
    # The committed counters were measured with the workload's own formats.
    traffic, traffic_source = (None, None) if args.state_format else load_traffic(args.workload)
    dtype = "f32"
    result = {
        "metric": {
            "adamw": "AdamW-SR step: params updated/sec and achieved HBM GB/s (% of peak), 1 MI355X",
            "sgdm": "SGDM-SR step: params updated/sec and achieved HBM GB/s (% of peak), 1 MI355X",
            "copy": "device copy (counter calibration): elements/sec, 1 MI355X",
            "cast": "SR cast FP32->{}: elements/sec and achieved HBM GB/s, 1 MI355X".format(
                {torch.bfloat16: "BF16", torch.float16: "FP16", torch.float8_e4m3fn: "E4M3",
                 torch.float8_e5m2: "E5M2"}.get(spec["formats"][0][0] if spec["formats"] else None, "")),
        }[spec["optimizer"]],
        "value": elements / (ms_per_step / 1e3),
        "unit": "params/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": "synthetic (seeded normal draws on the GPU)",
        "config": {
            "workload": args.workload,
            "optimizer": spec["optimizer"],
            "elements": elements,
            "tensors": len(spec["shapes"]),
            "param_dtype": str(spec["p_dtype"]).replace("torch.", ""),
            "grad_dtype": str(spec["g_dtype"]).replace("torch.", ""),
            "state_formats": [f"{str(d).replace('torch.', '')}/{r}" for d, r in spec["formats"]],
            "bytes_per_element": bpe,
            "resident_cap": os.environ.get("SR_STATES_RESIDENT_CAP") or "rule",
            "state_allocation": None if work.optimizer is None else (
                "separate" if args.separate_states else "shared"),
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBPS,
            "traffic": traffic,
            "traffic_source": traffic_source,
            "kernel_ms": kernel_ms,
            "step_ms_median": step_ms[len(step_ms) // 2],
            "step_ms_min": step_ms[0],
            "step_ms_max": step_ms[-1],
            "algorithmic_bytes_per_launch": bytes_per_launch,
        },
        "host_ms_submit": statistics.median(submit_ms),
        "host_ms_wall": statistics.median(wall_ms),
        "torch_fused": None,
        "torch_cast": None,
        "cpu_baseline": None,
        "validation": None,
    }
    if not args.no_torch_baseline:
        baseline = torch_fused_baseline(spec, work, args.steps, args.warmup)
        if baseline is not None and "ms_per_step" in baseline:
            baseline["speedup"] = baseline["ms_per_step"] / ms_per_step
        result["torch_fused"] = baseline
        cast_baseline = torch_cast_baseline(spec, work, args.steps, args.warmup)
        if cast_baseline is not None and "ms_per_step" in cast_baseline:
            cast_baseline["speedup"] = cast_baseline["ms_per_step"] / ms_per_step
        result["torch_cast"] = cast_baseline
    del work, step
    torch.cuda.empty_cache()
    if not args.no_ceiling:
        # Timed like the fused steps: back-to-back launches between two events.
        ceiling = pattern_ceiling(spec, elements, reps=max(5, min(2000, int(300 / kernel_ms))))
        if ceiling is not None:
            ceiling["frac"] = achieved / ceiling["achieved"]
        result["roofline"]["pattern_ceiling"] = ceiling
    if not args.no_cpu_baseline and spec["optimizer"] != "copy":
        result["cpu_baseline"] = cpu_baseline(spec, args.cpu_seconds)
        result["validation"] = validate(spec, samples, finals, total_steps)
    print(json.dumps(result), flush=True)
    if result["validation"] and result["validation"]["mismatches"]:
        raise SystemExit(f"validation failed: {result['validation']}")


if __name__ == "__main__":
    main()
