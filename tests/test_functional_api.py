"""The reference's eager and functional names, without a GPU.

The reference exports ``AdamWReferenceSR/RN`` and ``SGDMReferenceSR/RN`` at
the top level (sr_states/__init__.py:3-17) and the functional updates in
``sr_states.reference`` (reference/adamw.py:12-127, reference/sgd.py:12-84,
reference/rounding.py:1-14).  Here they run the HIP kernels, so on a CPU
tensor they raise before any work instead of computing.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import sr_states
import sr_states.reference as functional
from sr_states import StateFormat

ADAMW = {"lr": 1e-3, "beta1": 0.9, "beta2": 0.999, "eps": 1e-8, "weight_decay": 1e-2, "step": 1}


def test_reference_names_are_exported():
    for name in ("AdamWReferenceSR", "AdamWReferenceRN", "SGDMReferenceSR", "SGDMReferenceRN"):
        assert name in sr_states.__all__
        assert issubclass(getattr(sr_states, name), sr_states.StateOptimizer)
    from sr_states.optim.adamw import AdamWReferenceRN, AdamWReferenceSR
    from sr_states.optim.sgd import SGDMReferenceRN, SGDMReferenceSR
    from sr_states.reference.adamw import adamw_step, adamw_step_
    from sr_states.reference.rounding import stochastic_round_bf16
    from sr_states.reference.sgd import sgdm_step, sgdm_step_

    assert AdamWReferenceSR is sr_states.AdamWReferenceSR and AdamWReferenceRN is sr_states.AdamWReferenceRN
    assert SGDMReferenceSR is sr_states.SGDMReferenceSR and SGDMReferenceRN is sr_states.SGDMReferenceRN
    assert functional.adamw_step is adamw_step and functional.adamw_step_ is adamw_step_
    assert functional.sgdm_step is sgdm_step and functional.sgdm_step_ is sgdm_step_
    assert functional.stochastic_round_bf16 is stochastic_round_bf16
    assert functional.cast is sr_states.cast
    # The optimizers call the functional update through a replaceable hook, as the reference's do.
    assert sr_states.AdamWReferenceSR._update is adamw_step_.__wrapped__
    assert sr_states.SGDMReferenceSR._update is sgdm_step_.__wrapped__
    with pytest.raises(AttributeError):
        from sr_states.optim import adamw

        adamw.NotAnOptimizer  # noqa: B018


def test_defaults_and_group_layout_are_the_reference_ones():
    """Defaults of optim/adamw.py:28-37 and optim/sgd.py:26-33."""
    params = [torch.nn.Parameter(torch.zeros(3))]
    adamw = sr_states.AdamWReferenceSR(params)
    assert {k: adamw.defaults[k] for k in ("lr", "betas", "eps", "weight_decay")} == {
        "lr": 1e-3, "betas": (0.9, 0.999), "eps": 1e-8, "weight_decay": 1e-2}
    assert adamw.defaults["state_format"] == {
        name: {"dtype": torch.bfloat16, "rounding": "stochastic"} for name in ("exp_avg", "exp_avg_sq")}
    rn = sr_states.SGDMReferenceRN(params, lr=0.1, state_dtype=torch.float16)
    assert rn.defaults["momentum"] == 0.9
    assert rn.defaults["state_format"] == {"momentum_buffer": {"dtype": torch.float16, "rounding": "nearest"}}
    with pytest.raises(TypeError):
        sr_states.SGDMReferenceSR(params)  # lr is required
    with pytest.raises(ValueError, match="invalid beta values"):
        sr_states.AdamWReferenceSR(params, betas=(0.9, 1.0))
    with pytest.raises(ValueError, match="invalid momentum value"):
        sr_states.SGDMReferenceSR(params, lr=0.1, momentum=1.0)
    # The eager and fused optimizers share group keys apart from the fused block size.
    fused = sr_states.AdamWHip(params)
    assert set(fused.defaults) - set(adamw.defaults) == {"block_size"}


def test_eager_optimizers_accept_rules_without_a_hip_kernel():
    name = "sr_states_cpu_test_truncate"
    try:
        sr_states.register_rounding(name, torch.bfloat16, reference=lambda x, *, dtype, seed, offset: x.to(dtype))
    except ValueError:
        pass  # registered by an earlier run in this process
    fmt = StateFormat(torch.bfloat16, name)
    params = [torch.nn.Parameter(torch.zeros(3))]
    sr_states.AdamWReferenceSR(params, state_format=fmt)
    sr_states.SGDMReferenceSR(params, lr=0.1, state_format=fmt)
    with pytest.raises(ValueError, match="no HIP implementation"):
        sr_states.AdamWHip(params, state_format=fmt)


def _adamw_inputs(device="cpu", n=8):
    return [torch.zeros(n, device=device) for _ in range(2)] + [
        torch.zeros(n, dtype=torch.bfloat16, device=device) for _ in range(2)]


@pytest.mark.parametrize("update", ["adamw_step", "adamw_step_"])
def test_cpu_tensors_are_refused(update):
    tensors = _adamw_inputs()
    with pytest.raises(ValueError, match="run on the GPU"):
        getattr(functional, update)(*tensors, **ADAMW)
    assert all(not t.any() for t in tensors)


@pytest.mark.parametrize("update", ["sgdm_step", "sgdm_step_"])
def test_cpu_tensors_are_refused_by_sgdm(update):
    tensors = [torch.zeros(8), torch.ones(8), torch.zeros(8, dtype=torch.bfloat16)]
    with pytest.raises(ValueError, match="run on the GPU"):
        getattr(functional, update)(*tensors, lr=0.1, momentum_factor=0.9)


def test_stochastic_round_bf16_refuses_cpu_input():
    with pytest.raises(ValueError, match="on the GPU"):
        functional.stochastic_round_bf16(torch.zeros(4), seed=1)


def test_neighbor_helpers_keep_the_reference_names_and_errors():
    """reference/rounding.py:1-9 re-exports them; _bf16.py:24-26 and _minifloat.py:79-82 raise."""
    from sr_states.reference.rounding import bf16_neighbors, minifloat_neighbors

    assert functional.bf16_neighbors is bf16_neighbors
    assert functional.minifloat_neighbors is minifloat_neighbors
    assert {"bf16_neighbors", "cast", "minifloat_neighbors", "stochastic_round_bf16"} <= set(functional.__all__)
    with pytest.raises(TypeError, match="expected torch.float32 input, got torch.float64"):
        bf16_neighbors(torch.zeros(4, dtype=torch.float64))
    with pytest.raises(TypeError, match="expected torch.float32 input"):
        minifloat_neighbors(torch.zeros(4, dtype=torch.bfloat16), dtype=torch.float16)
    with pytest.raises(ValueError, match="neighbors supports E4M3, E5M2, and FP16"):
        minifloat_neighbors(torch.zeros(4), dtype=torch.bfloat16)
    for call in (lambda: bf16_neighbors(torch.zeros(4)),
                 lambda: minifloat_neighbors(torch.zeros(4), dtype=torch.float8_e5m2)):
        with pytest.raises(ValueError, match="on the GPU"):
            call()


def test_argument_errors_come_before_device_checks():
    tensors = _adamw_inputs()
    with pytest.raises(ValueError, match="step must be at least 1"):
        functional.adamw_step(*tensors, **{**ADAMW, "step": 0})
    with pytest.raises(TypeError, match="step must be a real number"):
        functional.adamw_step(*tensors, **{**ADAMW, "step": torch.tensor(3)})
    with pytest.raises(TypeError, match="step must be a real number"):
        functional.adamw_step(*tensors, **{**ADAMW, "step": "3"})
    with pytest.raises(ValueError, match="step must be at least 1"):
        functional.adamw_step(*tensors, **{**ADAMW, "step": np.int64(0)})
    # Steps the reference takes reach the device check (no CPU path here).
    for step in (np.int64(3), 2.5, np.float32(7.0), True):
        with pytest.raises(ValueError, match="on the GPU"):
            functional.adamw_step(*tensors, **{**ADAMW, "step": step})
    with pytest.raises(TypeError, match="expected real tensors"):
        functional.adamw_step(tensors[0].to(torch.complex64), *tensors[1:], **ADAMW)
    with pytest.raises(ValueError, match="cannot be combined"):
        functional.adamw_step(*tensors, formats=StateFormat(torch.bfloat16), state_dtype=torch.float16, **ADAMW)
    with pytest.raises(ValueError, match="no rounding"):
        functional.sgdm_step(*tensors[:3], lr=0.1, momentum_factor=0.9, rounding="sideways")
    with pytest.raises(TypeError, match="must be tensors"):
        functional.sgdm_step(tensors[0], [0.0] * 8, tensors[2], lr=0.1, momentum_factor=0.9)
