"""Host-side API contract (CPU): formats, rounding registry, validation, checkpoints.

Mirrors tests/test_state_formats.py, tests/test_rounding_registry.py,
tests/test_state_optimizers.py:13-45,110-127, tests/test_triton_api.py and
tests/test_rng_streams.py:180-215 of the reference.  Nothing here launches a
kernel.
"""

from __future__ import annotations

import copy
import io
from pathlib import Path

import pytest
import torch

import sr_states
import sr_states.rounding as rounding_module
from sr_states import (
    AdamWHip,
    AdamWHipRN,
    AdamWReferenceRN,
    AdamWReferenceSR,
    SGDMHip,
    SGDMHipRN,
    SGDMReferenceRN,
    SGDMReferenceSR,
    StateFormat,
    cast,
    register_rounding,
)
from sr_states.rounding import validate_rounding

CLASSES = [AdamWHip, SGDMHip]
# The fused optimizers and the per-parameter ones share the host contract.
ALL_CLASSES = [AdamWHip, SGDMHip, AdamWReferenceSR, SGDMReferenceSR]
GOLDEN = Path(__file__).parent / "golden" / "reference_trajectories.pt"


@pytest.fixture(autouse=True)
def isolated_registry(monkeypatch):
    monkeypatch.setattr(rounding_module, "_ROUTINES", rounding_module._ROUTINES.copy())


def bits(x):
    return x.contiguous().view(torch.uint8)


def toward_zero(x, *, dtype, seed, offset):
    return (x.contiguous().view(torch.int32) & -65536).view(torch.float32).to(dtype)


# -- formats ------------------------------------------------------------------
def test_state_format_serialization_and_backends():
    fmt = StateFormat(torch.bfloat16, "nearest")
    assert StateFormat.from_dict(fmt.to_dict()) == fmt
    fmt.validate("reference")
    fmt.validate("hip")
    with pytest.raises(ValueError, match="backend"):
        fmt.validate("missing")
    for invalid in ({"dtype": torch.bfloat16}, {"dtype": torch.bfloat16, "rounding": "nearest", "extra": 1}):
        with pytest.raises(ValueError):
            StateFormat.from_dict(invalid)
    assert StateFormat(torch.float8_e4m3fn).to_dict() == {"dtype": torch.float8_e4m3fn, "rounding": "stochastic"}


@pytest.mark.parametrize("cls", ALL_CLASSES)
def test_format_validation_and_group_overrides(cls):
    """tests/test_state_formats.py:103-134."""
    p, q = [torch.nn.Parameter(torch.ones(3)) for _ in range(2)]
    fmt = StateFormat(torch.float32, "nearest")
    for extra in ({"state_dtype": torch.float32}, {"rounding": "nearest"}):
        with pytest.raises(ValueError, match="combined"):
            cls([p], lr=0.1, state_format=fmt, **extra)
    with pytest.raises(TypeError, match="StateFormat"):
        cls([{"params": [p], "state_format": (fmt,) * len(cls._state_names)}], lr=0.1)
    with pytest.raises(ValueError, match="keys"):
        cls([p], lr=0.1, state_format={"bad": fmt})
    opt = cls([{"params": [p], "state_format": fmt}], lr=0.1)
    assert all(f["dtype"] == torch.float32 for f in opt.param_groups[0]["state_format"].values())
    opt.add_param_group({"params": [q], "rounding": "nearest"})
    assert all(f == StateFormat(torch.bfloat16, "nearest").to_dict()
               for f in opt.param_groups[1]["state_format"].values())
    with pytest.raises(ValueError, match="registered"):
        opt.add_param_group({"params": [torch.nn.Parameter(torch.ones(1))],
                             "state_format": StateFormat(torch.bfloat16, "missing")})
    assert len(opt.param_groups) == 2
    with pytest.raises(ValueError):
        opt.add_param_group({"params": [torch.nn.Parameter(torch.ones(1))], "lr": -1})
    assert len(opt.param_groups) == 2


def test_shorthand_single_and_dict_formats_serialize_identically():
    fmt = StateFormat(torch.float8_e5m2, "nearest")
    p = torch.nn.Parameter(torch.ones(2))
    variants = [{"state_dtype": fmt.dtype, "rounding": fmt.rounding}, {"state_format": fmt},
                {"state_format": dict.fromkeys(AdamWHip._state_names, fmt)}]
    groups = [AdamWHip([p], **v).param_groups[0]["state_format"] for v in variants]
    assert groups[0] == groups[1] == groups[2]


@pytest.mark.parametrize("rn,sr", [(AdamWHipRN, AdamWHip), (SGDMHipRN, SGDMHip),
                                   (AdamWReferenceRN, AdamWReferenceSR), (SGDMReferenceRN, SGDMReferenceSR)])
def test_rn_classes_force_nearest(rn, sr):
    """tests/test_state_formats.py:258-293 (host part)."""
    dtypes = (torch.float8_e4m3fn, torch.float8_e5m2)
    per_state = {n: StateFormat(d) for n, d in zip(rn._state_names, dtypes)}
    nearest = {n: StateFormat(d, "nearest") for n, d in zip(rn._state_names, dtypes)}
    opt = rn([torch.nn.Parameter(torch.ones(3))], lr=0.01, state_format=per_state, seed=5)
    expected = sr([torch.nn.Parameter(torch.ones(3))], lr=0.01, state_format=nearest, seed=5)
    assert opt.param_groups[0]["state_format"] == expected.param_groups[0]["state_format"]
    for override in ({"state_format": StateFormat(torch.bfloat16)}, {"rounding": "stochastic"}):
        opt.add_param_group({"params": [torch.nn.Parameter(torch.ones(2))], **override})
        assert all(f["rounding"] == "nearest" for f in opt.param_groups[-1]["state_format"].values())
    with pytest.raises(ValueError, match="combined"):
        rn([torch.nn.Parameter(torch.ones(1))], lr=0.01, state_format=per_state, rounding="nearest")


# -- registry ------------------------------------------------------------------
def test_registration_validation_and_builtins():
    """tests/test_rounding_registry.py:113-128."""
    with pytest.raises(ValueError, match="already registered"):
        register_rounding("nearest", torch.bfloat16, reference=toward_zero)
    with pytest.raises(ValueError, match="nonempty"):
        register_rounding("", torch.bfloat16, reference=toward_zero)
    with pytest.raises(ValueError, match="floating-point"):
        register_rounding("rule", torch.int32, reference=toward_zero)
    with pytest.raises(TypeError, match="callable"):
        register_rounding("rule", torch.bfloat16, reference=None)
    for dtype in (torch.float32, torch.bfloat16, torch.float16, torch.float8_e4m3fn, torch.float8_e5m2):
        for mode in ("nearest", "stochastic"):
            validate_rounding(dtype, mode, backend="hip")
            with pytest.raises(ValueError, match="already registered"):
                register_rounding(mode, dtype, reference=toward_zero)
    with pytest.raises(ValueError, match="backend"):
        validate_rounding(torch.bfloat16, "nearest", backend="unknown")


def test_registrations_with_a_triton_callback_run_unchanged():
    """tests/test_triton_rounding_extensions.py:32-43: ``triton=`` is accepted, checked and unused.

    The rule then behaves as any registered rule without a HIP implementation:
    the fused optimizers refuse it by name, the per-parameter ones and
    ``cast`` take it (the GPU tests run them).
    """

    def callback(value, counter, dtype):
        raise AssertionError("the Triton callback is never called")

    with pytest.raises(TypeError, match="callable"):
        register_rounding("toward_zero", torch.bfloat16, reference=toward_zero, triton=5)
    register_rounding("toward_zero", torch.bfloat16, reference=toward_zero, triton=callback)
    register_rounding("custom_nearest", torch.float16, reference=lambda x, **kw: x.to(kw["dtype"]),
                      triton=callback)
    validate_rounding(torch.bfloat16, "toward_zero")
    with pytest.raises(ValueError, match="no HIP implementation"):
        validate_rounding(torch.bfloat16, "toward_zero", backend="hip")
    p = torch.nn.Parameter(torch.ones(4))
    with pytest.raises(ValueError, match="no HIP implementation"):
        AdamWHip([p], lr=0.01, rounding="toward_zero")
    with pytest.raises(ValueError, match="no HIP implementation"):
        SGDMHip([p], lr=0.01, state_dtype=torch.float16, rounding="custom_nearest")
    for cls in (AdamWReferenceSR, SGDMReferenceSR):
        cls([p], lr=0.01, rounding="toward_zero")


def test_custom_rule_cast_contract():
    """tests/test_rounding_registry.py:131-139: custom routines run as registered."""
    register_rounding("toward_zero", torch.bfloat16, reference=toward_zero)
    x = torch.tensor([1.003, -1.006, 0.0])
    assert torch.equal(cast(x, dtype=torch.bfloat16, rounding="toward_zero"), toward_zero(x, dtype=torch.bfloat16, seed=0, offset=0))
    register_rounding("bad_dtype", torch.bfloat16, reference=lambda x, **kw: x)
    register_rounding("bad_shape", torch.bfloat16, reference=lambda x, **kw: x[:1].bfloat16())
    register_rounding("not_tensor", torch.bfloat16, reference=lambda x, **kw: None)
    for name in ("bad_dtype", "bad_shape"):
        with pytest.raises(ValueError, match="requested dtype"):
            cast(torch.ones(2), dtype=torch.bfloat16, rounding=name)
    with pytest.raises(TypeError, match="return a tensor"):
        cast(torch.ones(2), dtype=torch.bfloat16, rounding="not_tensor")
    with pytest.raises(TypeError, match="float32"):
        cast(torch.ones(2, dtype=torch.float64), dtype=torch.bfloat16)


def test_builtin_casts_never_run_on_the_cpu():
    """The built-in rules are the HIP kernels: a CPU tensor is an error, not a fallback."""
    x = torch.ones(4)
    assert cast(x, dtype=torch.float32) is x  # FP32 built-ins are the identity
    for dtype in (torch.bfloat16, torch.float16, torch.float8_e4m3fn):
        with pytest.raises(ValueError, match="GPU"):
            cast(x, dtype=dtype, rounding="stochastic")
    with pytest.raises(ValueError, match="GPU"):
        sr_states.sr_cast_bf16(x, seed=1)


def test_cast_output_must_not_overlap_the_input():
    """The cast's native entry refuses an output sharing any byte with the input.

    Its output checks come before its device check, so CPU tensors show them
    without a GPU: an acceptable output gets as far as the GPU requirement.
    """
    from sr_states import _lib

    launcher = _lib.launcher()
    code = _lib.DTYPE_CODES

    def error(x, out):
        with pytest.raises(ValueError) as caught:
            launcher.cast(x, out, code[out.dtype], _lib.SR_STOCHASTIC, 7, 0, 256, 0)
        return str(caught.value)

    storage = torch.zeros(64)
    x = storage[:16]
    assert "GPU" in error(x, torch.empty(16, dtype=torch.bfloat16))  # disjoint
    assert "GPU" in error(x, storage[16:24].view(torch.bfloat16))  # adjacent
    for out in (storage[:8].view(torch.bfloat16), storage[15:23].view(torch.bfloat16),
                storage[10:14].view(torch.float8_e4m3fn)):
        assert "overlap" in error(x, out)
    assert "GPU" in error(storage[:0], storage[:0].view(torch.bfloat16))  # empty: nothing shared
    with pytest.raises(ValueError, match="contiguous tensor of the requested dtype"):
        launcher.cast(x, torch.empty(16, dtype=torch.float16), code[torch.bfloat16], 1, 7, 0, 256, 0)
    with pytest.raises(ValueError, match="contiguous tensor of the requested dtype"):
        launcher.cast(x, torch.empty(15, dtype=torch.bfloat16), code[torch.bfloat16], 1, 7, 0, 256, 0)
    with pytest.raises(ValueError, match="contiguous tensor of the requested dtype"):
        launcher.cast(x, torch.empty(32, dtype=torch.bfloat16)[::2], code[torch.bfloat16], 1, 7, 0, 256, 0)
    with pytest.raises(TypeError, match="tensors"):
        launcher.cast(x, [0.0] * 16, code[torch.bfloat16], 1, 7, 0, 256, 0)


def test_update_entries_check_their_tensors_before_the_device():
    """The functional updates' native entries: argument and state-format checks, then the GPU one."""
    from sr_states import _lib
    from sr_states.optim.adamw import adamw_scalars
    from sr_states.optim.sgd import sgdm_scalars

    launcher = _lib.launcher()
    bf16, e4m3 = _lib.DTYPE_CODES[torch.bfloat16], _lib.DTYPE_CODES[torch.float8_e4m3fn]
    sr = _lib.SR_STOCHASTIC
    p, g = torch.zeros(8), torch.zeros(8)
    m, v = torch.zeros(8, dtype=torch.bfloat16), torch.zeros(8, dtype=torch.bfloat16)
    scalars = adamw_scalars(1e-3, 0.9, 0.999, 1e-8, 0.01, 1)
    assert len(scalars) == 8 and len(sgdm_scalars(1e-3, 0.9)) == 2

    def adamw(*tensors, m_code=bf16):
        return launcher.adamw_step(*tensors, m_code, sr, bf16, sr, scalars, 7, 0, 256, 0)

    with pytest.raises(ValueError, match="require GPU tensors"):
        adamw(p, g, m, v)
    with pytest.raises(ValueError, match="state dtype does not match its state format"):
        adamw(p, g, m, v, m_code=e4m3)
    with pytest.raises(TypeError, match="must be tensors"):
        adamw(p, g, m, [0.0] * 8)
    with pytest.raises(TypeError):
        launcher.adamw_step(p, g, m, v, bf16, sr, bf16, sr, scalars[:7], 7, 0, 256, 0)
    with pytest.raises(ValueError, match="require GPU tensors"):
        launcher.sgdm_step(p, g, m, bf16, sr, sgdm_scalars(1e-3, 0.9), 7, 0, 256, 0)
    with pytest.raises(ValueError, match="state dtype does not match its state format"):
        launcher.sgdm_step(p, g, m, e4m3, sr, sgdm_scalars(1e-3, 0.9), 7, 0, 256, 0)
    with pytest.raises(ValueError, match="require GPU tensors"):
        sr_states.hip_adamw_step_(p, g, m, v, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.0,
                                  step=1, seed=7)
    with pytest.raises(ValueError, match="require GPU tensors"):
        sr_states.hip_sgdm_step_(p, g, m, lr=1e-3, momentum_factor=0.9, seed=7)


def test_native_entries_refuse_tensors_without_memory():
    """A wrapper subclass on the GPU device holds no memory: refused, never launched.

    Building one needs no GPU, so the refusal shows on the CPU.
    """
    from sr_states import _lib

    class Storageless(torch.Tensor):
        @staticmethod
        def __new__(cls, size, dtype):
            return torch.Tensor._make_wrapper_subclass(cls, size, dtype=dtype, device="cuda")

        @classmethod
        def __torch_dispatch__(cls, func, types, args=(), kwargs=None):
            raise NotImplementedError(func)

    launcher = _lib.launcher()
    bf16, sr = _lib.DTYPE_CODES[torch.bfloat16], _lib.SR_STOCHASTIC
    x, out = Storageless((16,), torch.float32), Storageless((16,), torch.bfloat16)
    with pytest.raises(ValueError, match="without device memory"):
        launcher.cast(x, out, bf16, sr, 0, 0, 256, 0)
    p, g = Storageless((16,), torch.float32), Storageless((16,), torch.float32)
    m, v = Storageless((16,), torch.bfloat16), Storageless((16,), torch.bfloat16)
    with pytest.raises(ValueError, match="hold device memory"):
        launcher.adamw_step(p, g, m, v, bf16, sr, bf16, sr, (0.0,) * 8, 0, 0, 256, 0)
    with pytest.raises(ValueError, match="hold device memory"):
        launcher.sgdm_step(p, g, m, bf16, sr, (0.0, 0.0), 0, 0, 256, 0)


@pytest.mark.parametrize("arch", ["gfx950:sramecc+:xnack-", "gfx950", "gfx942:sramecc+:xnack-", "gfx90a", "gfx1100"])
def test_device_check_accepts_only_the_built_architecture(monkeypatch, arch):
    """tests/test_fp8_storage.py:88-108, with the gfx950 check in place of sm_89.

    The library holds gfx950 code only, so every dtype (FP8 included) runs on
    gfx950 and nothing runs elsewhere; the architecture is queried once per
    device and CPU tensors are refused before any query.
    """
    from sr_states.hip import _common

    _common._device_arch.cache_clear()
    seen = []

    class Properties:
        gcnArchName = arch

    def properties(device):
        seen.append(torch.device(device))
        return Properties()

    monkeypatch.setattr(torch.cuda, "get_device_properties", properties)
    try:
        for _ in range(2):
            if arch.split(":")[0] == "gfx950":
                _common.validate_update_device(torch.device("cuda", 0), torch.float8_e4m3fn, torch.float8_e5m2)
                _common.validate_device("cuda:0")
            else:
                with pytest.raises(ValueError, match=f"built for gfx950, not {arch.split(':')[0]}"):
                    _common.validate_update_device(torch.device("cuda", 0), torch.float8_e4m3fn)
        with pytest.raises(ValueError, match="GPU tensors"):
            _common.validate_device(torch.device("cpu"))
        assert seen == [torch.device("cuda", 0)]
    finally:
        _common._device_arch.cache_clear()


@pytest.mark.parametrize("cls", CLASSES)
def test_hip_optimizers_reject_reference_only_rules(cls):
    """tests/test_rounding_registry.py:86-90."""
    register_rounding("toward_zero", torch.bfloat16, reference=toward_zero)
    with pytest.raises(ValueError, match="no HIP implementation"):
        cls([torch.nn.Parameter(torch.ones(1))], lr=0.1, rounding="toward_zero")


@pytest.mark.parametrize("cls", ALL_CLASSES)
def test_group_overrides_and_checkpoints_require_registration(cls):
    """tests/test_rounding_registry.py:93-110."""
    p = torch.nn.Parameter(torch.ones(1))
    with pytest.raises(ValueError, match="rounding"):
        cls([{"params": [p], "rounding": "missing"}], lr=0.1)
    optimizer = cls([p], lr=0.1)
    with pytest.raises(ValueError, match="rounding"):
        optimizer.add_param_group({"params": [torch.nn.Parameter(torch.ones(1))], "rounding": "missing"})
    checkpoint = copy.deepcopy(optimizer.state_dict())
    checkpoint["param_groups"][0]["state_format"][cls._state_names[0]]["rounding"] = "missing"
    with pytest.raises(ValueError, match="rounding"):
        optimizer.load_state_dict(checkpoint)
    assert optimizer.param_groups[0]["state_format"][cls._state_names[0]]["rounding"] == "stochastic"


# -- hyperparameter validation ----------------------------------------------------
@pytest.mark.parametrize(
    "kwargs",
    [{"lr": -1}, {"lr": float("nan")}, {"eps": -1}, {"eps": float("inf")}, {"betas": (0.9, 1)},
     {"betas": (float("nan"), 0.9)}, {"weight_decay": -1}, {"state_dtype": torch.int32},
     {"rounding": "invalid"}, {"block_size": 64}],
)
def test_adamw_rejects_invalid_options(kwargs):
    """tests/test_state_optimizers.py:110-127."""
    with pytest.raises(ValueError):
        AdamWHip([torch.nn.Parameter(torch.ones(1))], **kwargs)


@pytest.mark.parametrize(
    ("kwargs", "message"),
    [({"lr": -0.1}, "learning rate"), ({"lr": 0.1, "momentum": 1.0}, "momentum value"),
     ({"lr": 0.1, "rounding": "invalid"}, "rounding"), ({"lr": 0.1, "block_size": 64}, "block_size")],
)
def test_sgdm_rejects_invalid_options(kwargs, message):
    """tests/test_triton_api.py:23-35."""
    with pytest.raises(ValueError, match=message):
        SGDMHip([torch.nn.Parameter(torch.ones(4))], **kwargs)


# -- checkpoints -------------------------------------------------------------------
@pytest.mark.parametrize("cls", ALL_CLASSES)
@pytest.mark.parametrize("state_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("parameter_dtype", [torch.float32, torch.bfloat16])
def test_checkpoint_keeps_state_precision(cls, state_dtype, parameter_dtype):
    """tests/test_state_optimizers.py:13-44."""
    p = torch.nn.Parameter(torch.ones(4, dtype=parameter_dtype))
    optimizer = cls([p], lr=0.01, state_dtype=state_dtype, seed=42)
    original = torch.tensor([0.0, -0.0, 1.003125, 0.503125], dtype=state_dtype)
    for name in optimizer._state_names:
        optimizer.state[p][name] = original.clone()
    if "exp_avg" in optimizer._state_names:
        optimizer.state[p]["step"] = 7
    optimizer.param_groups[0]["sr_step"] = 2**32 + 31
    checkpoint = copy.deepcopy(optimizer.state_dict())
    q = torch.nn.Parameter(p.detach().clone())
    restored = cls([q], lr=0.3, state_dtype=torch.float32, seed=99)
    seen = []
    restored.register_load_state_dict_post_hook(lambda opt: seen.append(opt.state[q][opt._state_names[0]].dtype))
    restored.load_state_dict(checkpoint)
    assert seen == [state_dtype]
    for name in optimizer._state_names:
        actual = restored.state[q][name]
        assert actual.dtype == state_dtype
        assert torch.equal(bits(actual), bits(original))
        assert actual.data_ptr() != checkpoint["state"][0][name].data_ptr()
    assert restored.param_groups[0]["sr_step"] == 2**32 + 31
    assert restored.param_groups[0]["sr_seed"] == 42
    if "exp_avg" in optimizer._state_names:
        assert restored.state[q]["step"] == 7


def test_checkpoint_before_first_step_keeps_state_lazy():
    """tests/test_triton_api.py:68-72."""
    parameter = torch.nn.Parameter(torch.ones(4))
    optimizer = SGDMHip([parameter], lr=0.1)
    optimizer.load_state_dict(copy.deepcopy(optimizer.state_dict()))
    assert not optimizer.state


def test_bf16_state_survives_checkpoint_with_groups():
    """tests/test_triton_api.py:38-65."""
    source = torch.nn.Parameter(torch.ones(4))
    unused = torch.nn.Parameter(torch.ones(4))
    optimizer = SGDMHip([{"params": [source]}, {"params": [unused]}], lr=0.1, seed=44)
    buffer = torch.tensor([0.0, -0.0, 1.0078125, -0.50390625], dtype=torch.bfloat16)
    optimizer.state[source]["momentum_buffer"] = buffer.clone()
    optimizer.param_groups[0]["sr_step"] = 2**32 + 17
    checkpoint = copy.deepcopy(optimizer.state_dict())
    target, target_unused = torch.nn.Parameter(torch.ones(4)), torch.nn.Parameter(torch.ones(4))
    resumed = SGDMHip([{"params": [target]}, {"params": [target_unused]}], lr=0.9, seed=999)
    resumed.load_state_dict(checkpoint)
    restored = resumed.state[target]["momentum_buffer"]
    assert restored.dtype == torch.bfloat16 and torch.equal(restored.view(torch.int16), buffer.view(torch.int16))
    assert target_unused not in resumed.state
    assert resumed.param_groups[0]["sr_step"] == 2**32 + 17
    assert resumed.param_groups[1]["sr_step"] == 0
    assert resumed.param_groups[0]["sr_seed"] == 44 and resumed.param_groups[0]["lr"] == 0.1


def test_legacy_group_keys_are_migrated():
    """tests/test_rng_streams.py:180-215 and tests/test_state_formats.py:168-175."""
    p = torch.nn.Parameter(torch.ones(9, dtype=torch.bfloat16))
    opt = AdamWHip([p], lr=0.01, seed=7)
    opt.state[p]["exp_avg"] = torch.ones(9, dtype=torch.bfloat16)
    opt.state[p]["exp_avg_sq"] = torch.ones(9, dtype=torch.bfloat16)
    opt.state[p]["step"] = 2
    checkpoint = copy.deepcopy(opt.state_dict())
    group = checkpoint["param_groups"][0]
    del group["sr_step"]
    group["sr_offset"] = 2**32 + 29
    resumed = AdamWHip([torch.nn.Parameter(p.detach().clone())], seed=3)
    resumed.load_state_dict(checkpoint)
    restored = resumed.param_groups[0]
    assert restored["sr_step"] == 0 and restored["sr_seed"] == 7 and "sr_offset" not in restored
    assert group["sr_offset"] == 2**32 + 29 and "sr_step" not in group  # caller's copy untouched
    old = copy.deepcopy(checkpoint)
    old["param_groups"][0].pop("state_format")
    old["param_groups"][0].update(state_dtype=torch.float32, rounding="nearest")
    resumed.load_state_dict(old)
    q = resumed.param_groups[0]["params"][0]
    assert all(resumed.state[q][n].dtype == torch.float32 for n in AdamWHip._state_names)
    assert "state_format" not in old["param_groups"][0]


@pytest.mark.parametrize("eager", [False, True], ids=["fused", "eager"])
@pytest.mark.parametrize("name", ["adamw_mixed", "adamw_minifloat", "sgdm_mixed"])
def test_reference_checkpoints_load_into_hip_optimizers(name, eager):
    """A state_dict written by the reference's eager optimizer loads unchanged, into either kind."""
    case = torch.load(GOLDEN, weights_only=True)["cases"][name]
    checkpoint = case["state_dict"]
    stream = io.BytesIO()
    torch.save(checkpoint, stream)
    stream.seek(0)
    checkpoint = torch.load(stream, weights_only=True)
    dtypes = {"torch.float32": torch.float32, "torch.bfloat16": torch.bfloat16}
    params = [torch.nn.Parameter(raw.view(dtypes[dt]).clone()) for raw, dt in zip(case["initial"], case["dtypes"])]
    groups, at = [], 0
    for group in case["groups"]:
        groups.append({"params": params[at: at + len(group["sizes"])]})
        at += len(group["sizes"])
    if eager:
        cls = AdamWReferenceSR if case["kind"] == "adamw" else SGDMReferenceSR
    else:
        cls = AdamWHip if case["kind"] == "adamw" else SGDMHip
    opt = cls(groups, lr=0.5, seed=1)
    opt.load_state_dict(checkpoint)
    for group, saved in zip(opt.param_groups, checkpoint["param_groups"]):
        assert group["sr_seed"] == saved["sr_seed"] and group["sr_step"] == saved["sr_step"]
        assert group["state_format"] == saved["state_format"]
        assert group["lr"] == saved["lr"]
    last = case["steps"][-1]["states"]
    for p, want in zip(params, last):
        for state_name, value in want.items():
            got = opt.state[p][state_name]
            if isinstance(value, torch.Tensor):
                assert torch.equal(bits(got), value)
            else:
                assert got == value


def test_overlap_rule_equals_the_pairwise_definition():
    """Written byte ranges may share no byte with any other range; read ranges may share."""
    import random

    from sr_states.hip._optimizer import validate_no_overlap

    def clashes(spans):
        return any(
            (w1 or w2) and s1 < e2 and s2 < e1
            for i, (s1, e1, w1) in enumerate(spans)
            for (s2, e2, w2) in spans[i + 1:]
        )

    rng = random.Random(7)
    for _ in range(5000):
        spans = []
        for _ in range(rng.randint(1, 7)):
            start = rng.randint(0, 40)
            spans.append((start, start + rng.randint(1, 12), rng.random() < 0.6))
        try:
            validate_no_overlap(spans)
            refused = False
        except ValueError as error:
            assert "must not overlap optimizer writes" in str(error)
            refused = True
        assert refused == clashes(spans), spans
