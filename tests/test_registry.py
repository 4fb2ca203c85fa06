"""Registry / constraint behaviour (host logic; no GPU).  Modelled on the reference's
tests/test_backends.py and tests/test_constraints.py, run against a private registry
with stub backends so nothing here touches a device."""
import types

import pytest
import torch

import comfy_kitchen as ck
from comfy_kitchen.constraints import (DivisibleBy, ExactDims, FunctionConstraints, MinDims, ParamConstraint,
                                       validate_function_call)
from comfy_kitchen.exceptions import BackendNotFoundError, BackendNotImplementedError, NoCapableBackendError
from comfy_kitchen.registry import BackendRegistry


def _stub(name):
    return types.SimpleNamespace(op=lambda **kw: name, other=lambda **kw: name)


@pytest.fixture
def reg():
    r = BackendRegistry()
    cpu = FunctionConstraints(params={"x": ParamConstraint(dtypes=frozenset({torch.float32}))},
                              default_devices=frozenset({"cpu"}))
    r.register("a", _stub("a"), {"op": cpu})
    r.register("b", _stub("b"), {"op": FunctionConstraints(default_devices=frozenset({"cpu"})),
                                 "other": FunctionConstraints()})
    r.set_priority(["a", "b"])
    return r


def test_priority_and_constraints(reg):
    assert reg.get_implementation("op", kwargs={"x": torch.zeros(2)})() == "a"
    # dtype constraint of "a" fails -> falls through to "b"
    assert reg.get_implementation("op", kwargs={"x": torch.zeros(2, dtype=torch.float16)})() == "b"
    reg.set_priority(["b", "a"])
    assert reg.get_implementation("op", kwargs={"x": torch.zeros(2)})() == "b"


def test_disable_enable(reg):
    reg.disable("a")
    assert reg.get_implementation("op", kwargs={"x": torch.zeros(2)})() == "b"
    with pytest.raises(BackendNotFoundError):
        reg.get_implementation("op", backend="a")
    reg.enable("a")
    assert reg.get_implementation("op", backend="a")() == "a"


def test_use_backend_is_nestable_and_thread_local(reg):
    x = {"x": torch.zeros(2)}
    with reg.use_backend("b"):
        assert reg.get_implementation("op", kwargs=x)() == "b"
        with reg.use_backend("a"):
            assert reg.get_implementation("op", kwargs=x)() == "a"
        assert reg.get_implementation("op", kwargs=x)() == "b"
    assert reg.get_implementation("op", kwargs=x)() == "a"
    with pytest.raises(BackendNotFoundError):
        with reg.use_backend("nope"):
            pass


def test_errors(reg):
    with pytest.raises(BackendNotImplementedError):
        reg.get_implementation("other", backend="a")
    with pytest.raises(NoCapableBackendError) as ei:
        reg.get_implementation("missing", kwargs={"x": torch.zeros(1)})
    assert ei.value.failures == {}
    reg.mark_unavailable("c", "library not built")
    reg.set_priority(["c"])
    with pytest.raises(NoCapableBackendError) as ei:
        reg.get_implementation("op", kwargs={"x": torch.zeros(1)})
    assert "library not built" in str(ei.value)
    st = reg.list_backends()
    assert st["c"]["available"] is False and st["c"]["unavailable_reason"] == "library not built"
    assert st["a"]["capabilities"] == ["op"]


def test_shape_rules_and_arch_gate():
    c = FunctionConstraints(params={"x": ParamConstraint(shape_rules=(ExactDims(2), DivisibleBy(1, 32)))},
                            default_devices=frozenset({"*"}), required_arch=("gfx950",))
    x = torch.zeros(4, 64)
    assert validate_function_call(c, {"x": x}, arch="gfx950:sramecc+:xnack-").success
    r = validate_function_call(c, {"x": x}, arch="gfx942")
    assert not r.success and r.failed_param == "__hardware__"
    r = validate_function_call(c, {"x": torch.zeros(4, 48)}, arch="gfx950")
    assert not r.success and "divisible by 32" in r.failure_reason
    assert MinDims(3).check(torch.zeros(1, 1, 1)) and not MinDims(3).check(x)


def test_public_api_surface():
    for name in ["quantize_per_tensor_fp8", "dequantize_per_tensor_fp8", "quantize_nvfp4", "dequantize_nvfp4",
                 "quantize_mxfp8", "dequantize_mxfp8", "scaled_mm_nvfp4", "scaled_mm_mxfp8", "apply_rope",
                 "apply_rope1", "swap_nibbles", "to_blocked", "from_blocked", "list_backends",
                 "set_backend_priority", "enable_backend", "disable_backend", "use_backend"]:
        assert callable(getattr(ck, name)), name
    for op in ["quantize_fp8", "dequantize_fp8", "quantize_nvfp4", "dequantize_nvfp4", "scaled_mm_nvfp4",
               "quantize_mxfp8", "dequantize_mxfp8", "scaled_mm_mxfp8", "apply_rope", "apply_rope1"]:
        assert hasattr(torch.ops.comfy_kitchen, op), op


def test_no_cpu_fallback():
    """The product path never computes on the CPU: a CPU tensor is refused loudly."""
    with pytest.raises(NoCapableBackendError):
        ck.quantize_per_tensor_fp8(torch.zeros(4, 4, dtype=torch.bfloat16), torch.ones(1))
    with pytest.raises(NoCapableBackendError):
        ck.apply_rope1(torch.zeros(1, 1, 4, 8, dtype=torch.bfloat16), torch.zeros(1, 1, 4, 4, 2, 2))


def test_fake_shapes_under_meta():
    """register_fake output shapes (what torch.compile sees)."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        x = torch.empty(100, 100, dtype=torch.bfloat16)
        q, s = torch.ops.comfy_kitchen.quantize_mxfp8(x, True)
        assert q.shape == (128, 128) and s.shape == (128, 4) and s.dtype == torch.float8_e8m0fnu
        q, s = torch.ops.comfy_kitchen.quantize_nvfp4(x, torch.empty(1), 0.0, True, True)
        assert q.shape == (112, 56) and s.shape == (128, 8) and s.dtype == torch.float8_e4m3fn
        y = torch.ops.comfy_kitchen.scaled_mm_mxfp8(torch.empty(8, 64, dtype=torch.float8_e4m3fn),
                                                    torch.empty(16, 64, dtype=torch.float8_e4m3fn),
                                                    torch.empty(128, 4, dtype=torch.float8_e8m0fnu),
                                                    torch.empty(128, 4, dtype=torch.float8_e8m0fnu), None, 2)
        assert y.shape == (8, 16) and y.dtype == torch.bfloat16
