"""Checkpoint format of the QuantizedTensor layouts (state-dict keys and bytes).

The reference serialises a quantized weight as key suffixes "" (codes), "_scale" and, for
NVFP4, "_scale_2" (`tensor/fp8.py:74-80`, `tensor/mxfp8.py:86-87`, `tensor/nvfp4.py:94-101`),
and its NVFP4 sample loader rebuilds the layer from "weight", "weight_scale",
"weight_scale_2" and an optional "input_scale" (`samples/nvfp4_linear.py:39-68`).  These
tests write the layouts' state dicts to a safetensors file, load it back with the safe
loader, rebuild the tensors the way that loader does, and check every byte survives.

tests/golden/checkpoints.safetensors (made by tests/golden/make_checkpoints.py with the CPU
oracle) holds one layer per layout in that key convention plus the oracle's outputs; the
GPU tests load it as the reference's loaders do and compare F.linear with the oracle, and
re-quantize its source weight on the GPU and compare the bytes.
"""
import pytest
import torch
from safetensors.torch import load_file, save_file

from comfy_kitchen.tensor import (QuantizedTensor, TensorCoreFP8Layout, TensorCoreMXFP8Layout,
                                  TensorCoreNVFP4Layout)
from oracle import eager_ref as ref


def _bits(t: torch.Tensor) -> torch.Tensor:
    return t.contiguous().view(torch.uint8) if t.element_size() == 1 else t.contiguous()


def _same(a: torch.Tensor, b: torch.Tensor) -> bool:
    return a.dtype == b.dtype and a.shape == b.shape and torch.equal(_bits(a), _bits(b))


def _weights(seed: int, n: int = 96, k: int = 160) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(n, k, generator=g) * 0.05).bfloat16()


def _fp8(w):
    scale = (w.abs().amax() / 448).float().reshape(())
    q = ref.quantize_per_tensor_fp8(w, scale.reshape(1))
    return QuantizedTensor(q, "TensorCoreFP8Layout",
                           TensorCoreFP8Layout.Params(scale=scale, orig_dtype=w.dtype, orig_shape=tuple(w.shape)))


def _mxfp8(w):
    q, s = ref.quantize_mxfp8(w, pad_32x=True)
    return QuantizedTensor(q, "TensorCoreMXFP8Layout",
                           TensorCoreMXFP8Layout.Params(scale=s, orig_dtype=w.dtype, orig_shape=tuple(w.shape)))


def _nvfp4(w):
    g = (w.abs().amax() / 2688).float().reshape(1)
    q, s = ref.quantize_nvfp4(w, g, pad_16x=True)
    return QuantizedTensor(q, "TensorCoreNVFP4Layout",
                           TensorCoreNVFP4Layout.Params(scale=g, orig_dtype=w.dtype, orig_shape=tuple(w.shape),
                                                        block_scale=s))


@pytest.mark.parametrize("make,keys", [
    (_fp8, {"weight", "weight_scale"}),
    (_mxfp8, {"weight", "weight_scale"}),
    (_nvfp4, {"weight", "weight_scale", "weight_scale_2"}),
], ids=["fp8", "mxfp8", "nvfp4"])
def test_state_dict_round_trip_through_safetensors(make, keys, tmp_path):
    qt = make(_weights(3))
    sd = qt.state_dict("weight")
    assert set(sd) == keys
    path = tmp_path / "layer.safetensors"
    save_file({k: v.contiguous() for k, v in sd.items()}, str(path))
    back = load_file(str(path))
    assert set(back) == keys
    for k in keys:
        assert _same(back[k], sd[k]), k


def test_nvfp4_sample_loader_rebuilds_the_weight(tmp_path):
    """The reference sample's `_load_from_state_dict`: Params(scale=weight_scale_2,
    block_scale=weight_scale viewed as e4m3), codes from "weight"; input_scale optional."""
    w = _weights(4, 128, 256)
    qt = _nvfp4(w)
    sd = qt.state_dict("weight")
    sd["input_scale"] = torch.tensor([0.0125], dtype=torch.float32)
    path = tmp_path / "nvfp4_linear.safetensors"
    save_file({k: v.contiguous() for k, v in sd.items()}, str(path))
    st = load_file(str(path))
    params = TensorCoreNVFP4Layout.Params(scale=st.pop("weight_scale_2"), orig_dtype=torch.bfloat16,
                                          orig_shape=(128, 256),
                                          block_scale=st.pop("weight_scale").view(torch.float8_e4m3fn))
    rebuilt = QuantizedTensor(st.pop("weight"), "TensorCoreNVFP4Layout", params)
    assert set(st) == {"input_scale"}
    assert rebuilt.shape == w.shape and rebuilt.dtype == w.dtype
    assert _same(rebuilt._qdata, qt._qdata)
    assert _same(rebuilt._params.block_scale, qt._params.block_scale)
    assert _same(rebuilt._params.scale, qt._params.scale)


@pytest.mark.gpu
@pytest.mark.parametrize("make", [_fp8, _mxfp8, _nvfp4], ids=["fp8", "mxfp8", "nvfp4"])
def test_reloaded_weight_gives_the_same_linear(make, tmp_path, hip):
    """F.linear with the weight reloaded from disk equals F.linear with the original."""
    w = make(_weights(5, 256, 256))
    x = (torch.randn(64, 256, generator=torch.Generator().manual_seed(6))).bfloat16().cuda()
    path = tmp_path / "w.safetensors"
    save_file({k: v.contiguous() for k, v in w.state_dict("weight").items()}, str(path))
    st = {k: v.cuda() for k, v in load_file(str(path)).items()}
    p = w._params
    if w._layout_cls == "TensorCoreNVFP4Layout":
        params = type(p)(scale=st["weight_scale_2"], orig_dtype=p.orig_dtype, orig_shape=p.orig_shape,
                         block_scale=st["weight_scale"])
    else:
        params = type(p)(scale=st["weight_scale"], orig_dtype=p.orig_dtype, orig_shape=p.orig_shape)
    reloaded = QuantizedTensor(st["weight"], w._layout_cls, params)
    original = w.to("cuda")
    want = torch.nn.functional.linear(x, original)
    got = torch.nn.functional.linear(x, reloaded)
    assert torch.equal(got, want)


# ------------------------------------------------- committed fixture (oracle-made)
GOLDEN = __import__("pathlib").Path(__file__).resolve().parent / "golden" / "checkpoints.safetensors"
LAYOUTS = {"fp8": "TensorCoreFP8Layout", "mxfp8": "TensorCoreMXFP8Layout", "nvfp4": "TensorCoreNVFP4Layout"}


def _golden():
    return load_file(str(GOLDEN))


def test_golden_checkpoint_is_what_the_oracle_writes():
    """tests/golden/checkpoints.safetensors equals a fresh run of its generator (the CPU
    oracle), so the GPU tests below compare against the oracle."""
    import importlib.util

    spec = importlib.util.spec_from_file_location("make_checkpoints", GOLDEN.with_name("make_checkpoints.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    fresh, disk = mod.make(), _golden()
    assert set(fresh) == set(disk)
    for k in fresh:
        if k.split(".")[-1].startswith("expected"):
            # fp32 CPU matmuls: the summation order, hence the last bits, depends on the host BLAS
            assert fresh[k].dtype == disk[k].dtype and torch.allclose(fresh[k], disk[k], rtol=1e-5, atol=1e-6), k
        else:
            assert _same(fresh[k], disk[k]), k


def _load_layer(st, name, device):
    """Rebuild a layer's weight the way the reference's loaders do: codes from `weight`, the
    NVFP4 block scales from `weight_scale` viewed as e4m3 with `weight_scale_2` as the tensor
    scale (samples/nvfp4_linear.py:39-61); FP8 / MXFP8 scales from `weight_scale`
    (tensor/fp8.py:74-80, tensor/mxfp8.py:86-87)."""
    w = st["w_bf16"]
    shape = tuple(w.shape)
    codes = st[f"{name}.weight"].to(device)
    if name == "nvfp4":
        params = TensorCoreNVFP4Layout.Params(scale=st["nvfp4.weight_scale_2"].to(device), orig_dtype=w.dtype,
                                              orig_shape=shape,
                                              block_scale=st["nvfp4.weight_scale"].to(device).view(torch.float8_e4m3fn))
        return QuantizedTensor(codes, LAYOUTS[name], params)
    if name == "mxfp8":
        params = TensorCoreMXFP8Layout.Params(scale=st["mxfp8.weight_scale"].to(device).view(torch.float8_e8m0fnu),
                                              orig_dtype=w.dtype, orig_shape=shape)
    else:
        params = TensorCoreFP8Layout.Params(scale=st["fp8.weight_scale"].reshape(()).to(device), orig_dtype=w.dtype,
                                            orig_shape=shape)
    return QuantizedTensor(codes.view(torch.float8_e4m3fn), LAYOUTS[name], params)


def _rel_l2(got, want):
    return ((got.float().cpu() - want).norm() / want.norm()).item()


@pytest.mark.gpu
@pytest.mark.parametrize("name,static", [("fp8", False), ("mxfp8", False), ("nvfp4", False), ("nvfp4", True)],
                         ids=["fp8", "mxfp8", "nvfp4-dynamic", "nvfp4-static"])
def test_golden_checkpoint_linear_matches_the_oracle(name, static, hip):
    """F.linear on the GPU, with the weight loaded from the oracle-made checkpoint and the
    activation quantized by the layout (dynamic scale, or the checkpoint's input_scale),
    equals the oracle's result within bf16 output rounding (rel-L2 <= 1e-2)."""
    st = _golden()
    dev = torch.device("cuda", 0)
    w = _load_layer(st, name, dev)
    x = st["x"].to(dev)
    kw = {"scale": st["nvfp4.input_scale"].to(dev)} if static else {}
    xq = QuantizedTensor.from_float(x, LAYOUTS[name], **kw)
    y = torch.nn.functional.linear(xq, w, st[f"{name}.bias"].to(dev))
    assert y.dtype == torch.bfloat16 and tuple(y.shape) == (x.shape[0], w.shape[0])
    want = st[f"{name}.expected_static" if static else f"{name}.expected"]
    assert _rel_l2(y, want) <= 4e-3


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["fp8", "mxfp8", "nvfp4"])
def test_golden_checkpoint_bytes_from_the_gpu_quantizers(name, hip):
    """Quantizing the checkpoint's source weight on the GPU through the layout reproduces the
    committed state-dict tensors: the same keys, dtypes, shapes and bytes."""
    st = _golden()
    qt = QuantizedTensor.from_float(st["w_bf16"].cuda(), LAYOUTS[name])
    sd = {k: v.cpu() for k, v in qt.state_dict("weight").items()}
    keys = {"weight", "weight_scale", "weight_scale_2"} if name == "nvfp4" else {"weight", "weight_scale"}
    assert set(sd) == keys
    for k in keys:
        assert _same(sd[k], st[f"{name}.{k}"]), (k, sd[k].dtype, tuple(sd[k].shape), st[f"{name}.{k}"].dtype,
                                                 tuple(st[f"{name}.{k}"].shape))
