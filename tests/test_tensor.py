"""QuantizedTensor and the three layouts (the reference's tests/test_tensor.py cases).

CPU tests build QuantizedTensors from hand-made storage and cover params, shapes, the
generic aten handlers, flatten/unflatten and the shape-op handlers.  GPU tests cover
quantize/dequantize parity against the oracle and F.linear / mm / addmm on the gfx950
GEMMs against an fp32 matmul of the dequantized operands (rel-L2 <= 1e-2, the GEMM bar).
"""
import dataclasses

import pytest
import torch

from comfy_kitchen.tensor import (QuantizedTensor, TensorCoreFP8Layout, TensorCoreMXFP8Layout,
                                  TensorCoreNVFP4Layout, get_layout_class)

REL_L2 = 1e-2


def rel_l2(a, b):
    a, b = a.float(), b.float()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def fp8_qt(shape=(4, 8), scale=0.5, dtype=torch.bfloat16):
    q = torch.arange(torch.Size(shape).numel(), dtype=torch.uint8).reshape(shape).view(torch.float8_e4m3fn)
    p = TensorCoreFP8Layout.Params(scale=torch.tensor(scale), orig_dtype=dtype, orig_shape=tuple(shape))
    return QuantizedTensor(q, "TensorCoreFP8Layout", p)


def nvfp4_qt(shape=(20, 40)):
    rows, cols = TensorCoreNVFP4Layout.get_padded_shape(shape)
    q = torch.zeros(rows, cols // 2, dtype=torch.uint8)
    bs = torch.zeros(128, 4 * ((cols // 16 + 3) // 4), dtype=torch.uint8).view(torch.float8_e4m3fn)
    p = TensorCoreNVFP4Layout.Params(scale=torch.tensor(2.0), orig_dtype=torch.bfloat16, orig_shape=shape,
                                     block_scale=bs)
    return QuantizedTensor(q, "TensorCoreNVFP4Layout", p)


def mxfp8_qt(shape=(40, 70)):
    rows, cols = TensorCoreMXFP8Layout.get_padded_shape(shape)
    q = torch.zeros(rows, cols, dtype=torch.uint8).view(torch.float8_e4m3fn)
    s = torch.zeros(128, 4, dtype=torch.uint8)
    p = TensorCoreMXFP8Layout.Params(scale=s, orig_dtype=torch.bfloat16, orig_shape=shape)
    return QuantizedTensor(q, "TensorCoreMXFP8Layout", p)


# ----------------------------------------------------------------------------- CPU
class TestParams:
    def test_fp8_scale_cast_to_f32(self):
        p = TensorCoreFP8Layout.Params(scale=torch.tensor(2.0, dtype=torch.float64), orig_dtype=torch.bfloat16,
                                       orig_shape=(2, 2))
        assert p.scale.dtype == torch.float32

    def test_nvfp4_tensor_fields_clone_and_copy(self):
        qt = nvfp4_qt()
        p = qt.params
        assert p._tensor_fields() == ["scale", "block_scale"]
        c = p.clone()
        assert c.block_scale.data_ptr() != p.block_scale.data_ptr() and c.scale.data_ptr() != p.scale.data_ptr()
        src = dataclasses.replace(p, scale=torch.tensor(7.0), block_scale=torch.ones_like(p.block_scale.view(torch.uint8)).view(torch.float8_e4m3fn))
        c.copy_from(src)
        assert c.scale.item() == 7.0 and bool((c.block_scale.view(torch.uint8) == 1).all())

    def test_to_device_same_device(self):
        p = nvfp4_qt().params.to_device(torch.device("cpu"))
        assert p.block_scale.device.type == "cpu"

    @pytest.mark.parametrize("layout", [TensorCoreFP8Layout, TensorCoreMXFP8Layout, TensorCoreNVFP4Layout])
    def test_params_inherit_base(self, layout):
        from comfy_kitchen.tensor import BaseLayoutParams

        assert issubclass(layout.Params, BaseLayoutParams)


class TestShapes:
    def test_nvfp4_padded_and_storage(self):
        assert TensorCoreNVFP4Layout.get_padded_shape((20, 40)) == (32, 48)
        assert TensorCoreNVFP4Layout.get_storage_shape((20, 40)) == (32, 24)
        assert TensorCoreNVFP4Layout.get_logical_shape_from_storage((32, 24)) == (32, 48)

    def test_mxfp8_padded_and_storage(self):
        assert TensorCoreMXFP8Layout.get_padded_shape((40, 70)) == (64, 96)
        assert TensorCoreMXFP8Layout.get_storage_shape((64, 96)) == (64, 96)

    @pytest.mark.parametrize("layout", [TensorCoreMXFP8Layout, TensorCoreNVFP4Layout])
    def test_requires_2d(self, layout):
        with pytest.raises(ValueError):
            layout.quantize(torch.randn(2, 3, 32))
        with pytest.raises(ValueError):
            layout.get_padded_shape((2, 3, 4))

    def test_shape_vs_storage(self):
        qt = nvfp4_qt((20, 40))
        assert qt.shape == (20, 40) and qt.storage_shape == (32, 24)
        assert qt.padded_shape == (32, 48) and qt.is_padded
        assert not fp8_qt((4, 8)).is_padded


class TestGenericHandlers:
    def test_repr_and_props(self):
        qt = fp8_qt()
        assert "TensorCoreFP8Layout" in repr(qt)
        assert qt.dtype == torch.bfloat16 and qt.storage_dtype == torch.float8_e4m3fn
        assert qt.nbytes == 32 and qt.layout_cls is TensorCoreFP8Layout

    def test_detach_clone(self):
        qt = fp8_qt()
        d = qt.detach()
        assert isinstance(d, QuantizedTensor) and d._qdata.data_ptr() == qt._qdata.data_ptr()
        c = qt.clone()
        assert c._qdata.data_ptr() != qt._qdata.data_ptr()
        assert torch.equal(c._qdata.view(torch.uint8), qt._qdata.view(torch.uint8))

    def test_to_dtype(self):
        qt = fp8_qt()
        h = qt.to(torch.float16)
        assert isinstance(h, QuantizedTensor) and h.dtype == torch.float16
        assert h._qdata.dtype == torch.float8_e4m3fn and qt.dtype == torch.bfloat16
        assert qt.to(torch.bfloat16) is qt

    def test_to_copy_same_dtype_copies(self):
        qt = fp8_qt()
        c = torch.ops.aten._to_copy.default(qt)
        assert isinstance(c, QuantizedTensor) and c._qdata.data_ptr() != qt._qdata.data_ptr()

    def test_contiguous(self):
        qt = fp8_qt()
        assert qt.contiguous() is qt and qt.is_contiguous()

    def test_copy_(self):
        dst, src = fp8_qt(scale=1.0, dtype=torch.float16), fp8_qt(scale=3.0)
        src._qdata.view(torch.uint8).fill_(9)
        dst.copy_(src)
        assert bool((dst._qdata.view(torch.uint8) == 9).all())
        assert dst.params.scale.item() == 3.0 and dst.dtype == torch.float16 and dst.params.orig_dtype == torch.float16

    def test_copy_validation(self):
        with pytest.raises(TypeError):
            fp8_qt().copy_(torch.zeros(4, 8, dtype=torch.bfloat16))
        with pytest.raises(TypeError):
            mxfp8_qt((32, 32)).copy_(fp8_qt((32, 32)))

    def test_empty_like(self):
        qt = fp8_qt()
        e = torch.empty_like(qt)
        assert isinstance(e, QuantizedTensor) and e.shape == qt.shape
        e2 = torch.empty_like(qt, dtype=torch.float16)
        assert e2.dtype == torch.float16 and e2._qdata.dtype == torch.float8_e4m3fn

    def test_state_dict(self):
        assert set(fp8_qt().state_dict("w").keys()) == {"w", "w_scale"}
        assert set(nvfp4_qt().state_dict("w").keys()) == {"w", "w_scale", "w_scale_2"}
        assert set(mxfp8_qt().state_dict().keys()) == {"", "_scale"}

    @pytest.mark.parametrize("make", [fp8_qt, nvfp4_qt, mxfp8_qt])
    def test_flatten_unflatten(self, make):
        qt = make()
        inner, ctx = qt.__tensor_flatten__()
        back = QuantizedTensor.__tensor_unflatten__({k: getattr(qt, k) for k in inner}, ctx, None, None)
        assert back._layout_cls == qt._layout_cls and back.shape == qt.shape
        assert torch.equal(back._qdata.view(torch.uint8), qt._qdata.view(torch.uint8))

    def test_layout_registry(self):
        assert get_layout_class("TensorCoreNVFP4Layout") is TensorCoreNVFP4Layout

    def test_no_fast_matmul_without_gpu(self):
        if torch.cuda.is_available():
            pytest.skip("CPU-only check")
        assert TensorCoreFP8Layout.supports_fast_matmul() is False
        req = TensorCoreMXFP8Layout.get_requirements()
        assert req["fast_matmul_supported"] is False and req["required_arch"] == ("gfx950",)


class TestShapeHandlers:
    def test_fp8_view_reshape_t(self):
        qt = fp8_qt((4, 8))
        v = qt.view(8, 4)
        assert isinstance(v, QuantizedTensor) and v.shape == (8, 4) and v.params.orig_shape == (8, 4)
        r = qt.reshape(-1)
        assert r.shape == (32,)
        t = qt.t()
        assert t.shape == (8, 4) and torch.equal(t._qdata.view(torch.uint8), qt._qdata.view(torch.uint8).t())

    @pytest.mark.parametrize("make", [nvfp4_qt, mxfp8_qt])
    def test_block_layout_t_is_flag(self, make):
        qt = make()
        t = qt.t()
        assert t.params.transposed and t.shape == (qt.shape[1], qt.shape[0])
        assert t._qdata.data_ptr() == qt._qdata.data_ptr()
        tt = t.t()
        assert not tt.params.transposed and tt.shape == qt.shape


# ----------------------------------------------------------------------------- GPU
dev = torch.device("cuda")


@pytest.mark.gpu
class TestQuantizeGPU:
    def test_fp8_from_float_matches_oracle(self, hip):
        from oracle import eager_ref as ref

        x = (torch.randn(96, 256) * 3).bfloat16()
        qt = QuantizedTensor.from_float(x.to(dev), "TensorCoreFP8Layout")
        scale = (torch.amax(x.abs()) / 448.0).float().reshape(())
        assert torch.equal(qt.params.scale.cpu().reshape(()), scale)  # default scale in x's dtype
        want = ref.quantize_per_tensor_fp8(x, scale.reshape(1))
        assert torch.equal(qt._qdata.cpu().view(torch.uint8), want.view(torch.uint8))
        dq = qt.dequantize().cpu()
        assert torch.equal(dq.view(torch.int16), ref.dequantize_per_tensor_fp8(want, scale.reshape(1)).view(torch.int16))

    @pytest.mark.parametrize("shape", [(128, 256), (40, 70)])
    def test_mxfp8_from_float(self, hip, shape):
        from oracle import eager_ref as ref

        x = torch.randn(*shape).bfloat16()
        qt = QuantizedTensor.from_float(x.to(dev), "TensorCoreMXFP8Layout")
        pad = TensorCoreMXFP8Layout.get_padded_shape(shape) != shape
        q, s = ref.quantize_mxfp8(x, pad_32x=pad)
        assert qt.storage_shape == TensorCoreMXFP8Layout.get_storage_shape(shape)
        assert torch.equal(qt._qdata.cpu().view(torch.uint8), q.view(torch.uint8))
        assert torch.equal(qt.params.scale.cpu().view(torch.uint8), s.view(torch.uint8))
        dq = qt.dequantize().cpu()
        assert dq.shape == shape
        want = ref.dequantize_mxfp8(q, s)[: shape[0], : shape[1]]
        assert torch.equal(dq.view(torch.int16), want.view(torch.int16))

    @pytest.mark.parametrize("shape", [(128, 256), (20, 40)])
    def test_nvfp4_from_float(self, hip, shape):
        from oracle import eager_ref as ref

        x = torch.randn(*shape).bfloat16()
        qt = QuantizedTensor.from_float(x.to(dev), "TensorCoreNVFP4Layout")
        scale = (torch.amax(x.abs()) / (448.0 * 6.0)).float().reshape(1)
        assert torch.equal(qt.params.scale.cpu().reshape(1), scale)
        pad = TensorCoreNVFP4Layout.get_padded_shape(shape) != shape
        q, s = ref.quantize_nvfp4(x, scale, pad_16x=pad)
        assert qt.storage_shape == TensorCoreNVFP4Layout.get_storage_shape(shape)
        assert torch.equal(qt._qdata.cpu(), q)
        assert torch.equal(qt.params.block_scale.cpu().view(torch.uint8), s.view(torch.uint8))
        dq = qt.dequantize().cpu()
        want = ref.dequantize_nvfp4(q, scale, s)[: shape[0], : shape[1]]
        assert dq.shape == shape and torch.equal(dq.view(torch.int16), want.view(torch.int16))

    @pytest.mark.parametrize("name", ["TensorCoreMXFP8Layout", "TensorCoreNVFP4Layout"])
    def test_transposed_dequantize(self, hip, name):
        x = torch.randn(64, 96, device=dev).bfloat16()
        qt = QuantizedTensor.from_float(x, name)
        assert torch.equal(qt.t().dequantize(), qt.dequantize().t())

    def test_to_device_roundtrip(self, hip):
        qt = QuantizedTensor.from_float(torch.randn(32, 64, device=dev).bfloat16(), "TensorCoreNVFP4Layout")
        back = qt.to("cpu").to(dev)
        assert torch.equal(back._qdata, qt._qdata) and torch.equal(back.dequantize(), qt.dequantize())

    def test_fallback_op_dequantizes(self, hip):
        qt = QuantizedTensor.from_float(torch.randn(16, 32, device=dev).bfloat16(), "TensorCoreFP8Layout")
        out = qt + 1
        assert not isinstance(out, QuantizedTensor)
        assert torch.equal(out, qt.dequantize() + 1)


def _ref_linear(x, w, bias=None):
    """fp32 linear on dequantized operands (the GEMM bar's reference)."""
    out = x.dequantize().float() @ w.dequantize().float().t() if isinstance(x, QuantizedTensor) else None
    if bias is not None:
        out = out + bias.float()
    return out


@pytest.mark.gpu
class TestMatmulGPU:
    @pytest.mark.parametrize("name", ["TensorCoreFP8Layout", "TensorCoreMXFP8Layout", "TensorCoreNVFP4Layout"])
    @pytest.mark.parametrize("with_bias", [False, True])
    def test_linear(self, hip, name, with_bias):
        x = torch.randn(96, 256, device=dev).bfloat16()
        w = (torch.randn(160, 256, device=dev) * 0.05).bfloat16()
        b = torch.randn(160, device=dev).bfloat16() if with_bias else None
        qx, qw = QuantizedTensor.from_float(x, name), QuantizedTensor.from_float(w, name)
        y = torch.nn.functional.linear(qx, qw, b)
        assert not isinstance(y, QuantizedTensor) and y.shape == (96, 160) and y.dtype == torch.bfloat16
        assert rel_l2(y, _ref_linear(qx, qw, b)) <= REL_L2

    @pytest.mark.parametrize("name", ["TensorCoreMXFP8Layout", "TensorCoreNVFP4Layout"])
    def test_linear_padded(self, hip, name):
        x = torch.randn(50, 100, device=dev).bfloat16()
        w = (torch.randn(70, 100, device=dev) * 0.05).bfloat16()
        b = torch.randn(70, device=dev).bfloat16()
        qx, qw = QuantizedTensor.from_float(x, name), QuantizedTensor.from_float(w, name)
        assert qx.is_padded and qw.is_padded
        y = torch.nn.functional.linear(qx, qw, b)
        assert y.shape == (50, 70)
        assert rel_l2(y, _ref_linear(qx, qw, b)) <= REL_L2

    def test_fp8_linear_3d_input(self, hip):
        x = torch.randn(4, 16, 64, device=dev).bfloat16()
        w = torch.randn(128, 64, device=dev).bfloat16()
        qx, qw = QuantizedTensor.from_float(x, "TensorCoreFP8Layout"), QuantizedTensor.from_float(w, "TensorCoreFP8Layout")
        y = torch.nn.functional.linear(qx, qw)
        assert y.shape == (4, 16, 128)
        want = qx.dequantize().float() @ qw.dequantize().float().t()
        assert rel_l2(y, want) <= REL_L2

    @pytest.mark.parametrize("name", ["TensorCoreFP8Layout", "TensorCoreMXFP8Layout", "TensorCoreNVFP4Layout"])
    def test_mm_with_transposed_b(self, hip, name):
        a = torch.randn(64, 128, device=dev).bfloat16()
        w = torch.randn(96, 128, device=dev).bfloat16()
        qa, qw = QuantizedTensor.from_float(a, name), QuantizedTensor.from_float(w, name)
        y = torch.mm(qa, qw.t())
        assert y.shape == (64, 96)
        assert rel_l2(y, qa.dequantize().float() @ qw.dequantize().float().t()) <= REL_L2

    @pytest.mark.parametrize("name", ["TensorCoreFP8Layout", "TensorCoreMXFP8Layout", "TensorCoreNVFP4Layout"])
    def test_addmm(self, hip, name):
        a = torch.randn(64, 128, device=dev).bfloat16()
        w = torch.randn(96, 128, device=dev).bfloat16()
        b = torch.randn(96, device=dev).bfloat16()
        qa, qw = QuantizedTensor.from_float(a, name), QuantizedTensor.from_float(w, name)
        y = torch.addmm(b, qa, qw.t())
        want = b.float() + qa.dequantize().float() @ qw.dequantize().float().t()
        assert y.shape == (64, 96) and rel_l2(y, want) <= REL_L2

    @pytest.mark.parametrize("name", ["TensorCoreFP8Layout", "TensorCoreMXFP8Layout", "TensorCoreNVFP4Layout"])
    def test_weight_only_quantized_falls_back(self, hip, name):
        x = torch.randn(32, 64, device=dev).bfloat16()
        qw = QuantizedTensor.from_float(torch.randn(48, 64, device=dev).bfloat16(), name)
        y = torch.nn.functional.linear(x, qw)
        want = torch.nn.functional.linear(x, qw.dequantize())
        assert y.shape == (32, 48) and rel_l2(y, want) <= 1e-3

    def test_fp16_output_dtype(self, hip):
        x = torch.randn(64, 128, device=dev).half()
        w = torch.randn(96, 128, device=dev).half()
        for name in ("TensorCoreFP8Layout", "TensorCoreMXFP8Layout", "TensorCoreNVFP4Layout"):
            y = torch.nn.functional.linear(QuantizedTensor.from_float(x, name), QuantizedTensor.from_float(w, name))
            assert y.dtype == torch.float16, name

    def test_fp8_different_scales(self, hip):
        x = torch.randn(64, 128, device=dev).bfloat16()
        w = torch.randn(96, 128, device=dev).bfloat16()
        qx = QuantizedTensor.from_float(x, "TensorCoreFP8Layout", scale=0.01)
        qw = QuantizedTensor.from_float(w, "TensorCoreFP8Layout", scale=torch.tensor(0.02))
        y = torch.nn.functional.linear(qx, qw)
        assert rel_l2(y, _ref_linear(qx, qw)) <= REL_L2

    def test_fp8_gemm_entry_point_parity(self, hip):
        """ck.scaled_mm_fp8 directly: scales, bias and a K that is a multiple of 16 only."""
        import comfy_kitchen as ck

        # (4352, 4196, 64): 289 tiles, so the last 33 run as half tiles in the same grid
        for m, n, k in ((256, 256, 256), (300, 200, 48), (5, 7, 16), (4352, 4196, 64)):
            a = (torch.randn(m, k, device=dev) * 2).to(torch.float8_e4m3fn)
            b = (torch.randn(n, k, device=dev) * 2).to(torch.float8_e4m3fn)
            sa, sb = torch.tensor([0.25], device=dev), torch.tensor([3.0], device=dev)
            bias = torch.randn(n, device=dev)
            y = ck.scaled_mm_fp8(a, b, sa, sb, bias, torch.float32)
            want = (a.float() @ b.float().t()) * 0.75 + bias
            # fp32 output: only the summation order differs from torch's fp32 matmul
            # (measured ~1.5e-5, as for the MXFP8 GEMM)
            assert rel_l2(y, want) <= 1e-4, (m, n, k)
