"""TensorCoreFP8Layout: per-tensor-scaled FP8 (E4M3 by default), one code per element.

Interface and semantics follow the reference's tensor/fp8.py:21-222.  The scale default
is amax(|x|) / finfo(dtype).max computed in x's own dtype, then cast to fp32
(fp8.py:56-61).  The matmuls (linear / mm / addmm) run on the gfx950 per-tensor FP8 GEMM
(`ck.scaled_mm_fp8`: out = scale_a * scale_b * a @ b.T + bias) where the reference calls
torch F.scaled_mm (fp8.py:86-101); like the reference they fall back to dequantize +
the torch op when an operand is not quantized or the kernel rejects the call.
view / reshape / t act on the codes directly (codes map 1:1 to elements).
"""
from __future__ import annotations

import logging
from dataclasses import dataclass

import torch

from .base import BaseLayoutParams, QuantizedLayout, QuantizedTensor, dequantize_args, register_layout_op

logger = logging.getLogger(__name__)
aten = torch.ops.aten
_FAILURES = (RuntimeError, TypeError, ValueError)


class TensorCoreFP8Layout(QuantizedLayout):
    """FP8 with one fp32 scale per tensor: x ~= code * scale."""

    MIN_SM_VERSION = (8, 9)

    @dataclass(frozen=True)
    class Params(BaseLayoutParams):
        def _validate_tensor_fields(self):
            if isinstance(self.scale, torch.Tensor) and self.scale.dtype != torch.float32:
                object.__setattr__(self, "scale", self.scale.to(dtype=torch.float32, non_blocking=True))

    @classmethod
    def quantize(cls, tensor: torch.Tensor, scale: torch.Tensor | float | str | None = None,
                 dtype: torch.dtype = torch.float8_e4m3fn, **kwargs):
        import comfy_kitchen as ck

        if scale is None or (isinstance(scale, str) and scale == "recalculate"):
            # amax(|x|) / max in x's dtype, as one device-side reduction
            scale = ck.amax_scale(tensor, torch.finfo(dtype).max)
        if not isinstance(scale, torch.Tensor):
            scale = torch.tensor(scale)
        scale = scale.to(device=tensor.device, dtype=torch.float32)
        qdata = ck.quantize_per_tensor_fp8(tensor, scale, dtype)
        return qdata, cls.Params(scale=scale, orig_dtype=tensor.dtype, orig_shape=tuple(tensor.shape))

    @classmethod
    def dequantize(cls, qdata: torch.Tensor, params: Params) -> torch.Tensor:
        import comfy_kitchen as ck

        return ck.dequantize_per_tensor_fp8(qdata, params.scale, params.orig_dtype)

    @classmethod
    def get_plain_tensors(cls, qtensor: QuantizedTensor) -> tuple[torch.Tensor, torch.Tensor]:
        return qtensor._qdata, qtensor._params.scale

    @classmethod
    def state_dict_tensors(cls, qdata: torch.Tensor, params: Params) -> dict[str, torch.Tensor]:
        return {"": qdata, "_scale": params.scale}


def _fp8_pair(x, w) -> bool:
    return (isinstance(x, QuantizedTensor) and isinstance(w, QuantizedTensor)
            and x._layout_cls == w._layout_cls == "TensorCoreFP8Layout")


def _matmul(x: QuantizedTensor, w_nk: torch.Tensor, scale_b: torch.Tensor, bias, out_dtype) -> torch.Tensor:
    """x (any leading dims) @ w_nk.T on the per-tensor FP8 GEMM; w_nk is [N, K] codes."""
    import comfy_kitchen as ck

    xq, scale_a = TensorCoreFP8Layout.get_plain_tensors(x)
    if xq.dtype != torch.float8_e4m3fn or w_nk.dtype != torch.float8_e4m3fn:
        raise TypeError("the FP8 GEMM takes E4M3 operands")
    if out_dtype in (torch.float8_e4m3fn, torch.float8_e5m2):
        raise TypeError("FP8 output is not produced by the FP8 GEMM")
    lead = xq.shape[:-1]
    out = ck.scaled_mm_fp8(xq.reshape(-1, xq.shape[-1]), w_nk, scale_a, scale_b, bias, out_dtype)
    return out.reshape(*lead, w_nk.shape[0])


@register_layout_op(aten.linear.default, TensorCoreFP8Layout)
def _linear(qt, args, kwargs):
    x, w = args[0], args[1]
    bias = args[2] if len(args) > 2 else kwargs.get("bias")
    if not _fp8_pair(x, w) or w._qdata.dim() != 2:
        return torch.nn.functional.linear(*dequantize_args((x, w, bias)))
    try:
        wq, sb = TensorCoreFP8Layout.get_plain_tensors(w)
        return _matmul(x, wq, sb, bias, kwargs.get("out_dtype", x._params.orig_dtype))
    except _FAILURES as e:
        logger.warning("FP8 linear on the hip GEMM failed (%s); dequantizing", e)
        return torch.nn.functional.linear(*dequantize_args((x, w, bias)))


@register_layout_op(aten.mm.default, TensorCoreFP8Layout)
def _mm(qt, args, kwargs):
    a, b = args[0], args[1]
    if not _fp8_pair(a, b) or a._qdata.dim() != 2 or b._qdata.dim() != 2:
        return torch.mm(*dequantize_args((a, b)))
    try:
        bq, sb = TensorCoreFP8Layout.get_plain_tensors(b)
        return _matmul(a, bq.t(), sb, None, kwargs.get("out_dtype", a._params.orig_dtype))
    except _FAILURES as e:
        logger.warning("FP8 mm on the hip GEMM failed (%s); dequantizing", e)
        return torch.mm(*dequantize_args((a, b)))


@register_layout_op(aten.addmm.default, TensorCoreFP8Layout)
def _addmm(qt, args, kwargs):
    bias, a, b = args[0], args[1], args[2]
    plain = kwargs.get("beta", 1) == 1 and kwargs.get("alpha", 1) == 1
    if not plain or not _fp8_pair(a, b) or a._qdata.dim() != 2 or b._qdata.dim() != 2:
        return torch.addmm(*dequantize_args((bias, a, b)), **kwargs)
    try:
        bq, sb = TensorCoreFP8Layout.get_plain_tensors(b)
        return _matmul(a, bq.t(), sb, bias, kwargs.get("out_dtype", a._params.orig_dtype))
    except _FAILURES as e:
        logger.warning("FP8 addmm on the hip GEMM failed (%s); dequantizing", e)
        return torch.addmm(*dequantize_args((bias, a, b)))


def _shape_op(op):
    """view / reshape / t on the codes themselves; the scale is shared with the input."""

    def handler(qt, args, kwargs):
        x = args[0]
        if not isinstance(x, QuantizedTensor):
            return op(*args, **kwargs)
        q = op(x._qdata, *args[1:], **kwargs)
        params = TensorCoreFP8Layout.Params(scale=x._params.scale, orig_dtype=x._params.orig_dtype,
                                            orig_shape=tuple(q.shape))
        return QuantizedTensor(q, "TensorCoreFP8Layout", params)

    return handler


for _op in (aten.view.default, aten.reshape.default, aten.t.default):
    register_layout_op(_op, TensorCoreFP8Layout)(_shape_op(_op))
