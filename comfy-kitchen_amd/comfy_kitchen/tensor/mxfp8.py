"""TensorCoreMXFP8Layout: E4M3 codes with E8M0 scales per 32-element block along K.

Interface and semantics follow the reference's tensor/mxfp8.py:21-236: 2-D tensors
only, padded to multiples of 32 in both dimensions, scales in the 32_4_4 swizzled
layout, `t()` as a flag flip, and linear / mm / addmm on the block-scaled GEMM
(`ck.scaled_mm_mxfp8`, here the gfx950 MFMA kernel) with the result sliced back to the
unpadded shape.  Other shape ops fall back to dequantization.
"""
from __future__ import annotations

import logging
from dataclasses import dataclass

import torch

from ..float_utils import roundup
from .base import (BaseLayoutParams, QuantizedLayout, QuantizedTensor, dequantize_args, register_layout_op,
                   slice_to)

logger = logging.getLogger(__name__)
aten = torch.ops.aten
_FAILURES = (RuntimeError, TypeError, ValueError)
NAME = "TensorCoreMXFP8Layout"


class TensorCoreMXFP8Layout(QuantizedLayout):
    """MXFP8: E4M3 data, power-of-two (E8M0) scale per 32 elements along the last dim."""

    MIN_SM_VERSION = (10, 0)

    @dataclass(frozen=True)
    class Params(BaseLayoutParams):
        transposed: bool = False

    @classmethod
    def quantize(cls, tensor: torch.Tensor, **kwargs):
        import comfy_kitchen as ck

        if tensor.dim() != 2:
            raise ValueError(f"MXFP8 requires 2D tensor, got {tensor.dim()}D")
        shape = tuple(tensor.shape)
        qdata, block_scale = ck.quantize_mxfp8(tensor, pad_32x=cls.get_padded_shape(shape) != shape)
        return qdata, cls.Params(scale=block_scale, orig_dtype=tensor.dtype, orig_shape=shape)

    @classmethod
    def dequantize(cls, qdata: torch.Tensor, params: Params) -> torch.Tensor:
        import comfy_kitchen as ck

        return ck.dequantize_mxfp8(qdata, params.scale, params.orig_dtype)

    @classmethod
    def get_plain_tensors(cls, qtensor: QuantizedTensor) -> tuple[torch.Tensor, torch.Tensor]:
        return qtensor._qdata, qtensor._params.scale

    @classmethod
    def state_dict_tensors(cls, qdata: torch.Tensor, params: Params) -> dict[str, torch.Tensor]:
        return {"": qdata, "_scale": params.scale}

    @classmethod
    def get_padded_shape(cls, orig_shape: tuple[int, ...]) -> tuple[int, ...]:
        if len(orig_shape) != 2:
            raise ValueError(f"MXFP8 requires 2D shape, got {len(orig_shape)}D")
        return (roundup(orig_shape[0], 32), roundup(orig_shape[1], 32))

    @classmethod
    def get_storage_shape(cls, orig_shape: tuple[int, ...]) -> tuple[int, ...]:
        return cls.get_padded_shape(orig_shape)

    @classmethod
    def get_logical_shape_from_storage(cls, storage_shape: tuple[int, ...]) -> tuple[int, ...]:
        return storage_shape


def _gemm(x: QuantizedTensor, w: QuantizedTensor, bias, out_dtype, rows: int, cols: int) -> torch.Tensor:
    """x @ w_physical.T on the MXFP8 GEMM (w's storage is [N, K]), sliced to [rows, cols]."""
    import comfy_kitchen as ck

    xq, sa = TensorCoreMXFP8Layout.get_plain_tensors(x)
    wq, sb = TensorCoreMXFP8Layout.get_plain_tensors(w)
    if bias is not None and bias.numel() != wq.shape[0]:  # the kernel's N is the padded one
        bias = torch.nn.functional.pad(bias.reshape(-1), (0, wq.shape[0] - bias.numel()))
    out = ck.scaled_mm_mxfp8(xq, wq, block_scale_a=sa, block_scale_b=sb, bias=bias, out_dtype=out_dtype)
    return slice_to(out, rows, cols)


def _pair(x, w) -> bool:
    return (isinstance(x, QuantizedTensor) and isinstance(w, QuantizedTensor)
            and x._layout_cls == w._layout_cls == NAME and x._qdata.dim() == 2)


@register_layout_op(aten.t.default, TensorCoreMXFP8Layout)
def _t(qt, args, kwargs):
    x = args[0]
    if not isinstance(x, QuantizedTensor):
        return aten.t.default(*args, **kwargs)
    r, c = x._params.orig_shape
    params = TensorCoreMXFP8Layout.Params(scale=x._params.scale, orig_dtype=x._params.orig_dtype,
                                          orig_shape=(c, r), transposed=not x._params.transposed)
    return QuantizedTensor(x._qdata, NAME, params)


@register_layout_op(aten.mm.default, TensorCoreMXFP8Layout)
def _mm(qt, args, kwargs):
    a, b = args[0], args[1]
    if not _pair(a, b) or a._params.transposed or not b._params.transposed:
        return torch.mm(*dequantize_args((a, b)))
    try:
        return _gemm(a, b, None, kwargs.get("out_dtype", a._params.orig_dtype),
                     a._params.orig_shape[0], b._params.orig_shape[1])
    except _FAILURES as e:
        logger.warning("MXFP8 mm failed (%s); dequantizing", e)
        return torch.mm(*dequantize_args((a, b)))


@register_layout_op(aten.addmm.default, TensorCoreMXFP8Layout)
def _addmm(qt, args, kwargs):
    bias, a, b = args[0], args[1], args[2]
    plain = kwargs.get("beta", 1) == 1 and kwargs.get("alpha", 1) == 1
    if not plain or not _pair(a, b) or a._params.transposed or not b._params.transposed:
        return torch.addmm(*dequantize_args((bias, a, b)), **kwargs)
    try:
        return _gemm(a, b, bias, a._params.orig_dtype, a._params.orig_shape[0], b._params.orig_shape[1])
    except _FAILURES as e:
        logger.warning("MXFP8 addmm failed (%s); dequantizing", e)
        return torch.addmm(*dequantize_args((bias, a, b)))


@register_layout_op(aten.linear.default, TensorCoreMXFP8Layout)
def _linear(qt, args, kwargs):
    x, w = args[0], args[1]
    bias = args[2] if len(args) > 2 else kwargs.get("bias")
    if not _pair(x, w) or x._params.transposed or w._params.transposed:
        return torch.nn.functional.linear(*dequantize_args((x, w, bias)))
    try:
        return _gemm(x, w, bias, kwargs.get("out_dtype", x._params.orig_dtype),
                     x._params.orig_shape[0], w._params.orig_shape[0])
    except _FAILURES as e:
        logger.warning("MXFP8 linear failed (%s); dequantizing", e)
        return torch.nn.functional.linear(*dequantize_args((x, w, bias)))
