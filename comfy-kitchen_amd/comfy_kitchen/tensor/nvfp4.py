"""TensorCoreNVFP4Layout: E2M1 codes packed two per byte, an E4M3 scale per 16-element
block along K, and one fp32 tensor scale.

Interface and semantics follow the reference's tensor/nvfp4.py:21-264: 2-D tensors
only, padded to multiples of 16, storage [rows, cols / 2] uint8 (even element in the
high nibble), block scales in the 32_4_4 swizzled layout, the tensor-scale default
amax(|x|) / (448 * 6) computed in x's dtype then cast to fp32 (nvfp4.py:64-69),
state-dict keys "" / "_scale" (block scales) / "_scale_2" (tensor scale), `t()` as a
flag flip, and linear / mm on the block-scaled GEMM (`ck.scaled_mm_nvfp4`).  addmm
(F.linear with bias after decomposition) also runs on the GEMM here, where the
reference dequantizes.
"""
from __future__ import annotations

import logging
from dataclasses import dataclass

import torch

from ..float_utils import F4_E2M1_MAX, F8_E4M3_MAX, roundup
from .base import (BaseLayoutParams, QuantizedLayout, QuantizedTensor, dequantize_args, register_layout_op,
                   slice_to)

logger = logging.getLogger(__name__)
aten = torch.ops.aten
_FAILURES = (RuntimeError, TypeError, ValueError)
NAME = "TensorCoreNVFP4Layout"


class TensorCoreNVFP4Layout(QuantizedLayout):
    """NVFP4: x ~= E2M1(code) * E4M3(block scale) * fp32 tensor scale."""

    MIN_SM_VERSION = (10, 0)

    @dataclass(frozen=True)
    class Params(BaseLayoutParams):
        block_scale: torch.Tensor
        transposed: bool = False

        def _validate_tensor_fields(self):
            if isinstance(self.scale, torch.Tensor) and self.scale.dtype != torch.float32:
                object.__setattr__(self, "scale", self.scale.to(dtype=torch.float32, non_blocking=True))

    @classmethod
    def quantize(cls, tensor: torch.Tensor, scale: torch.Tensor | float | str | None = None, **kwargs):
        import comfy_kitchen as ck

        if tensor.dim() != 2:
            raise ValueError(f"NVFP4 requires 2D tensor, got {tensor.dim()}D")
        shape = tuple(tensor.shape)
        pad = cls.get_padded_shape(shape) != shape
        if scale is None or (isinstance(scale, str) and scale == "recalculate"):
            # amax(|x|) / max in x's dtype, reduced on the device in the quantize call
            qdata, block_scale, scale = ck.quantize_nvfp4_dynamic(tensor, F8_E4M3_MAX * F4_E2M1_MAX, pad_16x=pad)
            return qdata, cls.Params(scale=scale, orig_dtype=tensor.dtype, orig_shape=shape, block_scale=block_scale)
        if not isinstance(scale, torch.Tensor):
            scale = torch.tensor(scale)
        scale = scale.to(device=tensor.device, dtype=torch.float32)
        qdata, block_scale = ck.quantize_nvfp4(tensor, scale, pad_16x=pad)
        return qdata, cls.Params(scale=scale, orig_dtype=tensor.dtype, orig_shape=shape, block_scale=block_scale)

    @classmethod
    def dequantize(cls, qdata: torch.Tensor, params: Params) -> torch.Tensor:
        import comfy_kitchen as ck

        return ck.dequantize_nvfp4(qdata, params.scale, params.block_scale, params.orig_dtype)

    @classmethod
    def get_plain_tensors(cls, qtensor: QuantizedTensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        return qtensor._qdata, qtensor._params.scale, qtensor._params.block_scale

    @classmethod
    def state_dict_tensors(cls, qdata: torch.Tensor, params: Params) -> dict[str, torch.Tensor]:
        return {"": qdata, "_scale": params.block_scale, "_scale_2": params.scale}

    @classmethod
    def get_padded_shape(cls, orig_shape: tuple[int, ...]) -> tuple[int, ...]:
        if len(orig_shape) != 2:
            raise ValueError(f"NVFP4 requires 2D shape, got {len(orig_shape)}D")
        return (roundup(orig_shape[0], 16), roundup(orig_shape[1], 16))

    @classmethod
    def get_storage_shape(cls, orig_shape: tuple[int, ...]) -> tuple[int, ...]:
        rows, cols = cls.get_padded_shape(orig_shape)
        return (rows, cols // 2)

    @classmethod
    def get_logical_shape_from_storage(cls, storage_shape: tuple[int, ...]) -> tuple[int, ...]:
        return (storage_shape[0], storage_shape[1] * 2)


def _gemm(x: QuantizedTensor, w: QuantizedTensor, bias, out_dtype, rows: int, cols: int) -> torch.Tensor:
    """x @ w_physical.T on the NVFP4 GEMM (w's storage is [N, K/2]), sliced to [rows, cols]."""
    import comfy_kitchen as ck

    xq, ts_a, bs_a = TensorCoreNVFP4Layout.get_plain_tensors(x)
    wq, ts_b, bs_b = TensorCoreNVFP4Layout.get_plain_tensors(w)
    if bias is not None and bias.numel() != wq.shape[0]:  # the kernel's N is the padded one
        bias = torch.nn.functional.pad(bias.reshape(-1), (0, wq.shape[0] - bias.numel()))
    out = ck.scaled_mm_nvfp4(xq, wq, tensor_scale_a=ts_a, tensor_scale_b=ts_b, block_scale_a=bs_a,
                             block_scale_b=bs_b, bias=bias, out_dtype=out_dtype)
    return slice_to(out, rows, cols)


def _pair(x, w) -> bool:
    return (isinstance(x, QuantizedTensor) and isinstance(w, QuantizedTensor)
            and x._layout_cls == w._layout_cls == NAME and x._qdata.dim() == 2)


@register_layout_op(aten.t.default, TensorCoreNVFP4Layout)
def _t(qt, args, kwargs):
    x = args[0]
    if not isinstance(x, QuantizedTensor):
        return aten.t.default(*args, **kwargs)
    r, c = x._params.orig_shape
    params = TensorCoreNVFP4Layout.Params(scale=x._params.scale, orig_dtype=x._params.orig_dtype, orig_shape=(c, r),
                                          block_scale=x._params.block_scale, transposed=not x._params.transposed)
    return QuantizedTensor(x._qdata, NAME, params)


@register_layout_op(aten.mm.default, TensorCoreNVFP4Layout)
def _mm(qt, args, kwargs):
    a, b = args[0], args[1]
    if not _pair(a, b) or a._params.transposed or not b._params.transposed:
        return torch.mm(*dequantize_args((a, b)))
    try:
        return _gemm(a, b, None, kwargs.get("out_dtype", a._params.orig_dtype),
                     a._params.orig_shape[0], b._params.orig_shape[1])
    except _FAILURES as e:
        logger.warning("NVFP4 mm failed (%s); dequantizing", e)
        return torch.mm(*dequantize_args((a, b)))


@register_layout_op(aten.addmm.default, TensorCoreNVFP4Layout)
def _addmm(qt, args, kwargs):
    bias, a, b = args[0], args[1], args[2]
    plain = kwargs.get("beta", 1) == 1 and kwargs.get("alpha", 1) == 1
    if not plain or not _pair(a, b) or a._params.transposed or not b._params.transposed:
        return torch.addmm(*dequantize_args((bias, a, b)), **kwargs)
    try:
        return _gemm(a, b, bias, a._params.orig_dtype, a._params.orig_shape[0], b._params.orig_shape[1])
    except _FAILURES as e:
        logger.warning("NVFP4 addmm failed (%s); dequantizing", e)
        return torch.addmm(*dequantize_args((bias, a, b)))


@register_layout_op(aten.linear.default, TensorCoreNVFP4Layout)
def _linear(qt, args, kwargs):
    x, w = args[0], args[1]
    bias = args[2] if len(args) > 2 else kwargs.get("bias")
    if not _pair(x, w) or x._params.transposed or w._params.transposed:
        return torch.nn.functional.linear(*dequantize_args((x, w, bias)))
    try:
        return _gemm(x, w, bias, kwargs.get("out_dtype", x._params.orig_dtype),
                     x._params.orig_shape[0], w._params.orig_shape[0])
    except _FAILURES as e:
        logger.warning("NVFP4 linear failed (%s); dequantizing", e)
        return torch.nn.functional.linear(*dequantize_args((x, w, bias)))
