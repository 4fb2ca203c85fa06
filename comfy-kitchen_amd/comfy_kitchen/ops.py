"""torch.library custom ops `comfy_kitchen::*` and their fake (meta) implementations.

Op names, argument order, dtype codes and output shapes follow the reference
(backends/eager/quantization.py:31-39 for the codes, 411-730 for the quantization
ops, backends/eager/rope.py:26-58 for RoPE).  Each op body asks the registry for a
backend implementation and calls it with the eager backend's keyword arguments; the
fake implementations give torch.compile the output shapes without running anything.
"""
from __future__ import annotations

import torch

from .float_utils import roundup

DTYPE_CODE_TO_DTYPE = {
    0: torch.float32,
    1: torch.float16,
    2: torch.bfloat16,
    5: torch.float8_e4m3fn,
    6: torch.float8_e5m2,
}
DTYPE_TO_CODE = {v: k for k, v in DTYPE_CODE_TO_DTYPE.items()}


def _dispatch(func_name: str, **kwargs):
    from .registry import registry

    return registry.get_implementation(func_name, kwargs=kwargs)(**kwargs)


# --------------------------------------------------------------- per-tensor FP8
@torch.library.custom_op("comfy_kitchen::quantize_fp8", mutates_args=())
def quantize_fp8(x: torch.Tensor, scale: torch.Tensor, output_dtype_code: int) -> torch.Tensor:
    return _dispatch("quantize_per_tensor_fp8", x=x, scale=scale,
                     output_type=DTYPE_CODE_TO_DTYPE[output_dtype_code])


@quantize_fp8.register_fake
def _(x, scale, output_dtype_code):
    return torch.empty_like(x, dtype=DTYPE_CODE_TO_DTYPE[output_dtype_code])


@torch.library.custom_op("comfy_kitchen::dequantize_fp8", mutates_args=())
def dequantize_fp8(x: torch.Tensor, scale: torch.Tensor, output_dtype_code: int) -> torch.Tensor:
    return _dispatch("dequantize_per_tensor_fp8", x=x, scale=scale,
                     output_type=DTYPE_CODE_TO_DTYPE[output_dtype_code])


@dequantize_fp8.register_fake
def _(x, scale, output_dtype_code):
    return torch.empty_like(x, dtype=DTYPE_CODE_TO_DTYPE[output_dtype_code])


# ------------------------------------------------------------------------ NVFP4
@torch.library.custom_op("comfy_kitchen::quantize_nvfp4", mutates_args=())
def quantize_nvfp4(x: torch.Tensor, per_tensor_scale: torch.Tensor, epsilon: float,
                   pad_16x: bool, hi_first: bool) -> tuple[torch.Tensor, torch.Tensor]:
    return _dispatch("quantize_nvfp4", x=x, per_tensor_scale=per_tensor_scale,
                     epsilon=epsilon, pad_16x=pad_16x, hi_first=hi_first)


@quantize_nvfp4.register_fake
def _(x, per_tensor_scale, epsilon, pad_16x, hi_first):
    rows, cols = x.shape
    if pad_16x:
        rows, cols = roundup(rows, 16), roundup(cols, 16)
    q = torch.empty((rows, cols // 2), dtype=torch.uint8, device=x.device)
    s = torch.empty((roundup(rows, 128), roundup(cols // 16, 4)), dtype=torch.float8_e4m3fn, device=x.device)
    return q, s


@torch.library.custom_op("comfy_kitchen::quantize_nvfp4_dynamic", mutates_args=())
def quantize_nvfp4_dynamic(x: torch.Tensor, divisor: float, pad_16x: bool,
                           hi_first: bool) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    return _dispatch("quantize_nvfp4_dynamic", x=x, divisor=divisor, pad_16x=pad_16x, hi_first=hi_first)


@quantize_nvfp4_dynamic.register_fake
def _(x, divisor, pad_16x, hi_first):
    rows, cols = x.shape
    if pad_16x:
        rows, cols = roundup(rows, 16), roundup(cols, 16)
    q = torch.empty((rows, cols // 2), dtype=torch.uint8, device=x.device)
    s = torch.empty((roundup(rows, 128), roundup(cols // 16, 4)), dtype=torch.float8_e4m3fn, device=x.device)
    return q, s, torch.empty((), dtype=torch.float32, device=x.device)


@torch.library.custom_op("comfy_kitchen::dequantize_nvfp4", mutates_args=())
def dequantize_nvfp4(qx: torch.Tensor, per_tensor_scale: torch.Tensor, block_scales: torch.Tensor,
                     output_dtype_code: int, hi_first: bool) -> torch.Tensor:
    return _dispatch("dequantize_nvfp4", qx=qx, per_tensor_scale=per_tensor_scale,
                     block_scales=block_scales, output_type=DTYPE_CODE_TO_DTYPE[output_dtype_code],
                     hi_first=hi_first)


@dequantize_nvfp4.register_fake
def _(qx, per_tensor_scale, block_scales, output_dtype_code, hi_first):
    rows, cols = qx.shape
    return torch.empty((rows, cols * 2), dtype=DTYPE_CODE_TO_DTYPE[output_dtype_code], device=qx.device)


@torch.library.custom_op("comfy_kitchen::scaled_mm_nvfp4", mutates_args=())
def scaled_mm_nvfp4(a: torch.Tensor, b: torch.Tensor, tensor_scale_a: torch.Tensor,
                    tensor_scale_b: torch.Tensor, block_scale_a: torch.Tensor,
                    block_scale_b: torch.Tensor, bias: torch.Tensor | None,
                    output_dtype_code: int, alpha: torch.Tensor | None) -> torch.Tensor:
    return _dispatch("scaled_mm_nvfp4", a=a, b=b, tensor_scale_a=tensor_scale_a,
                     tensor_scale_b=tensor_scale_b, block_scale_a=block_scale_a,
                     block_scale_b=block_scale_b, bias=bias,
                     out_dtype=DTYPE_CODE_TO_DTYPE[output_dtype_code], alpha=alpha)


@scaled_mm_nvfp4.register_fake
def _(a, b, tensor_scale_a, tensor_scale_b, block_scale_a, block_scale_b, bias, output_dtype_code, alpha):
    return torch.empty((a.shape[0], b.shape[0]), dtype=DTYPE_CODE_TO_DTYPE[output_dtype_code], device=a.device)


# ------------------------------------------------------------- dynamic scales
@torch.library.custom_op("comfy_kitchen::amax_scale", mutates_args=())
def amax_scale(x: torch.Tensor, divisor: float) -> torch.Tensor:
    return _dispatch("amax_scale", x=x, divisor=divisor)


@amax_scale.register_fake
def _(x, divisor):
    return torch.empty((), dtype=torch.float32, device=x.device)


# ------------------------------------------------------------------------ MXFP8
@torch.library.custom_op("comfy_kitchen::quantize_mxfp8", mutates_args=())
def quantize_mxfp8(x: torch.Tensor, pad_32x: bool) -> tuple[torch.Tensor, torch.Tensor]:
    return _dispatch("quantize_mxfp8", x=x, pad_32x=pad_32x)


@quantize_mxfp8.register_fake
def _(x, pad_32x):
    rows, cols = x.shape
    if pad_32x:
        rows, cols = roundup(rows, 32), roundup(cols, 32)
    q = torch.empty((rows, cols), dtype=torch.float8_e4m3fn, device=x.device)
    s = torch.empty((roundup(rows, 128), roundup(cols // 32, 4)), dtype=torch.float8_e8m0fnu, device=x.device)
    return q, s


@torch.library.custom_op("comfy_kitchen::dequantize_mxfp8", mutates_args=())
def dequantize_mxfp8(qx: torch.Tensor, block_scales: torch.Tensor, output_dtype_code: int) -> torch.Tensor:
    return _dispatch("dequantize_mxfp8", qx=qx, block_scales=block_scales,
                     output_type=DTYPE_CODE_TO_DTYPE[output_dtype_code])


@dequantize_mxfp8.register_fake
def _(qx, block_scales, output_dtype_code):
    return torch.empty_like(qx, dtype=DTYPE_CODE_TO_DTYPE[output_dtype_code])


@torch.library.custom_op("comfy_kitchen::scaled_mm_mxfp8", mutates_args=())
def scaled_mm_mxfp8(a: torch.Tensor, b: torch.Tensor, block_scale_a: torch.Tensor,
                    block_scale_b: torch.Tensor, bias: torch.Tensor | None,
                    output_dtype_code: int) -> torch.Tensor:
    return _dispatch("scaled_mm_mxfp8", a=a, b=b, block_scale_a=block_scale_a,
                     block_scale_b=block_scale_b, bias=bias,
                     out_dtype=DTYPE_CODE_TO_DTYPE[output_dtype_code])


@scaled_mm_mxfp8.register_fake
def _(a, b, block_scale_a, block_scale_b, bias, output_dtype_code):
    return torch.empty((a.shape[0], b.shape[0]), dtype=DTYPE_CODE_TO_DTYPE[output_dtype_code], device=a.device)


@torch.library.custom_op("comfy_kitchen::scaled_mm_fp8", mutates_args=())
def scaled_mm_fp8(a: torch.Tensor, b: torch.Tensor, scale_a: torch.Tensor, scale_b: torch.Tensor,
                  bias: torch.Tensor | None, output_dtype_code: int) -> torch.Tensor:
    return _dispatch("scaled_mm_fp8", a=a, b=b, scale_a=scale_a, scale_b=scale_b, bias=bias,
                     out_dtype=DTYPE_CODE_TO_DTYPE[output_dtype_code])


@scaled_mm_fp8.register_fake
def _(a, b, scale_a, scale_b, bias, output_dtype_code):
    return torch.empty((a.shape[0], b.shape[0]), dtype=DTYPE_CODE_TO_DTYPE[output_dtype_code], device=a.device)


# ------------------------------------------------------------------------- RoPE
@torch.library.custom_op("comfy_kitchen::apply_rope", mutates_args=())
def apply_rope(xq: torch.Tensor, xk: torch.Tensor, freqs_cis: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    return _dispatch("apply_rope", xq=xq, xk=xk, freqs_cis=freqs_cis)


@apply_rope.register_fake
def _(xq, xk, freqs_cis):
    return torch.empty_like(xq), torch.empty_like(xk)


@torch.library.custom_op("comfy_kitchen::apply_rope1", mutates_args=())
def apply_rope1(x: torch.Tensor, freqs_cis: torch.Tensor) -> torch.Tensor:
    return _dispatch("apply_rope1", x=x, freqs_cis=freqs_cis)


@apply_rope1.register_fake
def _(x, freqs_cis):
    return torch.empty_like(x)
