"""comfy_kitchen for MI355X: quantize / block-scaled GEMM / RoPE on gfx950.

Drop-in for the reference's public op API (comfy_kitchen/__init__.py:60-366): the
same function names, signatures, defaults and return types.  Every op goes through
the `comfy_kitchen::*` custom ops and the backend registry to the "hip" backend,
whose kernels are hand-written for gfx950 and reached through a C-ABI library.
"""
import torch

from . import ops as _ops  # noqa: F401  (registers torch.ops.comfy_kitchen.*)
from .backends import hip as _hip_backend  # noqa: F401  (registers the "hip" backend)
from .exceptions import (
    BackendError,
    BackendNotFoundError,
    BackendNotImplementedError,
    NoCapableBackendError,
)
from .float_utils import from_blocked, swap_nibbles, to_blocked
from .ops import DTYPE_TO_CODE
from .registry import registry

__version__ = "0.1.0"

__all__ = [
    "quantize_per_tensor_fp8",
    "dequantize_per_tensor_fp8",
    "quantize_nvfp4",
    "quantize_nvfp4_dynamic",
    "dequantize_nvfp4",
    "quantize_mxfp8",
    "dequantize_mxfp8",
    "scaled_mm_nvfp4",
    "scaled_mm_mxfp8",
    "apply_rope",
    "apply_rope1",
    "swap_nibbles",
    "to_blocked",
    "from_blocked",
    "list_backends",
    "set_backend_priority",
    "enable_backend",
    "disable_backend",
    "stochastic_rounding_fp8",
    "use_backend",
    "BackendError",
    "BackendNotFoundError",
    "BackendNotImplementedError",
    "NoCapableBackendError",
]


def amax_scale(x: torch.Tensor, divisor: float) -> torch.Tensor:
    """amax(|x|) / divisor computed in x's dtype, returned as a 0-dim fp32 device tensor.

    Not part of the reference's public API: it is the default scale of the layouts'
    quantize (reference tensor/fp8.py:56-61, tensor/nvfp4.py:64-69) as one device-side
    reduction, so dynamic quantization needs no host round trip.
    """
    return torch.ops.comfy_kitchen.amax_scale(x, float(divisor))


def quantize_per_tensor_fp8(x: torch.Tensor, scale: torch.Tensor,
                            output_type: torch.dtype = torch.float8_e4m3fn) -> torch.Tensor:
    """FP8 quantize with one fp32 scale: fp8(clamp(x * (1/scale), +-max))."""
    return torch.ops.comfy_kitchen.quantize_fp8(x, scale, DTYPE_TO_CODE[output_type])


def dequantize_per_tensor_fp8(x: torch.Tensor, scale: torch.Tensor,
                              output_type: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """FP8 dequantize: x.to(output_type) * scale.to(output_type)."""
    return torch.ops.comfy_kitchen.dequantize_fp8(x, scale, DTYPE_TO_CODE[output_type])


def stochastic_rounding_fp8(x: torch.Tensor, rng: torch.Tensor,
                            output_type: torch.dtype = torch.float8_e4m3fn) -> torch.Tensor:
    """Stochastic FP8 rounding.  Not provided by the hip backend (raises NoCapableBackendError)."""
    kwargs = {"x": x, "rng": rng, "output_type": output_type}
    return registry.get_implementation("stochastic_rounding_fp8", kwargs=kwargs)(**kwargs)


def quantize_nvfp4(x: torch.Tensor, per_tensor_scale: torch.Tensor, epsilon: float = 0.0,
                   pad_16x: bool = False, hi_first: bool = True) -> tuple[torch.Tensor, torch.Tensor]:
    """NVFP4: packed E2M1 codes [M, K/2] uint8 and swizzled E4M3 block-16 scales."""
    return torch.ops.comfy_kitchen.quantize_nvfp4(x, per_tensor_scale, epsilon, pad_16x, hi_first)


def quantize_nvfp4_dynamic(x: torch.Tensor, divisor: float = 448.0 * 6.0, pad_16x: bool = False,
                           hi_first: bool = True) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """quantize_nvfp4 with the per-tensor scale amax(|x|) / divisor (in x's dtype) formed on
    the device in the same call: returns (codes, block scales, 0-dim fp32 scale).

    Not part of the reference's public API: it is the scale=None branch of the NVFP4
    layout's quantize (reference tensor/nvfp4.py:64-69, the dynamic activation scale of
    samples/nvfp4_linear.py:55-59) with the reduction fused into the quantize launch.
    The results equal amax_scale followed by quantize_nvfp4 bit for bit."""
    return torch.ops.comfy_kitchen.quantize_nvfp4_dynamic(x, float(divisor), pad_16x, hi_first)


def dequantize_nvfp4(qx: torch.Tensor, per_tensor_scale: torch.Tensor, block_scales: torch.Tensor,
                     output_type: torch.dtype = torch.bfloat16, hi_first: bool = True) -> torch.Tensor:
    return torch.ops.comfy_kitchen.dequantize_nvfp4(
        qx, per_tensor_scale, block_scales, DTYPE_TO_CODE[output_type], hi_first)


def scaled_mm_nvfp4(a: torch.Tensor, b: torch.Tensor, tensor_scale_a: torch.Tensor,
                    tensor_scale_b: torch.Tensor, block_scale_a: torch.Tensor,
                    block_scale_b: torch.Tensor, bias: torch.Tensor | None = None,
                    out_dtype: torch.dtype | None = None,
                    alpha: torch.Tensor | None = None) -> torch.Tensor:
    """y = (a @ b.T) * (tensor_scale_a * tensor_scale_b) + bias on NVFP4 operands."""
    code = DTYPE_TO_CODE[out_dtype if out_dtype is not None else torch.bfloat16]
    return torch.ops.comfy_kitchen.scaled_mm_nvfp4(
        a, b, tensor_scale_a, tensor_scale_b, block_scale_a, block_scale_b, bias, code, alpha)


def quantize_mxfp8(x: torch.Tensor, pad_32x: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """MXFP8: E4M3 codes [M, K] and swizzled E8M0 block-32 scales."""
    return torch.ops.comfy_kitchen.quantize_mxfp8(x, pad_32x)


def dequantize_mxfp8(qx: torch.Tensor, block_scales: torch.Tensor,
                     output_type: torch.dtype = torch.bfloat16) -> torch.Tensor:
    return torch.ops.comfy_kitchen.dequantize_mxfp8(qx, block_scales, DTYPE_TO_CODE[output_type])


def scaled_mm_mxfp8(a: torch.Tensor, b: torch.Tensor, block_scale_a: torch.Tensor,
                    block_scale_b: torch.Tensor, bias: torch.Tensor | None = None,
                    out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """y = a @ b.T + bias on MXFP8 operands (both K-major, E8M0 block-32 scales)."""
    code = DTYPE_TO_CODE[out_dtype if out_dtype is not None else torch.bfloat16]
    return torch.ops.comfy_kitchen.scaled_mm_mxfp8(a, b, block_scale_a, block_scale_b, bias, code)


def scaled_mm_fp8(a: torch.Tensor, b: torch.Tensor, scale_a: torch.Tensor, scale_b: torch.Tensor,
                  bias: torch.Tensor | None = None, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """y = scale_a * scale_b * (a @ b.T) + bias on per-tensor E4M3 operands (both K-major).

    Not part of the reference's public API: it is the matmul behind TensorCoreFP8Layout's
    linear / mm / addmm, where the reference calls torch F.scaled_mm (scaled_mm_v2.py:27-53).
    """
    code = DTYPE_TO_CODE[out_dtype if out_dtype is not None else torch.bfloat16]
    return torch.ops.comfy_kitchen.scaled_mm_fp8(a, b, scale_a, scale_b, bias, code)


def apply_rope(xq: torch.Tensor, xk: torch.Tensor,
               freqs_cis: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Rotate query and key by the 2x2 matrices in freqs_cis [..., head_dim/2, 2, 2]."""
    return torch.ops.comfy_kitchen.apply_rope(xq, xk, freqs_cis)


def apply_rope1(x: torch.Tensor, freqs_cis: torch.Tensor) -> torch.Tensor:
    return torch.ops.comfy_kitchen.apply_rope1(x, freqs_cis)


def set_backend_priority(priority: list[str]) -> None:
    registry.set_priority(priority)


def disable_backend(name: str) -> None:
    registry.disable(name)


def enable_backend(name: str) -> None:
    registry.enable(name)


def list_backends() -> dict:
    return registry.list_backends()


def use_backend(name: str):
    return registry.use_backend(name)
