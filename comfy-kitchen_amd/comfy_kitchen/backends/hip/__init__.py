"""The "hip" backend: gfx950 kernels from libckh.so, called through its C ABI.

Role and contract follow the reference's CUDA backend (backends/cuda/__init__.py):
module-level functions with the eager backend's keyword arguments, outputs allocated
here with torch (the C side never allocates), launches on torch's current stream
(reference __init__.py:152), and per-function constraints registered with the
registry (reference __init__.py:516-691).  The binding is ctypes over a plain C ABI
(include/ckh.h) instead of nanobind/DLPack: raw device pointers, int64 sizes, dtype
codes and the stream handle.

There is no fallback: if libckh.so is missing or the device is not gfx950 the
backend is marked unavailable with the reason, and every `ck.*` call raises
NoCapableBackendError naming it.
"""
from __future__ import annotations

import ctypes
import functools
import os
from pathlib import Path

import torch

from ...float_utils import roundup
from ...ops import DTYPE_TO_CODE

__all__ = [
    "amax_scale",
    "apply_rope",
    "apply_rope1",
    "dequantize_mxfp8",
    "dequantize_nvfp4",
    "dequantize_per_tensor_fp8",
    "quantize_mxfp8",
    "quantize_nvfp4",
    "quantize_nvfp4_dynamic",
    "quantize_per_tensor_fp8",
    "scaled_mm_fp8",
    "scaled_mm_mxfp8",
    "scaled_mm_nvfp4",
]

LIB_PATH = Path(os.environ.get("CKH_LIBRARY", Path(__file__).with_name("libckh.so")))
REQUIRED_ARCH = ("gfx950",)

_p, _i64, _i32, _f32, _u64 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_uint64

# C signatures, exactly as declared in include/ckh.h
SIGNATURES: dict[str, tuple] = {
    "ckh_abi_version": (_i32, []),
    "ckh_last_error": (ctypes.c_char_p, []),
    "ckh_quantize_fp8": (_i32, [_p, _p, _p, _i64, _i32, _i32, _u64]),
    "ckh_dequantize_fp8": (_i32, [_p, _p, _p, _i64, _i32, _i32, _i32, _u64]),
    "ckh_quantize_mxfp8": (_i32, [_p, _p, _p, _i64, _i64, _i64, _i64, _i32, _u64]),
    "ckh_dequantize_mxfp8": (_i32, [_p, _p, _p, _i64, _i64, _i32, _u64]),
    "ckh_quantize_nvfp4": (_i32, [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _f32, _i32, _i32, _u64]),
    "ckh_dequantize_nvfp4": (_i32, [_p, _p, _p, _p, _i64, _i64, _i32, _i32, _u64]),
    "ckh_apply_rope": (_i32, [_p, _p, _p, _p, _p] + [_i64] * 13 + [_i32, _i32, _u64]),
    "ckh_scaled_mm_workspace_bytes": (_i64, [_i64] * 3),
    "ckh_scaled_mm_mxfp8": (_i32, [_p] * 6 + [_i64] * 3 + [_i32, _i32, _p, _i64, _u64]),
    "ckh_scaled_mm_fp8": (_i32, [_p] * 6 + [_i64] * 3 + [_i32, _i32, _p, _i64, _u64]),
    "ckh_scaled_mm_nvfp4": (_i32, [_p] * 7 + [_i64] * 3 + [_i32, _i32, _p, _i64, _u64]),
    "ckh_scaled_mm_nvfp4_workspace_bytes": (_i64, [_i64] * 3),
    "ckh_amax_scale": (_i32, [_p, _i64, _i32, _f32, _p, _p, _u64]),
    "ckh_amax_scale_noalloc": (_i32, [_p, _i64, _i32, _f32, _p, _u64]),
    "ckh_quantize_nvfp4_dynamic": (_i32, [_p, _f32, _p, _p, _p, _i64, _i64, _i64, _i64, _f32, _i32, _i32, _p, _u64]),
}
ABI_VERSION = 8
# CKH_AMAX_WORKSPACE_BYTES of include/ckh.h: the workspace ckh_amax_scale takes
AMAX_WORKSPACE_BYTES = 8192

_lib: ctypes.CDLL | None = None


def load_library(path: Path | str | None = None) -> ctypes.CDLL:
    """Load libckh.so and bind every entry point's signature (no GPU needed).

    torch is imported first (module import above), so the library binds to torch's
    HIP runtime: both carry the SONAME libamdhip64.so.7 and the loader reuses it.
    """
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise OSError(f"{p} not found: build it with `python comfy-kitchen_amd/build.py`")
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    if lib.ckh_abi_version() != ABI_VERSION:
        raise OSError(f"{p}: ABI version {lib.ckh_abi_version()} != expected {ABI_VERSION}")
    if path is None:
        _lib = lib
    return lib


def _call(name: str, *args) -> None:
    status = getattr(_lib, name)(*args)
    if status != 0:
        raise RuntimeError(f"{name}: {_lib.ckh_last_error().decode(errors='replace')}")


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


class _on_device:
    """Make t's device current for the launch (a no-op when it already is)."""

    def __init__(self, t: torch.Tensor):
        self.idx = t.device.index
        self.prev = None

    def __enter__(self):
        cur = torch.cuda.current_device()
        if self.idx is not None and self.idx != cur:
            self.prev = cur
            torch.cuda.set_device(self.idx)

    def __exit__(self, *exc):
        if self.prev is not None:
            torch.cuda.set_device(self.prev)


def _scalar_on(t: torch.Tensor | float, device: torch.device, name: str) -> torch.Tensor:
    """A one-element fp32 tensor on `device` (moving a host scalar if needed)."""
    if not isinstance(t, torch.Tensor):
        t = torch.tensor(float(t), dtype=torch.float32)
    if t.numel() != 1:
        raise ValueError(f"{name} must have exactly one element, got shape {tuple(t.shape)}")
    if t.dtype != torch.float32:
        t = t.to(torch.float32)
    if t.device != device:
        t = t.to(device)
    return t.reshape(1).contiguous()


def _scalar_keep(t: torch.Tensor, device: torch.device, name: str) -> torch.Tensor:
    """A one-element tensor of t's own float dtype on `device`: the kernel reads and widens
    it, as eager's scale.to(out dtype) does."""
    if not isinstance(t, torch.Tensor) or t.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        return _scalar_on(t, device, name)
    if t.numel() != 1:
        raise ValueError(f"{name} must have exactly one element, got shape {tuple(t.shape)}")
    if t.device != device:
        t = t.to(device)
    return t.reshape(1).contiguous()


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


# ------------------------------------------------------------------ per-tensor FP8
def quantize_per_tensor_fp8(x: torch.Tensor, scale: torch.Tensor,
                            output_type: torch.dtype = torch.float8_e4m3fn) -> torch.Tensor:
    x = x.contiguous()
    s = _scalar_on(scale, x.device, "scale")
    out = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    with _on_device(x):
        _call("ckh_quantize_fp8", x.data_ptr(), out.data_ptr(), s.data_ptr(), x.numel(),
              DTYPE_TO_CODE[x.dtype], DTYPE_TO_CODE[output_type], _stream(x))
    return out.view(output_type)


def dequantize_per_tensor_fp8(x: torch.Tensor, scale: torch.Tensor,
                              output_type: torch.dtype = torch.bfloat16) -> torch.Tensor:
    x = x.contiguous()
    s = _scalar_keep(scale, x.device, "scale")
    out = torch.empty(x.shape, dtype=output_type, device=x.device)
    with _on_device(x):
        _call("ckh_dequantize_fp8", x.data_ptr(), out.data_ptr(), s.data_ptr(), x.numel(),
              DTYPE_TO_CODE[x.dtype], DTYPE_TO_CODE[output_type], DTYPE_TO_CODE[s.dtype], _stream(x))
    return out


def amax_scale(x: torch.Tensor, divisor: float) -> torch.Tensor:
    """amax(|x|) / divisor computed in x's dtype, as a 0-dim fp32 tensor on x's device
    (the layouts' default scale, reference tensor/fp8.py:56-61, tensor/nvfp4.py:64-69)."""
    x = x.contiguous()
    if x.numel() == 0:
        raise RuntimeError("amax_scale: empty tensor")
    out = torch.empty((), dtype=torch.float32, device=x.device)
    # per-workgroup partial maxima (CKH_AMAX_WORKSPACE_BYTES), from torch's allocator
    work = torch.empty(AMAX_WORKSPACE_BYTES // 4, dtype=torch.int32, device=x.device)
    with _on_device(x):
        _call("ckh_amax_scale", x.data_ptr(), x.numel(), DTYPE_TO_CODE[x.dtype], float(divisor), out.data_ptr(),
              work.data_ptr(), _stream(x))
    return out


# --------------------------------------------------------------------------- MXFP8
def quantize_mxfp8(x: torch.Tensor, pad_32x: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    if x.dim() != 2:
        raise ValueError(f"quantize_mxfp8 expects a 2-D tensor, got {x.dim()}-D")
    x = x.contiguous()
    orows, ocols = x.shape
    rows, cols = (roundup(orows, 32), roundup(ocols, 32)) if pad_32x else (orows, ocols)
    if cols % 32:
        raise ValueError(f"K dimension must be divisible by 32 (got {cols}); pass pad_32x=True")
    qx = torch.empty((rows, cols), dtype=torch.float8_e4m3fn, device=x.device)
    sx = torch.empty((roundup(rows, 128), roundup(cols // 32, 4)), dtype=torch.uint8, device=x.device)
    with _on_device(x):
        _call("ckh_quantize_mxfp8", x.data_ptr(), qx.data_ptr(), sx.data_ptr(), rows, cols, orows, ocols,
              DTYPE_TO_CODE[x.dtype], _stream(x))
    return qx, sx.view(torch.float8_e8m0fnu)


def dequantize_mxfp8(qx: torch.Tensor, block_scales: torch.Tensor,
                     output_type: torch.dtype = torch.bfloat16) -> torch.Tensor:
    qx = qx.contiguous()
    rows, cols = qx.shape
    sc = block_scales.contiguous().view(torch.uint8)
    need = roundup(rows, 128) * roundup(cols // 32, 4)
    if cols % 32 or sc.numel() < need:
        raise ValueError(f"dequantize_mxfp8: qx {tuple(qx.shape)} needs K % 32 == 0 and {need} scale bytes, "
                         f"got {sc.numel()}")
    out = torch.empty((rows, cols), dtype=output_type, device=qx.device)
    with _on_device(qx):
        _call("ckh_dequantize_mxfp8", qx.data_ptr(), sc.data_ptr(), out.data_ptr(), rows, cols,
              DTYPE_TO_CODE[output_type], _stream(qx))
    return out


# --------------------------------------------------------------------------- NVFP4
def quantize_nvfp4(x: torch.Tensor, per_tensor_scale: torch.Tensor, epsilon: float = 0.0,
                   pad_16x: bool = False, hi_first: bool = True) -> tuple[torch.Tensor, torch.Tensor]:
    if x.dim() != 2:
        raise ValueError(f"quantize_nvfp4 expects a 2-D tensor, got {x.dim()}-D")
    x = x.contiguous()
    g = _scalar_on(per_tensor_scale, x.device, "per_tensor_scale")
    orows, ocols = x.shape
    rows, cols = (roundup(orows, 16), roundup(ocols, 16)) if pad_16x else (orows, ocols)
    if cols % 16:
        raise ValueError(f"K dimension must be divisible by 16 (got {cols}); pass pad_16x=True")
    qx = torch.empty((rows, cols // 2), dtype=torch.uint8, device=x.device)
    sx = torch.empty((roundup(rows, 128), roundup(cols // 16, 4)), dtype=torch.uint8, device=x.device)
    with _on_device(x):
        _call("ckh_quantize_nvfp4", x.data_ptr(), g.data_ptr(), qx.data_ptr(), sx.data_ptr(), rows, cols,
              orows, ocols, float(epsilon), DTYPE_TO_CODE[x.dtype], int(bool(hi_first)), _stream(x))
    return qx, sx.view(torch.float8_e4m3fn)


def quantize_nvfp4_dynamic(x: torch.Tensor, divisor: float, pad_16x: bool = False,
                           hi_first: bool = True) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """quantize_nvfp4 with the scale amax(|x|) / divisor formed on the device in the same
    pass: (codes, block scales, 0-dim fp32 scale), equal to amax_scale + quantize_nvfp4."""
    if x.dim() != 2:
        raise ValueError(f"quantize_nvfp4 expects a 2-D tensor, got {x.dim()}-D")
    x = x.contiguous()
    if x.numel() == 0:
        raise RuntimeError("quantize_nvfp4_dynamic: empty tensor")
    orows, ocols = x.shape
    rows, cols = (roundup(orows, 16), roundup(ocols, 16)) if pad_16x else (orows, ocols)
    if cols % 16:
        raise ValueError(f"K dimension must be divisible by 16 (got {cols}); pass pad_16x=True")
    qx = torch.empty((rows, cols // 2), dtype=torch.uint8, device=x.device)
    sx = torch.empty((roundup(rows, 128), roundup(cols // 16, 4)), dtype=torch.uint8, device=x.device)
    scale = torch.empty((), dtype=torch.float32, device=x.device)
    work = torch.empty(AMAX_WORKSPACE_BYTES // 4, dtype=torch.int32, device=x.device)
    with _on_device(x):
        _call("ckh_quantize_nvfp4_dynamic", x.data_ptr(), float(divisor), scale.data_ptr(), qx.data_ptr(),
              sx.data_ptr(), rows, cols, orows, ocols, 0.0, DTYPE_TO_CODE[x.dtype], int(bool(hi_first)),
              work.data_ptr(), _stream(x))
    return qx, sx.view(torch.float8_e4m3fn), scale


def dequantize_nvfp4(qx: torch.Tensor, per_tensor_scale: torch.Tensor, block_scales: torch.Tensor,
                     output_type: torch.dtype = torch.bfloat16, hi_first: bool = True) -> torch.Tensor:
    qx = qx.contiguous()
    rows, half = qx.shape
    cols = 2 * half
    g = _scalar_on(per_tensor_scale, qx.device, "per_tensor_scale")
    sc = block_scales.contiguous().view(torch.uint8)
    need = roundup(rows, 128) * roundup(cols // 16, 4)
    if cols % 16 or sc.numel() < need:
        raise ValueError(f"dequantize_nvfp4: qx {tuple(qx.shape)} needs K % 16 == 0 and {need} scale bytes, "
                         f"got {sc.numel()}")
    out = torch.empty((rows, cols), dtype=output_type, device=qx.device)
    with _on_device(qx):
        _call("ckh_dequantize_nvfp4", qx.data_ptr(), g.data_ptr(), sc.data_ptr(), out.data_ptr(), rows, cols,
              DTYPE_TO_CODE[output_type], int(bool(hi_first)), _stream(qx))
    return out


# ---------------------------------------------------------------------------- GEMMs
def _bias_args(bias: torch.Tensor | None, n: int, device) -> tuple[torch.Tensor | None, int]:
    if bias is None or bias.numel() == 0:
        return None, 0
    if bias.numel() != n:
        raise ValueError(f"bias must have {n} elements, got {bias.numel()}")
    b = bias.detach().reshape(-1).contiguous()
    if b.device != device:
        b = b.to(device)
    if b.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        b = b.to(torch.float32)
    return b, DTYPE_TO_CODE[b.dtype]


@functools.lru_cache(maxsize=256)
def _split_workspace_bytes(fn: str, m: int, n: int, k: int) -> int:
    return int(getattr(_lib, fn)(m, n, k))


def _gemm_workspace(m: int, n: int, k: int, device: torch.device,
                    fn: str = "ckh_scaled_mm_workspace_bytes") -> tuple[torch.Tensor | None, int]:
    """The workspace a GEMM splits K in at this shape (small tile grids), from torch's
    allocator (graph-capture safe), or (None, 0)."""
    nbytes = _split_workspace_bytes(fn, m, n, k)
    if nbytes <= 0:
        return None, 0
    return torch.empty(nbytes, dtype=torch.uint8, device=device), nbytes


def scaled_mm_mxfp8(a: torch.Tensor, b: torch.Tensor, block_scale_a: torch.Tensor,
                    block_scale_b: torch.Tensor, bias: torch.Tensor | None = None,
                    out_dtype: torch.dtype | None = None) -> torch.Tensor:
    out_dtype = out_dtype or torch.bfloat16
    a, b = a.contiguous(), b.contiguous()
    m, k = a.shape
    n, kb = b.shape
    if k != kb:
        raise ValueError(f"scaled_mm_mxfp8: K mismatch {k} vs {kb}")
    sa = block_scale_a.contiguous().view(torch.uint8)
    sb = block_scale_b.contiguous().view(torch.uint8)
    for name, s, rows in (("block_scale_a", sa, m), ("block_scale_b", sb, n)):
        need = roundup(rows, 128) * roundup(k // 32, 4)
        if s.numel() < need:
            raise ValueError(f"scaled_mm_mxfp8: {name} has {s.numel()} bytes, needs {need}")
    bias_t, bias_code = _bias_args(bias, n, a.device)
    out = torch.empty((m, n), dtype=out_dtype, device=a.device)
    ws, ws_bytes = _gemm_workspace(m, n, k, a.device)
    with _on_device(a):
        _call("ckh_scaled_mm_mxfp8", a.data_ptr(), b.data_ptr(), sa.data_ptr(), sb.data_ptr(), _ptr(bias_t),
              out.data_ptr(), m, n, k, DTYPE_TO_CODE[out_dtype], bias_code, _ptr(ws), ws_bytes, _stream(a))
    return out


def scaled_mm_fp8(a: torch.Tensor, b: torch.Tensor, scale_a: torch.Tensor, scale_b: torch.Tensor,
                  bias: torch.Tensor | None = None, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    out_dtype = out_dtype or torch.bfloat16
    a, b = a.contiguous(), b.contiguous()
    m, k = a.shape
    n, kb = b.shape
    if k != kb:
        raise ValueError(f"scaled_mm_fp8: K mismatch {k} vs {kb}")
    sa = _scalar_on(scale_a, a.device, "scale_a")
    sb = _scalar_on(scale_b, a.device, "scale_b")
    bias_t, bias_code = _bias_args(bias, n, a.device)
    out = torch.empty((m, n), dtype=out_dtype, device=a.device)
    ws, ws_bytes = _gemm_workspace(m, n, k, a.device)
    with _on_device(a):
        _call("ckh_scaled_mm_fp8", a.data_ptr(), b.data_ptr(), sa.data_ptr(), sb.data_ptr(), _ptr(bias_t),
              out.data_ptr(), m, n, k, DTYPE_TO_CODE[out_dtype], bias_code, _ptr(ws), ws_bytes, _stream(a))
    return out


def scaled_mm_nvfp4(a: torch.Tensor, b: torch.Tensor, tensor_scale_a: torch.Tensor,
                    tensor_scale_b: torch.Tensor, block_scale_a: torch.Tensor,
                    block_scale_b: torch.Tensor, bias: torch.Tensor | None = None,
                    out_dtype: torch.dtype | None = None,
                    alpha: torch.Tensor | None = None) -> torch.Tensor:
    out_dtype = out_dtype or torch.bfloat16
    a, b = a.contiguous(), b.contiguous()
    m, ka = a.shape
    n, kb = b.shape
    if ka != kb:
        raise ValueError(f"scaled_mm_nvfp4: K mismatch {2 * ka} vs {2 * kb}")
    k = 2 * ka
    if alpha is None:
        alpha = _scalar_on(tensor_scale_a, a.device, "tensor_scale_a") * _scalar_on(tensor_scale_b, a.device,
                                                                                    "tensor_scale_b")
    alpha = _scalar_on(alpha, a.device, "alpha")
    sa = block_scale_a.contiguous().view(torch.uint8)
    sb = block_scale_b.contiguous().view(torch.uint8)
    for name, s, rows in (("block_scale_a", sa, m), ("block_scale_b", sb, n)):
        need = roundup(rows, 128) * roundup(k // 16, 4)
        if s.numel() < need:
            raise ValueError(f"scaled_mm_nvfp4: {name} has {s.numel()} bytes, needs {need}")
    bias_t, bias_code = _bias_args(bias, n, a.device)
    out = torch.empty((m, n), dtype=out_dtype, device=a.device)
    ws, ws_bytes = _gemm_workspace(m, n, k, a.device, "ckh_scaled_mm_nvfp4_workspace_bytes")
    with _on_device(a):
        _call("ckh_scaled_mm_nvfp4", a.data_ptr(), b.data_ptr(), sa.data_ptr(), sb.data_ptr(), alpha.data_ptr(),
              _ptr(bias_t), out.data_ptr(), m, n, k, DTYPE_TO_CODE[out_dtype], bias_code, _ptr(ws), ws_bytes,
              _stream(a))
    return out


# ----------------------------------------------------------------------------- RoPE
def _rope_call(xq: torch.Tensor, xk: torch.Tensor | None, freqs_cis: torch.Tensor):
    if xq.dim() != 4 or freqs_cis.dim() != 6:
        raise ValueError(f"apply_rope expects 4-D x and 6-D freqs, got {xq.dim()}-D and {freqs_cis.dim()}-D")
    xq = xq.contiguous()
    xk = xk.contiguous() if xk is not None else None
    b, d1, d2, hd = xq.shape
    fb, fd1, fd2 = freqs_cis.shape[:3]
    if tuple(freqs_cis.shape[3:]) != (hd // 2, 2, 2) or hd % 2:
        raise ValueError(f"freqs_cis inner dims {tuple(freqs_cis.shape[3:])} != ({hd // 2}, 2, 2)")
    if d2 == 1 and fd2 != 1:
        raise ValueError(f"x dim 2 is 1 but freqs dim 2 is {fd2}: shapes do not broadcast back to x")
    f = freqs_cis
    if f.device != xq.device:
        f = f.to(xq.device)
    if f.stride(5) != 1 or f.stride(4) != 2 or f.stride(3) != 4:
        f = f.contiguous()
    oq = torch.empty_like(xq)
    ok = torch.empty_like(xk) if xk is not None else None
    with _on_device(xq):
        _call("ckh_apply_rope", xq.data_ptr(), _ptr(xk), f.data_ptr(), oq.data_ptr(), _ptr(ok), b, d1, d2, hd,
              fb, fd1, fd2, xq.stride(0), xq.stride(1), xq.stride(2), f.stride(0), f.stride(1), f.stride(2),
              DTYPE_TO_CODE[xq.dtype], DTYPE_TO_CODE[f.dtype], _stream(xq))
    return oq, ok


def apply_rope1(x: torch.Tensor, freqs_cis: torch.Tensor) -> torch.Tensor:
    return _rope_call(x, None, freqs_cis)[0]


def apply_rope(xq: torch.Tensor, xk: torch.Tensor, freqs_cis: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    if xq.shape != xk.shape or xq.dtype != xk.dtype:
        return apply_rope1(xq, freqs_cis), apply_rope1(xk, freqs_cis)
    return _rope_call(xq, xk, freqs_cis)


# ---------------------------------------------------------------------- registration
def _build_constraints() -> dict:
    from ...constraints import DivisibleBy, ExactDims, FunctionConstraints, ParamConstraint

    dev = frozenset({"cuda"})
    floats = frozenset({torch.float32, torch.float16, torch.bfloat16})
    half = frozenset({torch.float16, torch.bfloat16})
    fp8 = frozenset({torch.float8_e4m3fn, torch.float8_e5m2})
    f32 = frozenset({torch.float32})

    def fc(**params):
        return FunctionConstraints(params=params, default_devices=dev, required_arch=REQUIRED_ARCH)

    two_d = (ExactDims(2),)
    return {
        "amax_scale": fc(x=ParamConstraint(dtypes=floats)),
        "quantize_per_tensor_fp8": fc(x=ParamConstraint(dtypes=floats), scale=ParamConstraint(dtypes=f32, devices=frozenset({"cuda", "cpu"})),
                                      output_type=ParamConstraint(dtypes=fp8)),
        "dequantize_per_tensor_fp8": fc(x=ParamConstraint(dtypes=fp8), scale=ParamConstraint(dtypes=floats, devices=frozenset({"cuda", "cpu"})),
                                        output_type=ParamConstraint(dtypes=floats)),
        "quantize_mxfp8": fc(x=ParamConstraint(dtypes=floats, shape_rules=two_d)),
        "dequantize_mxfp8": fc(qx=ParamConstraint(dtypes=frozenset({torch.float8_e4m3fn}),
                                                  shape_rules=two_d + (DivisibleBy(1, 32),)),
                               block_scales=ParamConstraint(dtypes=frozenset({torch.float8_e8m0fnu})),
                               output_type=ParamConstraint(dtypes=floats)),
        "quantize_nvfp4": fc(x=ParamConstraint(dtypes=floats, shape_rules=two_d),
                             per_tensor_scale=ParamConstraint(dtypes=f32, devices=frozenset({"cuda", "cpu"}))),
        "quantize_nvfp4_dynamic": fc(x=ParamConstraint(dtypes=floats, shape_rules=two_d)),
        "dequantize_nvfp4": fc(qx=ParamConstraint(dtypes=frozenset({torch.uint8}),
                                                  shape_rules=two_d + (DivisibleBy(1, 8),)),
                               per_tensor_scale=ParamConstraint(dtypes=f32, devices=frozenset({"cuda", "cpu"})),
                               block_scales=ParamConstraint(dtypes=frozenset({torch.float8_e4m3fn})),
                               output_type=ParamConstraint(dtypes=floats)),
        "scaled_mm_mxfp8": fc(a=ParamConstraint(dtypes=frozenset({torch.float8_e4m3fn}),
                                                shape_rules=two_d + (DivisibleBy(1, 32),)),
                              b=ParamConstraint(dtypes=frozenset({torch.float8_e4m3fn}),
                                                shape_rules=two_d + (DivisibleBy(1, 32),)),
                              block_scale_a=ParamConstraint(dtypes=frozenset({torch.float8_e8m0fnu})),
                              block_scale_b=ParamConstraint(dtypes=frozenset({torch.float8_e8m0fnu})),
                              bias=ParamConstraint(dtypes=floats),
                              out_dtype=ParamConstraint(dtypes=floats)),
        "scaled_mm_fp8": fc(a=ParamConstraint(dtypes=frozenset({torch.float8_e4m3fn}),
                                              shape_rules=two_d + (DivisibleBy(1, 16),)),
                            b=ParamConstraint(dtypes=frozenset({torch.float8_e4m3fn}),
                                              shape_rules=two_d + (DivisibleBy(1, 16),)),
                            scale_a=ParamConstraint(dtypes=f32, devices=frozenset({"cuda", "cpu"})),
                            scale_b=ParamConstraint(dtypes=f32, devices=frozenset({"cuda", "cpu"})),
                            bias=ParamConstraint(dtypes=floats),
                            out_dtype=ParamConstraint(dtypes=floats)),
        "scaled_mm_nvfp4": fc(a=ParamConstraint(dtypes=frozenset({torch.uint8}),
                                                shape_rules=two_d + (DivisibleBy(1, 16),)),
                              b=ParamConstraint(dtypes=frozenset({torch.uint8}),
                                                shape_rules=two_d + (DivisibleBy(1, 16),)),
                              tensor_scale_a=ParamConstraint(dtypes=f32, devices=frozenset({"cuda", "cpu"})),
                              tensor_scale_b=ParamConstraint(dtypes=f32, devices=frozenset({"cuda", "cpu"})),
                              block_scale_a=ParamConstraint(dtypes=frozenset({torch.float8_e4m3fn})),
                              block_scale_b=ParamConstraint(dtypes=frozenset({torch.float8_e4m3fn})),
                              bias=ParamConstraint(dtypes=floats),
                              out_dtype=ParamConstraint(dtypes=floats)),
        "apply_rope1": fc(x=ParamConstraint(dtypes=floats, shape_rules=(ExactDims(4),)),
                          freqs_cis=ParamConstraint(dtypes=floats, shape_rules=(ExactDims(6),))),
        "apply_rope": fc(xq=ParamConstraint(dtypes=floats, shape_rules=(ExactDims(4),)),
                         xk=ParamConstraint(dtypes=floats, shape_rules=(ExactDims(4),)),
                         freqs_cis=ParamConstraint(dtypes=floats, shape_rules=(ExactDims(6),))),
    }


def _register() -> None:
    from ...registry import registry

    try:
        load_library()
    except OSError as e:
        registry.mark_unavailable("hip", f"failed to load {LIB_PATH.name}: {e}")
        return
    if not torch.cuda.is_available() or torch.version.hip is None:
        registry.mark_unavailable("hip", "no ROCm GPU visible (torch.cuda.is_available() is False)")
        return
    arch = getattr(torch.cuda.get_device_properties(torch.cuda.current_device()), "gcnArchName", "")
    if not any(arch.startswith(a) for a in REQUIRED_ARCH):
        registry.mark_unavailable("hip", f"device arch {arch!r} is not one of {REQUIRED_ARCH}")
        return
    registry.register("hip", __import__(__name__, fromlist=__all__), _build_constraints())


_register()
