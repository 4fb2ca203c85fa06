"""CPU restatement of the reference's eager backend -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
module, and only as the checker (or as the timed CPU baseline).  The product path
(comfy_kitchen) never imports it and has no CPU fallback.

Each function restates the reference eager implementation op for op, with the same
torch CPU routines in the same order, so its results are the eager backend's:

  quantize_per_tensor_fp8    backends/eager/quantization.py:41-55
  dequantize_per_tensor_fp8  backends/eager/quantization.py:57-61
  quantize_nvfp4             backends/eager/quantization.py:115-160
  dequantize_nvfp4           backends/eager/quantization.py:171-219
  quantize_mxfp8             backends/eager/quantization.py:257-324
  dequantize_mxfp8           backends/eager/quantization.py:327-364
  f32_to_e2m1                float_utils.py:41-150 (ebits=2, mbits=1)
  pack_nibbles               float_utils.py:253-260
  to_blocked / from_blocked  float_utils.py:292-352
  e8m0_to_f32                float_utils.py:376-382
  apply_rope1 / apply_rope   backends/eager/rope.py:7-18
  default_scale              tensor/fp8.py:56-61, tensor/nvfp4.py:64-69 (as evaluated
                             on a GPU tensor: multiply by the fp32 reciprocal)
  scaled_mm_*_ref            closed form: fp32 matmul of the dequantized operands
                             (eager routes to torch F.scaled_mm, which has no CPU
                             kernel; quantization.py:222-246, 367-402)

How it is pinned (tests/test_oracle.py): against oracle/scalar_ref.c, an independent
scalar C implementation that rounds by brute-force nearest-value search rather than
bit tricks, exhaustively over every bf16 input pattern; against the golden vectors in
tests/golden/; and against closed-form invariants (swizzle round trips, nibble swap).
default_scale is also checked on the GPU against torch's own device kernel
(tests/test_gpu_quant.py), and dequantize_nvfp4's rounding of the block total in the
output dtype against hand-derived known answers and ref_dequantize_nvfp4_value.
"""
from __future__ import annotations

import numpy as np
import torch

F4_E2M1_MAX = 6.0
F8_E4M3_MAX = 448.0
F8_E5M2_MAX = 57344.0
E8M0_BIAS = 127


def roundup(x: int, m: int) -> int:
    return (x + m - 1) // m * m


# ------------------------------------------------------------------ layouts
def to_blocked(scales: torch.Tensor) -> torch.Tensor:
    """[R, C] -> swizzled [ceil(R/128)*128, ceil(C/4)*4] (float_utils.py:292-326).

    Padded [Rb*128, Cb*4] viewed as (rb, q, i, cb, c) with r = rb*128 + q*32 + i and
    col = cb*4 + c is stored in the order (rb, cb, i, q, c).
    """
    rows, cols = scales.shape
    rb, cb = -(-rows // 128), -(-cols // 4)
    pad = torch.zeros((rb * 128, cb * 4), dtype=scales.dtype)
    pad[:rows, :cols] = scales
    v = pad.view(rb, 4, 32, cb, 4).permute(0, 3, 2, 1, 4).contiguous()
    return v.reshape(rb * 128, cb * 4)


def from_blocked(blocked: torch.Tensor, num_rows: int, num_cols: int) -> torch.Tensor:
    """Inverse of to_blocked, dropping padding (float_utils.py:329-352)."""
    rb, cb = -(-num_rows // 128), -(-num_cols // 4)
    v = blocked.reshape(rb, cb, 32, 4, 4).permute(0, 3, 2, 1, 4).contiguous()
    return v.reshape(rb * 128, cb * 4)[:num_rows, :num_cols]


def e8m0_to_f32(x: torch.Tensor) -> torch.Tensor:
    e = x.to(torch.int32)
    return torch.where(e == 0, torch.zeros_like(e), e << 23).view(torch.float32)


# ------------------------------------------------------------- per-tensor FP8
def default_scale(x: torch.Tensor, max_value: float) -> torch.Tensor:
    """The layouts' default per-tensor scale (tensor/fp8.py:56-61, tensor/nvfp4.py:64-69):
    torch.amax(x.abs()) / max_value, a 0-dim tensor of x's dtype, then cast to fp32.

    Restated as torch evaluates it on the GPU tensor the layout holds: a true divide by a
    Python-scalar divisor runs as a multiply by the divisor's fp32 reciprocal in fp32 (the
    op-math type of f32/f16/bf16), rounded once to x's dtype.  torch's CPU kernel divides
    instead; the two agree on every bf16 amax but not on about half of fp32 amaxes or on
    39 tiny f16 amaxes (tests/golden/known_answers.json "default_scale" has examples).
    """
    amax = torch.amax(x.abs()).to(torch.float32)
    inv = torch.tensor(1.0, dtype=torch.float32) / torch.tensor(max_value, dtype=torch.float32)
    return (amax * inv).to(x.dtype).to(torch.float32)


def quantize_per_tensor_fp8(x: torch.Tensor, scale: torch.Tensor,
                            output_type: torch.dtype = torch.float8_e4m3fn) -> torch.Tensor:
    lp_max = F8_E4M3_MAX if output_type == torch.float8_e4m3fn else F8_E5M2_MAX
    t = x * (1.0 / scale).to(x.dtype)
    t = torch.clamp(t, -lp_max, lp_max, out=t)
    return t.to(output_type)


def dequantize_per_tensor_fp8(x: torch.Tensor, scale: torch.Tensor,
                              output_type: torch.dtype = torch.bfloat16) -> torch.Tensor:
    return x.to(dtype=output_type) * scale.to(dtype=output_type)


# -------------------------------------------------------------------- E2M1
def f32_to_e2m1(x: torch.Tensor) -> torch.Tensor:
    """fp32 -> E2M1 code in the low 4 bits, RNE, saturating at 6 (float_utils.py:41-150).

    Three cases on |x|: >= 6 saturates to code 7; < 1 (the smallest normal) is rounded
    to a multiple of 0.5 by adding 2^22 in fp32 (ulp 0.5) and subtracting it as an
    integer; otherwise the exponent is rebiased (127 -> 1) and the 23-bit mantissa is
    rounded to 1 bit, half to even.  The sign goes to bit 3.
    """
    assert x.dtype == torch.float32
    bits = x.view(torch.int32)
    sign = (bits >> 28) & 8  # bit 31 -> bit 3 (arithmetic shift, then mask)
    mag = (bits & 0x7FFFFFFF).view(torch.float32)
    sat = mag >= 6.0
    small = (~sat) & (mag < 1.0)
    magic = 149 << 23  # 2^22 as fp32 bits
    sub = ((mag + torch.tensor(magic, dtype=torch.int32).view(torch.float32)).view(torch.int32) - magic)
    m = mag.view(torch.int32)
    odd = (m >> 22) & 1
    norm = (m + (((1 - 127) << 23) + (1 << 21) - 1) + odd) >> 22
    code = torch.full_like(m, 7)
    code = torch.where(small, sub, code)
    code = torch.where(~(sat | small), norm, code)
    return (code | sign).to(torch.uint8)


def pack_nibbles(codes: torch.Tensor, hi_first: bool = True) -> torch.Tensor:
    flat = codes.contiguous().view(-1)
    even, odd = flat[0::2], flat[1::2]
    packed = (even << 4 | odd) if hi_first else (odd << 4 | even)
    return packed.view(*codes.shape[:-1], codes.shape[-1] // 2)


E2M1_VALUES = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]


# ------------------------------------------------------------------- NVFP4
def quantize_nvfp4(x: torch.Tensor, per_tensor_scale: torch.Tensor, epsilon: float = 0.0,
                   pad_16x: bool = False, hi_first: bool = True) -> tuple[torch.Tensor, torch.Tensor]:
    if pad_16x:
        rows, cols = x.shape
        pr, pc = roundup(rows, 16), roundup(cols, 16)
        if (pr, pc) != (rows, cols):
            x = torch.nn.functional.pad(x, (0, pc - cols, 0, pr - rows))
    shape = x.shape
    xb = x.reshape(shape[0], -1, 16)
    block_scale = torch.amax(torch.abs(xb), dim=-1).to(torch.float32) / F4_E2M1_MAX
    s = torch.clamp(block_scale / per_tensor_scale, max=F8_E4M3_MAX)
    s_rounded = s.to(torch.float8_e4m3fn).to(torch.float32)
    total = per_tensor_scale * s_rounded
    zero = total == 0
    safe = torch.where(zero, torch.ones_like(total), total)
    data = xb.float() / safe.unsqueeze(-1)
    data = torch.where(zero.unsqueeze(-1), torch.zeros_like(data), data)
    data = torch.clamp(data, -F4_E2M1_MAX, F4_E2M1_MAX).view(shape)
    q = pack_nibbles(f32_to_e2m1(data), hi_first=hi_first)
    return q, to_blocked(s.to(torch.float8_e4m3fn).view(torch.uint8)).view(torch.float8_e4m3fn)


def dequantize_nvfp4(qx: torch.Tensor, per_tensor_scale: torch.Tensor, block_scales: torch.Tensor,
                     output_type: torch.dtype = torch.bfloat16, hi_first: bool = True) -> torch.Tensor:
    lut = torch.tensor(E2M1_VALUES, dtype=output_type)
    hi, lo = (qx >> 4).long(), (qx & 15).long()
    first, second = (hi, lo) if hi_first else (lo, hi)
    codes = torch.stack([first, second], dim=-1).reshape(qx.shape[0], -1)
    vals = lut[codes]
    rows, cols = vals.shape
    s = from_blocked(block_scales.view(torch.uint8), rows, cols // 16).view(torch.float8_e4m3fn)
    total = per_tensor_scale.to(output_type) * s.to(output_type)
    return (vals.reshape(rows, -1, 16) * total.unsqueeze(-1)).view(rows, cols).to(output_type)


# ------------------------------------------------------------------- MXFP8
def quantize_mxfp8(x: torch.Tensor, pad_32x: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    assert x.dim() == 2
    if pad_32x:
        rows, cols = x.shape
        pr, pc = roundup(rows, 32), roundup(cols, 32)
        if (pr, pc) != (rows, cols):
            x = torch.nn.functional.pad(x, (0, pc - cols, 0, pr - rows))
    else:
        assert x.shape[1] % 32 == 0
    rows, cols = x.shape
    xb = x.reshape(rows, cols // 32, 32)
    amax = torch.amax(torch.abs(xb), dim=-1)
    s = torch.clamp(amax.float() / F8_E4M3_MAX, min=2 ** (-127))
    e = torch.ceil(torch.log2(s)).to(torch.int32) + E8M0_BIAS
    e = torch.clamp(e, 0, 254).to(torch.uint8)
    sf = e8m0_to_f32(e)
    zero = amax == 0
    sf = torch.where(zero, torch.ones_like(sf), sf)
    data = xb.float() / sf.unsqueeze(-1)
    data = torch.where(zero.unsqueeze(-1), torch.zeros_like(data), data)
    data = torch.clamp(data, -F8_E4M3_MAX, F8_E4M3_MAX).reshape(rows, cols).to(torch.float8_e4m3fn)
    e = torch.where(zero, torch.zeros_like(e), e)
    return data, to_blocked(e).view(torch.float8_e8m0fnu)


def dequantize_mxfp8(qx: torch.Tensor, block_scales: torch.Tensor,
                     output_type: torch.dtype = torch.bfloat16) -> torch.Tensor:
    rows, cols = qx.shape
    e = from_blocked(block_scales.view(torch.uint8), rows, cols // 32)
    data = qx.to(torch.float32).reshape(rows, cols // 32, 32) * e8m0_to_f32(e).unsqueeze(-1)
    return data.reshape(rows, cols).to(output_type)


# -------------------------------------------------------------------- RoPE
def apply_rope1(x: torch.Tensor, freqs_cis: torch.Tensor) -> torch.Tensor:
    x_ = x.to(dtype=freqs_cis.dtype).reshape(*x.shape[:-1], -1, 1, 2)
    if x_.shape[2] != 1 and freqs_cis.shape[2] != 1 and x_.shape[2] != freqs_cis.shape[2]:
        freqs_cis = freqs_cis[:, :, :x_.shape[2]]
    out = freqs_cis[..., 0] * x_[..., 0]
    out.addcmul_(freqs_cis[..., 1], x_[..., 1])
    return out.reshape(*x.shape).type_as(x)


def apply_rope(xq, xk, freqs_cis):
    return apply_rope1(xq, freqs_cis), apply_rope1(xk, freqs_cis)


# ------------------------------------------------------------------- GEMMs
def scaled_mm_mxfp8_ref(a, b, sa, sb, bias=None, out_dtype=torch.bfloat16):
    """fp32 matmul of the fp32-dequantized MXFP8 operands (+ bias)."""
    A = dequantize_mxfp8(a, sa, torch.float32)
    B = dequantize_mxfp8(b, sb, torch.float32)
    y = A @ B.t()
    if bias is not None:
        y = y + bias.float()
    return y.to(out_dtype)


def scaled_mm_nvfp4_ref(a, b, ts_a, ts_b, sa, sb, bias=None, out_dtype=torch.bfloat16):
    """fp32 matmul of the fp32-dequantized NVFP4 operands (+ bias)."""
    A = dequantize_nvfp4(a, ts_a, sa, torch.float32)
    B = dequantize_nvfp4(b, ts_b, sb, torch.float32)
    y = A @ B.t()
    if bias is not None:
        y = y + bias.float()
    return y.to(out_dtype)


# ------------------------------------------------------------ bit helpers
def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def all_bf16() -> torch.Tensor:
    """Every one of the 65,536 bf16 bit patterns, as a bf16 tensor."""
    return torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
