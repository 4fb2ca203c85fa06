"""Format constants and byte-layout utilities shared by the API and the layouts.

Public helpers kept from the reference API (comfy_kitchen/__init__.py:15):
`to_blocked`, `from_blocked`, `swap_nibbles`.  They are written here as index
arithmetic on the closed-form swizzle offset rather than as reshape/permute chains,
so the package and the test oracle compute the layout two independent ways.

Scale swizzle ("32_4_4", reference float_utils.py:292-352 and float_utils.cuh:110-125):
a logical scale matrix [R, C] is zero-padded to [ceil(R/128)*128, ceil(C/4)*4] and
stored as 512-byte chunks, chunk index (r // 128) * ceil(C/4) + c // 4; inside a
chunk the byte for (r, c) sits at (r % 32) * 16 + ((r % 128) // 32) * 4 + c % 4.
The four scales of one row for block-columns 4j..4j+3 therefore form one aligned
32-bit word, which is what the GEMM kernels load.
"""
from __future__ import annotations

import torch

F4_E2M1_MAX = 6.0
F4_E2M1_EPS = 0.5
F8_E4M3_MAX = 448.0
F8_E4M3_EPS = 0.125
F8_E5M2_MAX = 57344.0
F8_E5M2_EPS = 0.0625
E8M0_BIAS = 127


def roundup(x: int, multiple: int) -> int:
    return -(-x // multiple) * multiple


def ceil_div(a: int, b: int) -> int:
    return -(-a // b)


def swizzled_offset(r: torch.Tensor | int, c: torch.Tensor | int, n_col_blocks: int):
    """Byte offset of logical scale (r, c) in the 32_4_4 layout."""
    return (((r // 128) * n_col_blocks + c // 4) * 32 + r % 32) * 16 + ((r % 128) // 32) * 4 + c % 4


def _offsets(rows: int, cols: int, device) -> torch.Tensor:
    r = torch.arange(rows, device=device, dtype=torch.int64).unsqueeze(1)
    c = torch.arange(cols, device=device, dtype=torch.int64).unsqueeze(0)
    return swizzled_offset(r, c, ceil_div(cols, 4))


def _as_bytes(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.uint8) if t.element_size() == 1 and t.dtype != torch.uint8 else t


def to_blocked(input_matrix: torch.Tensor, flatten: bool = True) -> torch.Tensor:
    """Logical [R, C] scales -> swizzled layout ([Rp*Cp] if flatten else [Rp, Cp])."""
    rows, cols = input_matrix.shape
    prow, pcol = roundup(rows, 128), roundup(cols, 4)
    src = _as_bytes(input_matrix.contiguous())
    out = torch.zeros(prow * pcol, dtype=src.dtype, device=src.device)
    out[_offsets(rows, cols, src.device).reshape(-1)] = src.reshape(-1)
    out = out.view(input_matrix.dtype) if src.dtype != input_matrix.dtype else out
    return out if flatten else out.reshape(prow, pcol)


def from_blocked(blocked_matrix: torch.Tensor, num_rows: int, num_cols: int) -> torch.Tensor:
    """Swizzled scales -> logical [num_rows, num_cols] (padding dropped)."""
    src = _as_bytes(blocked_matrix.contiguous()).reshape(-1)
    out = src[_offsets(num_rows, num_cols, src.device)]
    return out.view(blocked_matrix.dtype) if src.dtype != blocked_matrix.dtype else out


def swap_nibbles(packed: torch.Tensor) -> torch.Tensor:
    """0xAB -> 0xBA for every byte: converts between hi_first=True/False packing."""
    return ((packed << 4) | (packed >> 4)).to(torch.uint8)


def pack_uint4(codes: torch.Tensor, hi_first: bool = True) -> torch.Tensor:
    """Pack 4-bit codes pairwise along the last dim; even element high if hi_first."""
    even, odd = codes[..., 0::2].to(torch.uint8), codes[..., 1::2].to(torch.uint8)
    return ((even << 4) | odd) if hi_first else ((odd << 4) | even)


def unpack_uint4(packed: torch.Tensor, hi_first: bool = True) -> torch.Tensor:
    hi, lo = packed >> 4, packed & 0x0F
    first, second = (hi, lo) if hi_first else (lo, hi)
    return torch.stack([first, second], dim=-1).reshape(*packed.shape[:-1], -1)


def e8m0_to_f32(x: torch.Tensor) -> torch.Tensor:
    """E8M0 byte e -> 2**(e-127), with e == 0 mapped to 0.0 (reference float_utils.py:376-382)."""
    e = x.view(torch.uint8).to(torch.int32)
    return torch.where(e == 0, torch.zeros_like(e), e << 23).view(torch.float32)
