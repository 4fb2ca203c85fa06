"""Loader for tests/golden/known_answers.json (hand-derived known-answer vectors)."""
from __future__ import annotations

import json
from pathlib import Path

import torch

GOLDEN = Path(__file__).resolve().parent / "golden" / "known_answers.json"


def _load() -> dict:
    return json.loads(GOLDEN.read_text())


def _code(s):
    return int(s, 16)


def _expand(spec: dict, n: int, conv) -> list:
    out = [conv(spec["fill"])] * n
    for k, v in spec.get("set", {}).items():
        out[int(k)] = conv(v)
    return out


DTYPES = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}
BITS_VIEW = {torch.bfloat16: torch.int16, torch.float16: torch.int16, torch.float32: torch.int32}
VEC_LEN = 64  # per-tensor FP8 cases fill a tensor of this many elements (eager's vectorised loop)


def _from_bits(hexbits: str, dtype: torch.dtype, n: int) -> torch.Tensor:
    v = int(hexbits, 16)
    width = 32 if dtype == torch.float32 else 16
    if v >= 1 << (width - 1):
        v -= 1 << width
    return torch.full((n,), v, dtype=BITS_VIEW[dtype]).view(dtype)


def fp8_quant_cases():
    """(x [64] of the case's dtype, every element the case's value; scale f32 [1]; output
    dtype; expected code of every element)"""
    res = []
    for c in _load()["quantize_per_tensor_fp8"]:
        dt = torch.float8_e4m3fn if c["out"] == "e4m3" else torch.float8_e5m2
        xdt = DTYPES[c.get("dtype", "bf16")]
        x = _from_bits(c["x_bits"], xdt, VEC_LEN) if "x_bits" in c else torch.full((VEC_LEN,), c["x"], dtype=xdt)
        s = (_from_bits(c["scale_bits"], torch.float32, 1) if "scale_bits" in c
             else torch.tensor([c["scale"]], dtype=torch.float32))
        res.append((x, s, dt, int(c["code"], 16)))
    return res


def fp8_dequant_cases():
    """(codes uint8 [1] viewed as e4m3, scale f32 [1], expected bf16 bits)"""
    res = []
    for c in _load()["dequantize_per_tensor_fp8"]:
        q = torch.tensor([int(c["code"], 16)], dtype=torch.uint8).view(torch.float8_e4m3fn)
        res.append((q, torch.tensor([c["scale"]], dtype=torch.float32), int(c["bf16"], 16)))
    return res


def mxfp8_cases():
    """(block bf16 [32], expected scale byte, expected codes list[int])"""
    res = []
    for c in _load()["quantize_mxfp8"]:
        x = torch.tensor(_expand(c["block"], 32, float), dtype=torch.bfloat16)
        for k, v in c.get("block_bits", {}).items():
            x[int(k)] = _from_bits(v, torch.bfloat16, 1)[0]
        res.append((x, int(c["scale"], 16), _expand(c["codes"], 32, _code)))
    return res


def nvfp4_cases():
    """(block bf16 [16], g f32 [1], expected scale byte, expected unpacked codes)"""
    res = []
    for c in _load()["quantize_nvfp4"]:
        x = torch.tensor(c["block"], dtype=torch.bfloat16)
        res.append((x, torch.tensor([c["g"]], dtype=torch.float32), int(c["scale"], 16), list(c["codes"]),
                    [int(b, 16) for b in c.get("packed_hi_first", [])]))
    return res


def codes_match(got: list[int], want: list[int]) -> bool:
    """Byte-wise compare, NaN code bytes included (sign and all)."""
    return list(got) == list(want)


def unpack(packed: torch.Tensor, hi_first: bool = True) -> list[int]:
    out = []
    for b in packed.reshape(-1).tolist():
        hi, lo = b >> 4, b & 15
        out += [hi, lo] if hi_first else [lo, hi]
    return out


_CODES = {"f32": 0, "f16": 1, "bf16": 2}
_DTYPES = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def default_scale_cases():
    """(amax tensor [1] of the input dtype, dtype code, divisor, expected fp32 scale bits)"""
    res = []
    for c in _load()["default_scale"]:
        x = torch.tensor([c["amax"]], dtype=torch.float64).to(_DTYPES[c["dtype"]])
        assert float(x) == c["amax"], "known-answer amax must be exact in its dtype"
        res.append((x, _CODES[c["dtype"]], float(c["divisor"]), int(c["scale_bits"], 16)))
    return res


def dequantize_nvfp4_cases():
    """(output dtype, dtype code, g f32 [1], scale byte, E2M1 code, expected 16-bit output bits)"""
    res = []
    for c in _load()["dequantize_nvfp4"]:
        res.append((_DTYPES[c["out"]], _CODES[c["out"]], torch.tensor([c["g"]], dtype=torch.float32),
                    int(c["scale"], 16), int(c["code"]), int(c["value_bits"], 16)))
    return res


def nvfp4_block(code: int, scale_byte: int, hi_first: bool = True):
    """One NVFP4 block of 16 equal codes: packed [1, 8] uint8 and swizzled E4M3 [128, 4]."""
    q = torch.full((1, 8), (code << 4) | code, dtype=torch.uint8)
    s = torch.zeros(128, 4, dtype=torch.uint8)
    s[0, 0] = scale_byte  # logical (0, 0) is swizzled byte 0
    return q, s.view(torch.float8_e4m3fn)
