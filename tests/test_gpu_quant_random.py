"""Seeded random shapes, dtypes and magnitudes through the quantizers and dequantizers,
against the CPU oracle, bit for bit.

The kernels choose their form by size and alignment: 16-byte vector paths where a row's
byte length allows them, scalar tails, padded scale rows (pad_32x / pad_16x), persistent
or one-shot grids, rows shorter than a workgroup's share.  Each case draws a row count, a
row length, an input dtype, padding and a per-row magnitude spread from ranges that
straddle those choices, so the suite crosses them in combinations the hand-picked shapes
do not.  Inputs are finite, so every dequantized value compares bit for bit.
"""
import random

import pytest
import torch

import comfy_kitchen as ck
from conftest import bits
from oracle import eager_ref as ref

pytestmark = pytest.mark.gpu

DTYPES = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def _cases(seed: int, count: int, kmul: int):
    """(m, k, dtype, pad, spread, seed): k a multiple of kmul unless padded."""
    rng = random.Random(seed)
    out = []
    for _ in range(count):
        m = rng.choice([rng.randint(1, 8), rng.randint(9, 300), rng.randint(300, 1200)])
        pad = rng.random() < 0.3
        k = rng.randint(1, 3000) if pad else kmul * rng.randint(1, 96)
        out.append((m, k, rng.choice(list(DTYPES)), pad, rng.choice([0.0, 1.0, 3.0]), rng.randrange(1 << 30)))
    return out


def _input(m: int, k: int, dtype: str, spread: float, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g) * torch.exp(torch.randn(m, 1, generator=g) * spread)
    if m * k >= 64:
        x.view(-1)[:32] = 0  # a zero block (or the start of one)
    return x.clamp(-6e4, 6e4).to(DTYPES[dtype])  # finite in f16 too


def _codes_equal(got: torch.Tensor, want: torch.Tensor, what: str):
    g, w = bits(got).reshape(-1), bits(want).reshape(-1)
    bad = g != w
    assert int(bad.sum()) == 0, (f"{what}: {int(bad.sum())} of {g.numel()} bytes differ, first at "
                                 f"{bad.nonzero()[:5].flatten().tolist()}")


@pytest.mark.parametrize("m,k,dtype,pad,spread,seed", _cases(31, 24, 32))
def test_mxfp8_random(m, k, dtype, pad, spread, seed, hip):
    x = _input(m, k, dtype, spread, seed)
    want_q, want_s = ref.quantize_mxfp8(x, pad_32x=pad)
    q, s = ck.quantize_mxfp8(x.cuda(), pad_32x=pad)
    assert q.shape == want_q.shape and s.shape == want_s.shape
    _codes_equal(s, want_s, "scales")
    _codes_equal(q, want_q, "codes")
    out_dtype = [torch.bfloat16, torch.float16, torch.float32][seed % 3]
    want = ref.dequantize_mxfp8(want_q, want_s, out_dtype)
    got = ck.dequantize_mxfp8(q, s, out_dtype)
    assert got.shape == want.shape and torch.equal(bits(got), bits(want))


@pytest.mark.parametrize("m,k,dtype,pad,spread,seed", _cases(47, 24, 16))
def test_nvfp4_random(m, k, dtype, pad, spread, seed, hip):
    x = _input(m, k, dtype, spread, seed)
    hi_first = seed % 2 == 0
    g = (x.float().abs().amax() / 2688).reshape(1)
    want_q, want_s = ref.quantize_nvfp4(x, g, pad_16x=pad, hi_first=hi_first)
    q, s = ck.quantize_nvfp4(x.cuda(), g.cuda(), pad_16x=pad, hi_first=hi_first)
    assert q.shape == want_q.shape and s.shape == want_s.shape
    _codes_equal(s, want_s, "scales")
    _codes_equal(q, want_q, "codes")
    out_dtype = [torch.bfloat16, torch.float16, torch.float32][seed % 3]
    want = ref.dequantize_nvfp4(want_q, g, want_s, out_dtype, hi_first=hi_first)
    got = ck.dequantize_nvfp4(q, g.cuda(), s, out_dtype, hi_first=hi_first)
    assert got.shape == want.shape and torch.equal(bits(got), bits(want))


@pytest.mark.parametrize("m,k,dtype,pad,spread,seed", _cases(59, 16, 1))
def test_fp8_random(m, k, dtype, pad, spread, seed, hip):
    x = _input(m, k, dtype, spread, seed)
    out_type = torch.float8_e4m3fn if seed % 2 else torch.float8_e5m2
    scale = (x.float().abs().amax() / 448).clamp_min(1e-12).reshape(1)
    want = ref.quantize_per_tensor_fp8(x.clone(), scale, out_type)
    got = ck.quantize_per_tensor_fp8(x.cuda(), scale.cuda(), out_type)
    assert got.shape == want.shape and got.dtype == out_type
    _codes_equal(got, want, "codes")
    out_dtype = [torch.bfloat16, torch.float16, torch.float32][seed % 3]
    back = ref.dequantize_per_tensor_fp8(want, scale, out_dtype)
    assert torch.equal(bits(ck.dequantize_per_tensor_fp8(got, scale.cuda(), out_dtype)), bits(back))
