"""Seeded random GEMM shapes against the CPU oracle, both block formats.

The GEMM launchers choose among many forms by M, N and K: skinny kernels (waves, weight
tiles and staged activation rows by M and N), whole tiles, half tiles for a last or only
round, weight-prefetch workgroups on idle CUs, and split-K in full or half tiles with
ranges of any length.  Each case draws a shape from ranges that straddle those choices, so
the suite crosses their boundaries in combinations the hand-picked shapes do not; a few
larger grids with short K cover the whole-tile rounds and their last rounds.
"""
import random

import pytest
import torch

import comfy_kitchen as ck
from oracle import eager_ref as ref

pytestmark = pytest.mark.gpu

REL_L2 = {torch.float32: 1e-4, torch.bfloat16: 4e-3}


def rel_l2(got: torch.Tensor, want: torch.Tensor) -> float:
    got, want = got.float().cpu(), want.float().cpu()
    return ((got - want).norm() / want.norm().clamp_min(1e-30)).item()


def _shapes(seed: int, count: int):
    rng = random.Random(seed)
    out = []
    for _ in range(count):
        m = rng.choice([rng.randint(1, 64), rng.randint(65, 600)])
        n = rng.choice([rng.randint(1, 600), rng.randint(600, 2600)])
        k = 32 * rng.randint(1, 140)  # up to 4480
        out.append((m, n, k))
    return out


def _big_shapes(seed: int, count: int):
    """Grids of 72-378 tiles of 256 x 256 (one round of whole tiles, or several rounds and
    a last round of full or half tiles), with short K to keep the oracle fast."""
    rng = random.Random(seed)
    return [(rng.randint(1500, 4600), rng.randint(3000, 5200), 32 * rng.randint(1, 10)) for _ in range(count)]


@pytest.mark.parametrize("m,n,k", _shapes(2024, 24) + _big_shapes(77, 6))
def test_scaled_mm_mxfp8_random_shapes(m, n, k, hip):
    g = torch.Generator().manual_seed(m * 131 + n * 7 + k)
    x = (torch.randn(m, k, generator=g) * torch.exp(torch.randn(m, 1, generator=g))).bfloat16()
    w = (torch.randn(n, k, generator=g) * 0.02).bfloat16()
    qx, sx = ref.quantize_mxfp8(x, pad_32x=False)
    qw, sw = ref.quantize_mxfp8(w, pad_32x=False)
    want = ref.scaled_mm_mxfp8_ref(qx, qw, sx, sw, out_dtype=torch.float32)
    out_dtype = torch.float32 if (m + n) % 2 else torch.bfloat16
    got = ck.scaled_mm_mxfp8(qx.cuda(), qw.cuda(), sx.cuda(), sw.cuda(), out_dtype=out_dtype)
    assert got.shape == (m, n)
    assert rel_l2(got, want) <= REL_L2[out_dtype]
    # the per-tensor FP8 GEMM (the same paths with unit block scales) on the same codes
    ta, tb = torch.tensor([0.75]), torch.tensor([2e-3])
    want8 = (qx.float() @ qw.float().t()) * (ta * tb)
    got8 = ck.scaled_mm_fp8(qx.cuda(), qw.cuda(), ta.cuda(), tb.cuda(), out_dtype=out_dtype)
    assert rel_l2(got8, want8) <= REL_L2[out_dtype]


@pytest.mark.parametrize("m,n,k", _shapes(4048, 24) + _big_shapes(78, 6))
def test_scaled_mm_nvfp4_random_shapes(m, n, k, hip):
    g = torch.Generator().manual_seed(m * 137 + n * 11 + k)
    x = torch.randn(m, k, generator=g).bfloat16()
    w = (torch.randn(n, k, generator=g) * 0.02).bfloat16()
    gx = (x.float().abs().amax() / 2688).reshape(1)
    gw = (w.float().abs().amax() / 2688).reshape(1)
    qx, sx = ref.quantize_nvfp4(x, gx)
    qw, sw = ref.quantize_nvfp4(w, gw)
    want = ref.scaled_mm_nvfp4_ref(qx, qw, gx, gw, sx, sw, out_dtype=torch.float32)
    out_dtype = torch.float32 if (m + n) % 2 else torch.bfloat16
    got = ck.scaled_mm_nvfp4(qx.cuda(), qw.cuda(), gx.cuda(), gw.cuda(), sx.cuda(), sw.cuda(), out_dtype=out_dtype)
    assert got.shape == (m, n)
    assert rel_l2(got, want) <= REL_L2[out_dtype]
