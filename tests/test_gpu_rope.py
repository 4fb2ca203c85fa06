"""HIP RoPE vs the CPU oracle (reference eager rope.py:7-18).

Bar (north star): within 1 ULP of the output dtype for fp32 freqs.  With 16-bit
freqs the reference computes in that 16-bit type; the kernel emulates each rounding,
so the same 1-ULP bound is asserted there too.  fp32 x (served by eager on a GPU,
backends/eager/__init__.py:118-131): bit-exact with 16-bit freqs; with fp32 freqs within
2^-21 of the sum of the two product magnitudes (the kernel adds the second product with
one rounding, eager with two).
"""
import random

import pytest
import torch

import comfy_kitchen as ck
from oracle import eager_ref as ref

pytestmark = pytest.mark.gpu


def ulp_diff(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """|a - b| in units in the last place of the 16-bit format (ordered-integer distance)."""
    ia = a.detach().cpu().contiguous().view(torch.int16).to(torch.int32)
    ib = b.detach().cpu().contiguous().view(torch.int16).to(torch.int32)
    oa = torch.where(ia < 0, -(ia & 0x7FFF), ia)
    ob = torch.where(ib < 0, -(ib & 0x7FFF), ib)
    return (oa - ob).abs()


def check(got, want, max_ulp=1):
    assert got.shape == want.shape and got.dtype == want.dtype
    d = ulp_diff(got, want)
    assert int(d.max()) <= max_ulp, f"max ulp {int(d.max())}, {int((d > max_ulp).sum())} elements over"
    return float((d == 0).float().mean())


def test_config2_flux_full(hip):
    import bench

    q, k, f = bench.make_c2()
    wq, wk = ref.apply_rope(q, k, f)
    gq, gk = ck.apply_rope(q.cuda(), k.cuda(), f.cuda())
    exact = min(check(gq, wq), check(gk, wk))
    print(f"fraction bit-identical: {exact:.6f}")
    g1 = ck.apply_rope1(q.cuda(), f.cuda())
    assert torch.equal(g1.cpu(), gq.cpu())


@pytest.mark.parametrize("op", ["apply_rope", "apply_rope1"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("freqs_dtype", [torch.float32, torch.float16, torch.bfloat16],
                         ids=["f32", "f16", "bf16"])
@pytest.mark.parametrize("name,layout,shape", [
    ("FLUX", "BHND", (1, 24, 4352, 128)),
    ("LTX", "BHND", (2, 32, 4996, 64)),
    ("ZIMAGE", "BNHD", (1, 4096, 30, 128)),
], ids=["FLUX", "LTX", "ZIMAGE"])
def test_reference_configs(op, dtype, freqs_dtype, name, layout, shape, hip, seed):
    """The reference's own RoPE test configs (tests/test_rope.py:15-35)."""
    if layout == "BHND":
        b, h, n, d = shape
        fshape = (b, 1, n, d // 2, 2, 2)
    else:
        b, n, h, d = shape
        fshape = (1, n, 1, d // 2, 2, 2)
    f = torch.randn(fshape).to(freqs_dtype)
    xq = torch.randn(shape).to(dtype)
    if op == "apply_rope":
        xk = torch.randn(shape).to(dtype)
        wq, wk = ref.apply_rope(xq, xk, f)
        gq, gk = ck.apply_rope(xq.cuda(), xk.cuda(), f.cuda())
        check(gq, wq)
        check(gk, wk)
    else:
        check(ck.apply_rope1(xq.cuda(), f.cuda()), ref.apply_rope1(xq, f))


def test_freqs_longer_than_sequence_is_truncated(hip, seed):
    x = torch.randn(2, 4, 100, 64).bfloat16()
    f = torch.randn(1, 1, 130, 32, 2, 2)
    check(ck.apply_rope1(x.cuda(), f.cuda()), ref.apply_rope1(x, f))


def test_fully_broadcast_and_per_batch_freqs(hip, seed):
    x = torch.randn(3, 5, 7, 32).half()
    for fshape in [(1, 1, 1, 16, 2, 2), (3, 1, 7, 16, 2, 2), (3, 5, 7, 16, 2, 2), (1, 5, 1, 16, 2, 2)]:
        f = torch.randn(fshape)
        check(ck.apply_rope1(x.cuda(), f.cuda()), ref.apply_rope1(x, f))


def test_unvectorized_head_dim_and_noncontiguous(hip, seed):
    x = torch.randn(1, 3, 9, 6).bfloat16()  # head_dim 6: scalar path
    f = torch.randn(1, 1, 9, 3, 2, 2)
    check(ck.apply_rope1(x.cuda(), f.cuda()), ref.apply_rope1(x, f))
    xt = torch.randn(1, 9, 3, 64).bfloat16().transpose(1, 2)  # non-contiguous input
    f2 = torch.randn(1, 1, 9, 32, 2, 2)
    check(ck.apply_rope1(xt.cuda(), f2.cuda()), ref.apply_rope1(xt, f2))
    f3 = torch.randn(1, 1, 9, 32, 2, 2, 2)[..., 0]  # non-contiguous freqs
    check(ck.apply_rope1(xt.cuda(), f3.cuda()), ref.apply_rope1(xt, f3))


def test_mismatched_q_k_shapes(hip, seed):
    q = torch.randn(1, 8, 16, 64).bfloat16()
    k = torch.randn(1, 2, 16, 64).bfloat16()
    f = torch.randn(1, 1, 16, 32, 2, 2)
    gq, gk = ck.apply_rope(q.cuda(), k.cuda(), f.cuda())
    wq, wk = ref.apply_rope(q, k, f)
    check(gq, wq)
    check(gk, wk)


@pytest.mark.parametrize("freqs_dtype", [torch.float32, torch.float16, torch.bfloat16], ids=["f32", "f16", "bf16"])
@pytest.mark.parametrize("shape", [(1, 4, 64, 128), (2, 3, 9, 6), (1, 64, 3, 64)], ids=["vec", "scalar", "bnhd"])
def test_fp32_x(freqs_dtype, shape, hip, seed):
    b, h, n, d = shape
    f = torch.randn(1, 1, n, d // 2, 2, 2).to(freqs_dtype)
    xq, xk = torch.randn(shape) * 4, torch.randn(shape)
    wq, wk = ref.apply_rope(xq, xk, f)
    gq, gk = ck.apply_rope(xq.cuda(), xk.cuda(), f.cuda())
    g1 = ck.apply_rope1(xq.cuda(), f.cuda())
    assert torch.equal(g1.cpu(), gq.cpu())
    for g, w, x in ((gq, wq, xq), (gk, wk, xk)):
        assert g.dtype == torch.float32 and g.shape == x.shape
        g = g.cpu()
        if freqs_dtype != torch.float32:
            assert torch.equal(g, w)
            continue
        xp = x.double().reshape(b, h, n, d // 2, 1, 2)
        fd = f.double()
        mag = (fd[..., 0] * xp[..., 0]).abs() + (fd[..., 1] * xp[..., 1]).abs()
        err = (g.double() - w.double()).reshape(mag.shape).abs()
        assert bool((err <= mag * 2.0 ** -21 + 1e-38).all()), float((err / mag.clamp_min(1e-30)).max())


def _random_cases(seed: int, count: int):
    """(b, h, n, d, per-batch freqs, per-head freqs, x dtype, freqs dtype, seed)"""
    rng = random.Random(seed)
    return [(rng.randint(1, 3), rng.randint(1, 24), rng.randint(1, 600), rng.choice([6, 8, 16, 32, 48, 64, 96, 128, 256]),
             rng.random() < 0.3, rng.random() < 0.2, rng.choice(["bf16", "f16"]), rng.choice(["f32", "f16", "bf16"]),
             rng.randrange(1 << 30)) for _ in range(count)]


_DT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


@pytest.mark.parametrize("b,h,n,d,fb,fh,xdt,fdt,seed", _random_cases(7, 24))
def test_random_shapes(b, h, n, d, fb, fh, xdt, fdt, seed, hip):
    """Seeded random batch, heads, positions, head_dim (vector and scalar paths) and freqs
    broadcast over batch and heads or not, through both ops."""
    g = torch.Generator().manual_seed(seed)
    f = torch.randn(b if fb else 1, h if fh else 1, n, d // 2, 2, 2, generator=g).to(_DT[fdt])
    xq = torch.randn(b, h, n, d, generator=g).to(_DT[xdt])
    xk = torch.randn(b, h, n, d, generator=g).to(_DT[xdt])
    wq, wk = ref.apply_rope(xq, xk, f)
    gq, gk = ck.apply_rope(xq.cuda(), xk.cuda(), f.cuda())
    check(gq, wq)
    check(gk, wk)
    assert torch.equal(ck.apply_rope1(xq.cuda(), f.cuda()).cpu(), gq.cpu())
