"""Pin the CPU oracle (oracle/eager_ref.py) before trusting it.

Three independent checks, none of which retypes the oracle's own formula:
  * hand-derived known answers (tests/golden/known_answers.json);
  * oracle/scalar_ref.c, a scalar restatement that rounds by brute-force nearest-value
    search instead of bit manipulation, compared exhaustively over all 65,536 bf16
    inputs and over large random samples of blocks;
  * closed-form layout identities (swizzle offsets, round trips, nibble swap).
"""
import ctypes

import numpy as np
import pytest
import torch

import kat
from oracle import eager_ref as ref

pytestmark = []


def _u8(t: torch.Tensor) -> list[int]:
    return t.contiguous().view(torch.uint8).reshape(-1).tolist()


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data_as(ctypes.c_void_p).value


# ------------------------------------------------------------- known answers
@pytest.mark.parametrize("case", range(len(kat.fp8_quant_cases())))
def test_kat_quantize_fp8_oracle_and_scalar(case, scalar_ref):
    x, scale, dt, want = kat.fp8_quant_cases()[case]
    assert _u8(ref.quantize_per_tensor_fp8(x.clone(), scale, dt)) == [want] * x.numel()
    if x.dtype != torch.bfloat16:
        return  # the scalar C restatement covers bf16 input
    xb = ref.bf16_bits(x).copy()
    out = np.zeros(x.numel(), dtype=np.uint8)
    scalar_ref.ref_quantize_fp8_bf16(_ptr(xb), x.numel(), float(scale), int(dt == torch.float8_e5m2), _ptr(out))
    assert out.tolist() == [want] * x.numel()


def test_fp8_nan_bytes_follow_eager_vector_loop():
    """The eager per-tensor FP8 chain's NaN bytes, as torch's CPU kernels write them:
    bf16 products narrow every NaN to 0xFFFF (code 0xFF) in the vectorised loop, and
    c10::BFloat16's 0x7FC0 (code 0x7F) only in the scalar remainder; f16 and f32 keep the
    NaN's sign in both.  Tensors whose length is a multiple of 64 run the vectorised loop
    alone, which is the behaviour the HIP kernel follows."""
    nan_bits = {torch.bfloat16: (0x7FC0, -0x40), torch.float16: (0x7E00, -0x200),
                torch.float32: (0x7FC00000, -0x400000)}  # +NaN, -NaN
    for dt, (pb, nb) in nan_bits.items():
        n = 256
        xb = torch.zeros(n, dtype=kat.BITS_VIEW[dt])
        xb[0::2], xb[1::2] = pb, nb
        x = xb.view(dt)
        for out in (torch.float8_e4m3fn, torch.float8_e5m2):
            q = _u8(ref.quantize_per_tensor_fp8(x.clone(), torch.tensor([1.0]), out))
            want = [0xFF] * n if dt == torch.bfloat16 else [0x7F, 0xFF] * (n // 2)
            assert q == want, (dt, out)
    # a lone bf16 NaN runs the scalar remainder: code 0x7F (a property of eager on the CPU
    # only; the HIP kernel writes 0xFF throughout)
    one = torch.tensor([0x7FC0], dtype=torch.int16).view(torch.bfloat16)
    assert _u8(ref.quantize_per_tensor_fp8(one, torch.tensor([1.0]))) == [0x7F]


@pytest.mark.parametrize("case", range(len(kat.fp8_dequant_cases())))
def test_kat_dequantize_fp8_oracle(case):
    q, scale, want = kat.fp8_dequant_cases()[case]
    got = ref.dequantize_per_tensor_fp8(q, scale, torch.bfloat16)
    assert int(got.view(torch.int16).item()) & 0xFFFF == want


@pytest.mark.parametrize("case", range(len(kat.mxfp8_cases())))
def test_kat_mxfp8_oracle_and_scalar(case, scalar_ref):
    x, want_scale, want_codes = kat.mxfp8_cases()[case]
    q, s = ref.quantize_mxfp8(x.reshape(1, 32))
    assert ref.from_blocked(s.view(torch.uint8), 1, 1).item() == want_scale
    assert kat.codes_match(_u8(q), want_codes), _u8(q)
    xb = ref.bf16_bits(x).copy()
    e, c = np.zeros(1, np.uint8), np.zeros(32, np.uint8)
    scalar_ref.ref_quantize_mxfp8_row_bf16(_ptr(xb), 1, _ptr(e), _ptr(c))
    assert int(e[0]) == want_scale
    assert kat.codes_match(c.tolist(), want_codes)


@pytest.mark.parametrize("case", range(len(kat.nvfp4_cases())))
def test_kat_nvfp4_oracle_and_scalar(case, scalar_ref):
    x, g, want_scale, want_codes, want_packed = kat.nvfp4_cases()[case]
    q, s = ref.quantize_nvfp4(x.reshape(1, 16), g)
    assert ref.from_blocked(s.view(torch.uint8), 1, 1).item() == want_scale
    assert kat.unpack(q) == want_codes
    if want_packed:
        assert _u8(q) == want_packed
    xb = ref.bf16_bits(x).copy()
    sc, c = np.zeros(1, np.uint8), np.zeros(16, np.uint8)
    scalar_ref.ref_quantize_nvfp4_row_bf16(_ptr(xb), 1, float(g), _ptr(sc), _ptr(c))
    assert int(sc[0]) == want_scale and c.tolist() == want_codes


@pytest.mark.parametrize("case", range(len(kat.default_scale_cases())))
def test_kat_default_scale_oracle_and_scalar(case, scalar_ref):
    """The layouts' default scale: rounded to x's dtype, and formed as amax * RN32(1/d)
    as torch's GPU kernel does.  A scale kept in fp32, or a true division, fails."""
    x, code, divisor, want = kat.default_scale_cases()[case]
    got = ref.default_scale(x, divisor)
    assert got.dtype == torch.float32 and got.shape == ()
    assert int(got.view(torch.int32)) & 0xFFFFFFFF == want
    s = scalar_ref.ref_default_scale(float(x), divisor, code)
    assert int(np.float32(s).view(np.uint32)) == want


@pytest.mark.parametrize("case", range(len(kat.dequantize_nvfp4_cases())))
@pytest.mark.parametrize("hi_first", [True, False])
def test_kat_dequantize_nvfp4_oracle_and_scalar(case, hi_first, scalar_ref):
    """The block total g.to(out) * s8.to(out) and the element product round in the output
    dtype; forming either in fp32 gives a different last bit for these cases."""
    dt, code, g, sbyte, c4, want = kat.dequantize_nvfp4_cases()[case]
    q, s = kat.nvfp4_block(c4, sbyte)
    out = ref.dequantize_nvfp4(q, g, s, dt, hi_first=hi_first)
    assert out.shape == (1, 16)
    assert set((out.view(torch.int16).int() & 0xFFFF).tolist()[0]) == {want}
    v = scalar_ref.ref_dequantize_nvfp4_value(c4, sbyte, float(g), code)
    assert int(torch.tensor(v).to(dt).view(torch.int16)) & 0xFFFF == want


def _all16(dt):
    return torch.arange(65536, dtype=torch.int32).to(torch.int16).view(dt)


@pytest.mark.parametrize("divisor", [448.0, 2688.0, 57344.0])
def test_default_scale_oracle_vs_scalar(divisor, scalar_ref):
    """Every tiny f16 amax (where torch's device and CPU kernels disagree), a bf16 and
    an f32 sample, each as a one-element tensor through the oracle's expression."""
    g = torch.Generator().manual_seed(3)
    f16 = _all16(torch.float16)
    f16 = f16[(f16.float().abs() < 0.06) & (f16.float() >= 0)]
    bf16 = _all16(torch.bfloat16)
    bf16 = bf16[torch.isfinite(bf16.float()) & (bf16.float() >= 0)]
    bf16 = bf16[torch.randperm(bf16.numel(), generator=g)[:3000]]
    f32 = (torch.rand(3000, generator=g) * 2 ** torch.randint(-40, 40, (3000,), generator=g).float())
    for t, code in ((f16, 1), (bf16, 2), (f32, 0)):
        for v in t:
            got = ref.default_scale(v.reshape(1), divisor)
            want = scalar_ref.ref_default_scale(abs(float(v)), divisor, code)
            assert int(got.view(torch.int32)) == int(np.float32(want).view(np.int32)), (code, float(v))


@pytest.mark.parametrize("out_dtype, code", [(torch.bfloat16, 2), (torch.float16, 1), (torch.float32, 0)])
def test_dequantize_nvfp4_oracle_vs_scalar(out_dtype, code, scalar_ref):
    """Every E2M1 code x every finite E4M3 scale byte, for a few global scales."""
    codes = torch.arange(16, dtype=torch.uint8)
    for g in (1.005859375, 1.000732421875, 0.0123, 3e-3, 77.7):
        for sbyte in range(0, 0x7F):
            vals = [scalar_ref.ref_dequantize_nvfp4_value(c, sbyte, g, code) for c in range(16)]
            q = ((codes[0::2] << 4) | codes[1::2]).reshape(1, 8)
            s = torch.zeros(128, 4, dtype=torch.uint8)
            s[0, 0] = sbyte
            out = ref.dequantize_nvfp4(q, torch.tensor([g]), s.view(torch.float8_e4m3fn), out_dtype)
            want = torch.tensor(vals).to(out_dtype)
            assert torch.equal(out.reshape(16).view(torch.int16 if code else torch.int32),
                               want.view(torch.int16 if code else torch.int32)), (g, sbyte)


# -------------------------------------------------- exhaustive vs scalar C
@pytest.mark.parametrize("out_dtype", [torch.float8_e4m3fn, torch.float8_e5m2], ids=["e4m3", "e5m2"])
@pytest.mark.parametrize("scale", [1.0, 0.9481481481481482, 10.0 / 448, 2.0 ** -20, 3.0e4, 0.7])
def test_quantize_fp8_all_bf16_vs_scalar(scale, out_dtype, scalar_ref):
    x = ref.all_bf16()
    got = _u8(ref.quantize_per_tensor_fp8(x.clone(), torch.tensor([scale]), out_dtype))
    xb = ref.bf16_bits(x).copy()
    want = np.zeros(65536, np.uint8)
    scalar_ref.ref_quantize_fp8_bf16(_ptr(xb), 65536, scale, int(out_dtype == torch.float8_e5m2), _ptr(want))
    got = np.array(got, np.uint8)
    mism = np.nonzero(got != want)[0]  # NaN code bytes included
    assert mism.size == 0, f"{mism.size} mismatches, first x bits {xb[mism[:5]]}"


def test_fp8_library_cast_vs_bruteforce(scalar_ref):
    """torch's fp32->E4M3/E5M2 cast (the routine the oracle relies on) is RNE on the clamped range."""
    x = ref.all_bf16().float()
    for dt, lim, fn in ((torch.float8_e4m3fn, 448.0, scalar_ref.ref_f32_to_e4m3),
                        (torch.float8_e5m2, 57344.0, scalar_ref.ref_f32_to_e5m2)):
        v = x[(x.abs() <= lim) | x.isnan()]
        got = _u8(v.to(dt))
        want = [fn(float(f)) for f in v.tolist()]
        assert got == want
        # NaNs keep their sign in the cast: 0x7F | sign
        nans = torch.tensor([0x7FC00000, -0x400000, 0x7F800001, -0x7FFFFF], dtype=torch.int32).view(torch.float32)
        assert _u8(nans.to(dt)) == [0x7F, 0xFF, 0x7F, 0xFF]


def test_e2m1_oracle_vs_bruteforce(scalar_ref):
    g = torch.Generator().manual_seed(0)
    pieces = [ref.all_bf16().float(),
              (torch.rand(200_000, generator=g) * 13 - 6.5)]
    mids = torch.tensor([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 6.0, 1.0, 0.5])
    for m in mids.tolist():
        for k in range(-4, 5):
            f = np.float32(m).view(np.int32) + k
            pieces.append(torch.tensor([np.int32(f).view(np.float32), -np.int32(f).view(np.float32)]))
    x = torch.cat(pieces)
    x = x[~torch.isnan(x)].clamp(-6.0, 6.0)
    got = ref.f32_to_e2m1(x).tolist()
    want = [scalar_ref.ref_f32_to_e2m1(float(f)) for f in x.tolist()]
    assert got == want


def _lognormal_rows(rows, cols, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, cols, generator=g) * torch.exp(torch.randn(rows, 1, generator=g) * 3)
    x[0, :32] = 0.0  # a zero block
    x[1, 5] = 1e-38  # tiny values
    return x.to(dtype)


def test_mxfp8_oracle_vs_scalar(scalar_ref):
    x = _lognormal_rows(96, 1024, 1)
    q, s = ref.quantize_mxfp8(x)
    e = ref.from_blocked(s.view(torch.uint8), 96, 32).numpy()
    qn = q.view(torch.uint8).numpy()
    for r in range(96):
        xb = ref.bf16_bits(x[r]).copy()
        ee, cc = np.zeros(32, np.uint8), np.zeros(1024, np.uint8)
        scalar_ref.ref_quantize_mxfp8_row_bf16(_ptr(xb), 32, _ptr(ee), _ptr(cc))
        assert np.array_equal(ee, e[r]), r
        assert np.array_equal(cc, qn[r]), r


@pytest.mark.parametrize("g", [1.0, 0.0123, 3.7e-3, 250.0])
def test_nvfp4_oracle_vs_scalar(g, scalar_ref):
    x = _lognormal_rows(64, 512, 2)
    q, s = ref.quantize_nvfp4(x, torch.tensor([g]))
    sc = ref.from_blocked(s.view(torch.uint8), 64, 32).numpy()
    codes = np.array([kat.unpack(q[r]) for r in range(64)], np.uint8)
    for r in range(64):
        xb = ref.bf16_bits(x[r]).copy()
        ss, cc = np.zeros(32, np.uint8), np.zeros(512, np.uint8)
        scalar_ref.ref_quantize_nvfp4_row_bf16(_ptr(xb), 32, g, _ptr(ss), _ptr(cc))
        assert np.array_equal(ss, sc[r]), r
        assert np.array_equal(cc, codes[r]), r


# -------------------------------------------------------------- layouts
def test_swizzle_layout_closed_form():
    """Oracle to_blocked places (r, c) at the 32_4_4 offset formula; padding is zero."""
    rows, cols = 300, 11
    src = torch.arange(rows * cols, dtype=torch.int32).reshape(rows, cols) + 1
    blk = ref.to_blocked(src).reshape(-1)
    n_cb = -(-cols // 4)
    for r in range(rows):
        for c in range(cols):
            off = (((r // 128) * n_cb + c // 4) * 32 + r % 32) * 16 + ((r % 128) // 32) * 4 + c % 4
            assert blk[off].item() == src[r, c].item()
    assert int((blk == 0).sum()) == blk.numel() - rows * cols
    assert torch.equal(ref.from_blocked(ref.to_blocked(src), rows, cols), src)


def test_package_swizzle_matches_oracle():
    import comfy_kitchen as ck

    g = torch.Generator().manual_seed(3)
    for rows, cols in [(1, 1), (128, 4), (129, 5), (4608, 96), (33, 320)]:
        s = torch.randint(0, 255, (rows, cols), generator=g, dtype=torch.uint8)
        a = ck.to_blocked(s, flatten=False)
        b = ref.to_blocked(s)
        assert torch.equal(a, b)
        assert torch.equal(ck.from_blocked(a, rows, cols), s)
        assert torch.equal(ck.to_blocked(s).reshape(a.shape), a)


def test_swap_nibbles_and_hi_first():
    import comfy_kitchen as ck

    x = _lognormal_rows(16, 64, 4)
    g = torch.tensor([0.01])
    qh, sh = ref.quantize_nvfp4(x, g, hi_first=True)
    ql, sl = ref.quantize_nvfp4(x, g, hi_first=False)
    assert torch.equal(ck.swap_nibbles(qh), ql)
    assert torch.equal(sh.view(torch.uint8), sl.view(torch.uint8))
    assert torch.equal(ref.dequantize_nvfp4(qh, g, sh), ref.dequantize_nvfp4(ql, g, sl, hi_first=False))


# --------------------------------------------------------------------- RoPE
def _rotation(theta: torch.Tensor) -> torch.Tensor:
    """[..., 2, 2] rotation matrices [[cos, -sin], [sin, cos]] (the Flux EmbedND layout)."""
    c, s = torch.cos(theta), torch.sin(theta)
    return torch.stack([torch.stack([c, -s], -1), torch.stack([s, c], -1)], -2)


def test_rope_identity_and_quarter_turn():
    """Closed forms: the identity rotation returns x exactly; a quarter turn maps each
    pair (x0, x1) to (-x1, x0) exactly (every product is by 0 or +-1)."""
    g = torch.Generator().manual_seed(5)
    x = torch.randn(1, 3, 10, 16, generator=g).bfloat16()
    ident = _rotation(torch.zeros(1, 1, 10, 8, dtype=torch.float64)).float()
    assert torch.equal(ref.apply_rope1(x, ident), x)
    quarter = torch.tensor([[0.0, -1.0], [1.0, 0.0]]).expand(1, 1, 10, 8, 2, 2).contiguous()
    out = ref.apply_rope1(x, quarter).reshape(1, 3, 10, 8, 2)
    xp = x.reshape(1, 3, 10, 8, 2)
    assert torch.equal(out[..., 0], -xp[..., 1]) and torch.equal(out[..., 1], xp[..., 0])


def test_rope_matches_complex_rotation_within_one_ulp():
    """Against a float64 complex multiply (x0 + i x1) * e^{i theta}: the oracle computes in
    fp32 and rounds once to bf16, so it must sit within 1 bf16 ULP of the exact rotation.
    A swapped sign or transposed matrix would be off by far more."""
    g = torch.Generator().manual_seed(6)
    x = torch.randn(2, 4, 33, 64, generator=g).bfloat16()
    theta = torch.rand(1, 1, 33, 32, generator=g, dtype=torch.float64) * 6.3
    got = ref.apply_rope1(x, _rotation(theta).float()).double().reshape(2, 4, 33, 32, 2)
    z = torch.complex(x.double().reshape(2, 4, 33, 32, 2)[..., 0], x.double().reshape(2, 4, 33, 32, 2)[..., 1])
    r = z * torch.exp(1j * theta)
    for comp, exact in ((got[..., 0], r.real), (got[..., 1], r.imag)):
        ulp = torch.where(exact.abs() > 0, 2.0 ** (torch.floor(torch.log2(exact.abs())) - 7), 2.0 ** -133)
        assert bool(((comp - exact).abs() <= ulp).all())
    # apply_rope is apply_rope1 on each of q and k
    xk = torch.randn(2, 4, 33, 64, generator=g).bfloat16()
    q2, k2 = ref.apply_rope(x, xk, _rotation(theta).float())
    assert torch.equal(q2, ref.apply_rope1(x, _rotation(theta).float()))
    assert torch.equal(k2, ref.apply_rope1(xk, _rotation(theta).float()))


# ------------------------------------------------------------ GEMM references
E2M1_VALUES = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]


def _swz(r, c, n_cb):
    return (((r // 128) * n_cb + c // 4) * 32 + r % 32) * 16 + ((r % 128) // 32) * 4 + c % 4


def test_scaled_mm_mxfp8_ref_bruteforce():
    """Tiny MXFP8 GEMM summed element by element in float64 from raw code/scale bytes."""
    g = torch.Generator().manual_seed(8)
    m, n, k = 3, 2, 64
    a = torch.randint(0, 256, (m, k), generator=g, dtype=torch.uint8)
    b = torch.randint(0, 256, (n, k), generator=g, dtype=torch.uint8)
    a[(a & 0x7F) == 0x7F] = 0x12  # no NaN codes
    b[(b & 0x7F) == 0x7F] = 0x34
    sa = torch.zeros(128 * 4, dtype=torch.uint8)
    sb = torch.zeros(128 * 4, dtype=torch.uint8)
    ea = torch.randint(120, 134, (m, 2), generator=g)
    eb = torch.randint(120, 134, (n, 2), generator=g)
    for r in range(m):
        for c in range(2):
            sa[_swz(r, c, 1)] = int(ea[r, c])
    for r in range(n):
        for c in range(2):
            sb[_swz(r, c, 1)] = int(eb[r, c])
    av = a.view(torch.float8_e4m3fn).double()
    bv = b.view(torch.float8_e4m3fn).double()
    y = ref.scaled_mm_mxfp8_ref(a.view(torch.float8_e4m3fn), b.view(torch.float8_e4m3fn),
                                sa.view(torch.float8_e8m0fnu), sb.view(torch.float8_e8m0fnu), out_dtype=torch.float32)
    for i in range(m):
        for j in range(n):
            s = sum(float(av[i, kk]) * 2.0 ** (int(ea[i, kk // 32]) - 127) * float(bv[j, kk]) *
                    2.0 ** (int(eb[j, kk // 32]) - 127) for kk in range(k))
            assert abs(y[i, j].item() - s) <= 1e-5 * max(1.0, abs(s))


def test_scaled_mm_nvfp4_ref_bruteforce():
    """Tiny NVFP4 GEMM from raw nibbles (even element in the high nibble), E4M3 block
    scales and the two tensor scales, summed in float64."""
    g = torch.Generator().manual_seed(9)
    m, n, k = 2, 3, 32
    qa = torch.randint(0, 256, (m, k // 2), generator=g, dtype=torch.uint8)
    qb = torch.randint(0, 256, (n, k // 2), generator=g, dtype=torch.uint8)
    ca = torch.randint(0x20, 0x50, (m, 2), generator=g, dtype=torch.uint8)  # normal E4M3 scales
    cb = torch.randint(0x20, 0x50, (n, 2), generator=g, dtype=torch.uint8)
    sa = torch.zeros(128 * 4, dtype=torch.uint8)
    sb = torch.zeros(128 * 4, dtype=torch.uint8)
    for r in range(m):
        for c in range(2):
            sa[_swz(r, c, 1)] = int(ca[r, c])
    for r in range(n):
        for c in range(2):
            sb[_swz(r, c, 1)] = int(cb[r, c])
    ts_a, ts_b = torch.tensor([0.75]), torch.tensor([1.25])

    def val(q, row, kk):
        byte = int(q[row, kk // 2])
        nib = (byte >> 4) if kk % 2 == 0 else (byte & 15)
        return (-1.0 if nib & 8 else 1.0) * E2M1_VALUES[nib & 7]

    def e4m3(byte):
        return float(torch.tensor([byte], dtype=torch.uint8).view(torch.float8_e4m3fn).double())

    y = ref.scaled_mm_nvfp4_ref(qa, qb, ts_a, ts_b, sa.view(torch.float8_e4m3fn), sb.view(torch.float8_e4m3fn),
                                out_dtype=torch.float32)
    for i in range(m):
        for j in range(n):
            s = sum(val(qa, i, kk) * e4m3(int(ca[i, kk // 16])) * val(qb, j, kk) * e4m3(int(cb[j, kk // 16]))
                    for kk in range(k)) * 0.75 * 1.25
            assert abs(y[i, j].item() - s) <= 1e-5 * max(1.0, abs(s))
