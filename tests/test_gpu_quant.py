"""HIP quantizers / dequantizers vs the CPU oracle: bit-exact codes, scales and outputs.

Bar: every code byte, every scale byte (including swizzle padding) and every
dequantized element equal to the oracle's (the reference eager arithmetic).  Quantized
NaN code bytes compare exactly.  Inputs holding NaNs are sized in multiples of 64
elements, so that eager's vectorised loop alone produces them (its scalar remainder
writes other NaN bytes for bf16 input; the kernels follow the vectorised loop).
Dequantized NaN values compare by position: their payload bits are the device's.
"""
import pytest
import torch

import comfy_kitchen as ck
import kat
from conftest import bits
from oracle import eager_ref as ref

pytestmark = pytest.mark.gpu


def _fp8_equal(got: torch.Tensor, want: torch.Tensor, dt=torch.float8_e4m3fn):
    """Every code byte equal, NaN codes included (sign and all)."""
    g, w = bits(got).reshape(-1), bits(want).reshape(-1)
    bad = g != w
    assert int(bad.sum()) == 0, (f"{int(bad.sum())} of {g.numel()} codes differ; first at "
                                 f"{bad.nonzero()[:5].flatten().tolist()}: got {g[bad][:5].tolist()}, "
                                 f"want {w[bad][:5].tolist()}")


# ------------------------------------------------------------- known answers
@pytest.mark.parametrize("case", range(len(kat.fp8_quant_cases())))
def test_kat_quantize_fp8(case, hip, dev):
    x, scale, dt, want = kat.fp8_quant_cases()[case]
    got = ck.quantize_per_tensor_fp8(x.to(dev), scale.to(dev), dt)
    assert bits(got).tolist() == [want] * x.numel()


@pytest.mark.parametrize("case", range(len(kat.fp8_dequant_cases())))
def test_kat_dequantize_fp8(case, hip, dev):
    q, scale, want = kat.fp8_dequant_cases()[case]
    got = ck.dequantize_per_tensor_fp8(q.to(dev), scale.to(dev), torch.bfloat16)
    assert bits(got).item() & 0xFFFF == want


def test_kat_mxfp8(hip, dev):
    cases = kat.mxfp8_cases()
    x = torch.stack([c[0] for c in cases])  # one block per row
    q, s = ck.quantize_mxfp8(x.to(dev))
    e = ref.from_blocked(bits(s), len(cases), 1)
    for r, (_, want_s, want_c) in enumerate(cases):
        assert e[r, 0].item() == want_s, r
        assert kat.codes_match(bits(q[r]).tolist(), want_c), (r, bits(q[r]).tolist())


def test_kat_nvfp4(hip, dev):
    for x, g, want_s, want_c, want_p in kat.nvfp4_cases():
        q, s = ck.quantize_nvfp4(x.reshape(1, 16).to(dev), g.to(dev))
        assert ref.from_blocked(bits(s), 1, 1).item() == want_s
        assert kat.unpack(q.cpu()) == want_c
        if want_p:
            assert bits(q).tolist() == [want_p]


# ------------------------------------------------------- per-tensor FP8
@pytest.mark.parametrize("out_dtype", [torch.float8_e4m3fn, torch.float8_e5m2], ids=["e4m3", "e5m2"])
@pytest.mark.parametrize("scale", [1.0, 0.9481481481481482, 10.0 / 448, 2.0 ** -20, 3.0e4, 0.7])
def test_quantize_fp8_every_bf16(scale, out_dtype, hip, dev):
    """All 65,536 bf16 bit patterns (including NaN, inf, subnormals) at several scales."""
    x = ref.all_bf16()
    s = torch.tensor([scale])
    want = ref.quantize_per_tensor_fp8(x.clone(), s, out_dtype)
    got = ck.quantize_per_tensor_fp8(x.to(dev), s.to(dev), out_dtype)
    _fp8_equal(got, want, out_dtype)


def _nan_mix(dtype: torch.dtype, n: int, gen: torch.Generator) -> torch.Tensor:
    """n values of dtype: finite values, +-0, +-inf and NaNs of both signs, shuffled."""
    x = (torch.randn(n, generator=gen) * 30).to(dtype)
    pos, neg = {torch.bfloat16: (0x7FC0, -0x40), torch.float16: (0x7E00, -0x200),
                torch.float32: (0x7FC00000, -0x400000)}[dtype]
    xb = x.view(kat.BITS_VIEW[dtype])
    idx = torch.randperm(n, generator=gen)
    q = n // 8
    xb[idx[:q]] = pos
    xb[idx[q:2 * q]] = neg
    x[idx[2 * q:2 * q + q // 2]] = 0.0
    x[idx[2 * q + q // 2:3 * q]] = -0.0
    x[idx[3 * q:3 * q + q // 2]] = float("inf")
    x[idx[3 * q + q // 2:4 * q]] = -float("inf")
    return x


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("out_dtype", [torch.float8_e4m3fn, torch.float8_e5m2], ids=["e4m3", "e5m2"])
@pytest.mark.parametrize("scale_bits", [0x3F800000, 0x3E000000, 0x00000000, 0x7F800000, 0x7FC00000, -0x400000],
                         ids=["1", "0.125", "0", "inf", "nan", "-nan"])
@pytest.mark.parametrize("n", [64, 4096, 5184])
def test_quantize_fp8_nan_bytes(dtype, out_dtype, scale_bits, n, hip, dev):
    """NaN code bytes exactly as eager writes them (vectorised loop: n is a multiple of 64),
    for NaN inputs of both signs, 0 * inf, and NaN / zero / infinite scales; 4096 and 5184
    elements take the persistent kernel (16-bit input; 5184 leaves a remainder past the
    last 1024-element tile) or the vector kernel (fp32), 64 the scalar path."""
    g = torch.Generator().manual_seed(n + scale_bits)
    x = _nan_mix(dtype, n, g)
    scale = torch.tensor([scale_bits], dtype=torch.int32).view(torch.float32)
    want = ref.quantize_per_tensor_fp8(x.clone(), scale, out_dtype)
    got = ck.quantize_per_tensor_fp8(x.to(dev), scale.to(dev), out_dtype)
    _fp8_equal(got, want, out_dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(1000, 1000), (1024, 2048), (7, 13), (1,), (0, 5)])
def test_quantize_fp8_random(dtype, shape, hip, dev, seed):
    x = (torch.randn(shape) * 30).to(dtype)
    scale = torch.tensor([0.173])
    want = ref.quantize_per_tensor_fp8(x.clone(), scale)
    got = ck.quantize_per_tensor_fp8(x.to(dev), scale.to(dev))
    assert got.shape == x.shape and got.dtype == torch.float8_e4m3fn
    _fp8_equal(got, want)


def test_quantize_fp8_misaligned_view(hip, dev, seed):
    """A 2-byte-offset view takes the scalar path and still matches."""
    x = (torch.randn(4097) * 5).bfloat16()
    want = ref.quantize_per_tensor_fp8(x[1:].clone(), torch.tensor([0.05]))
    xd = x.to(dev)[1:]
    got = ck.quantize_per_tensor_fp8(xd, torch.tensor([0.05], device=dev))
    _fp8_equal(got, want)


@pytest.mark.parametrize("in_dtype", [torch.float8_e4m3fn, torch.float8_e5m2], ids=["e4m3", "e5m2"])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("scale", [1.0, 1.0048828125, 0.00123, 371.5])
def test_dequantize_fp8_every_code(in_dtype, out_dtype, scale, hip, dev):
    q = torch.arange(256, dtype=torch.int32).to(torch.uint8).repeat(40).view(in_dtype)
    s = torch.tensor([scale])
    want = ref.dequantize_per_tensor_fp8(q, s, out_dtype)
    got = ck.dequantize_per_tensor_fp8(q.to(dev), s.to(dev), out_dtype)
    assert got.dtype == out_dtype
    w, g = want.float(), got.cpu().float()
    nan = torch.isnan(w)
    assert torch.equal(nan, torch.isnan(g))
    assert torch.equal(bits(got)[~nan], bits(want)[~nan])


@pytest.mark.parametrize("in_dtype", [torch.float8_e4m3fn, torch.float8_e5m2], ids=["e4m3", "e5m2"])
@pytest.mark.parametrize("scale_dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_dequantize_fp8_16bit_scale(in_dtype, scale_dtype, out_dtype, hip, dev):
    """A f16 / bf16 scale, as eager accepts it (backends/eager/__init__.py:52-58): widened
    exactly, then rounded to the output dtype (scale.to(out)), for every code."""
    q = torch.arange(256, dtype=torch.int32).to(torch.uint8).repeat(40).view(in_dtype)
    for sv in (1.0, 1.0048828125, 0.00123, 371.5, 3.1e-5, 6.0e4):
        s = torch.tensor([sv]).to(scale_dtype)
        want = ref.dequantize_per_tensor_fp8(q, s, out_dtype)
        got = ck.dequantize_per_tensor_fp8(q.to(dev), s.to(dev), out_dtype)
        assert got.dtype == out_dtype
        nan = torch.isnan(want.float())
        assert torch.equal(nan, torch.isnan(got.cpu().float())), sv
        assert torch.equal(bits(got)[~nan], bits(want)[~nan]), sv


def test_c1_full_size_round_trip(hip, dev):
    """Config 1 at full size: codes bit-exact vs the oracle, dequantize bit-exact."""
    import bench

    x, scale = bench.make_c1()
    want_q = ref.quantize_per_tensor_fp8(x.clone(), scale)
    want_dq = ref.dequantize_per_tensor_fp8(want_q, scale)
    q = ck.quantize_per_tensor_fp8(x.to(dev), scale.to(dev))
    _fp8_equal(q, want_q)
    dq = ck.dequantize_per_tensor_fp8(q, scale.to(dev))
    assert torch.equal(bits(dq), bits(want_dq))


# ----------------------------------------------------------------- MXFP8
def _check_mx(x, pad):
    want_q, want_s = ref.quantize_mxfp8(x, pad_32x=pad)
    q, s = ck.quantize_mxfp8(x.cuda(), pad_32x=pad)
    assert q.shape == want_q.shape and s.shape == want_s.shape
    assert q.dtype == torch.float8_e4m3fn and s.dtype == torch.float8_e8m0fnu
    assert torch.equal(bits(s), bits(want_s)), "scale bytes differ"
    _fp8_equal(q, want_q)
    return q, s


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("m,k", [(1024, 2048), (512, 1024), (128, 256), (96, 32), (130, 4128), (130, 256), (1, 128),
                                 (257, 640)])
def test_quantize_mxfp8(dtype, m, k, hip, seed):
    x = (torch.randn(m, k) * torch.exp(torch.randn(m, 1) * 2)).to(dtype)
    x[0, :32] = 0  # zero block
    x[-1, :31] = 0
    x[-1, 31] = -3.0
    _check_mx(x, pad=False)


@pytest.mark.parametrize("m,k", [(65, 96), (33, 64), (100, 100), (1, 1), (129, 31)])
def test_quantize_mxfp8_padded(m, k, hip, seed):
    x = (torch.randn(m, k) * 10).bfloat16()
    _check_mx(x, pad=True)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_quantize_mxfp8_special_blocks(dtype, hip, seed):
    # 16-bit inputs with cols % 128 == 0 take the packed fast path; blocks with a zero,
    # tiny, infinite or NaN amax must leave it for the general encoder.
    m, k = 200, 384
    x = torch.randn(m, k) * torch.exp(torch.randn(m, 1) * 6)
    x[2, :32] = 0.0
    x[3, 32:64] = -0.0
    x[4, :32] = 1e-39  # subnormal in f32/bf16, zero in f16
    x[5, 64:96] = float("inf")
    x[6, 96:128] = float("-inf")
    x[7, 7] = float("nan")
    x[8, 40] = float("inf")
    x[9, :32] = 2.0 ** -120
    x[10, 128:160] = 65504.0
    x[11, 200] = float("nan")
    x[11, 201] = -1.0
    x = x.to(dtype)
    _check_mx(x, pad=False)


def test_quantize_mxfp8_config3_full(hip):
    import bench

    _check_mx(bench.make_c3(), pad=False)


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_dequantize_mxfp8(out_dtype, hip, seed):
    x = (torch.randn(256, 512) * torch.exp(torch.randn(256, 1) * 4)).bfloat16()
    q, s = ref.quantize_mxfp8(x)
    want = ref.dequantize_mxfp8(q, s, out_dtype)
    got = ck.dequantize_mxfp8(q.cuda(), s.cuda(), out_dtype)
    assert torch.equal(bits(got), bits(want))


def _same_or_both_nan(got: torch.Tensor, want: torch.Tensor) -> bool:
    """Bit-exact except that a NaN only has to be a NaN: dequantizing a NaN code or scale,
    or 0 * inf, gives the GPU's NaN payload, not the x86 payload of the CPU oracle."""
    got = got.cpu()
    nan_g, nan_w = torch.isnan(got.float()), torch.isnan(want.float())
    return torch.equal(nan_g, nan_w) and torch.equal(bits(got)[~nan_w], bits(want)[~nan_w])


def _misaligned(q: torch.Tensor, offset: int) -> torch.Tensor:
    """q on the GPU at a data pointer `offset` bytes past a 16-byte boundary."""
    buf = torch.zeros(q.numel() + offset, dtype=torch.uint8, device="cuda")
    buf[offset:] = q.reshape(-1).view(torch.uint8).cuda()
    return buf[offset:].view(q.dtype).view(q.shape)


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_dequantize_mxfp8_every_code_and_scale(out_dtype, hip, seed):
    # raw bytes: every E4M3 code (NaN included) and every E8M0 scale (0 -> 0.0, 255 ->
    # inf), 200 rows (padded scale rows); 16-bit outputs take the fast kernel, f32 output
    # the general one, and an 8-byte-offset view of the codes runs either
    rows, cols = 200, 320
    q = torch.randint(0, 256, (rows, cols), dtype=torch.uint8)
    q[0, :256] = torch.arange(256, dtype=torch.uint8)
    e = torch.randint(0, 256, (rows, cols // 32), dtype=torch.uint8)
    e.view(-1)[:256] = torch.arange(256, dtype=torch.uint8)
    q = q.view(torch.float8_e4m3fn)
    s = ref.to_blocked(e).view(torch.float8_e8m0fnu)
    want = ref.dequantize_mxfp8(q, s, out_dtype)
    assert _same_or_both_nan(ck.dequantize_mxfp8(q.cuda(), s.cuda(), out_dtype), want)
    assert _same_or_both_nan(ck.dequantize_mxfp8(_misaligned(q, 8), s.cuda(), out_dtype), want)


@pytest.mark.parametrize("hi_first", [True, False])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("cols", [320, 48, 512])
def test_dequantize_nvfp4_every_code_and_scale(cols, out_dtype, hi_first, hip, seed):
    # raw bytes: every code byte and every E4M3 scale byte (NaN included); 16-bit outputs
    # take the 256-column tile kernel (cols 512; 200 rows end inside a 128-row tile) or
    # the piece kernel (320, 48: a partial wave), f32 output the general one
    rows = 200
    q = torch.randint(0, 256, (rows, cols // 2), dtype=torch.uint8)
    q.view(-1)[:256] = torch.arange(256, dtype=torch.uint8)
    e = torch.randint(0, 256, (rows, cols // 16), dtype=torch.uint8)
    e.view(-1)[:256] = torch.arange(256, dtype=torch.uint8)
    s = ref.to_blocked(e).view(torch.float8_e4m3fn)
    for gv in [0.0123, 0.0, 3e38]:
        g = torch.tensor([gv])
        want = ref.dequantize_nvfp4(q, g, s, out_dtype, hi_first=hi_first)
        got = ck.dequantize_nvfp4(q.cuda(), g.cuda(), s.cuda(), out_dtype, hi_first=hi_first)
        assert _same_or_both_nan(got, want), gv


# ----------------------------------------------------------------- NVFP4
def _check_nv(x, g, pad, hi_first=True):
    want_q, want_s = ref.quantize_nvfp4(x, g, pad_16x=pad, hi_first=hi_first)
    q, s = ck.quantize_nvfp4(x.cuda(), g.cuda(), pad_16x=pad, hi_first=hi_first)
    assert q.shape == want_q.shape and s.shape == want_s.shape
    assert q.dtype == torch.uint8 and s.dtype == torch.float8_e4m3fn
    assert torch.equal(bits(s), bits(want_s)), "scale bytes differ"
    assert torch.equal(q.cpu(), want_q), f"{int((q.cpu() != want_q).sum())} code bytes differ"
    return q, s


@pytest.mark.parametrize("hi_first", [True, False])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("m,k", [(1024, 2048), (512, 1024), (128, 256), (16, 64), (130, 192), (1, 64), (257, 320),
                                 (130, 1600)])
def test_quantize_nvfp4(dtype, m, k, hi_first, hip, seed):
    x = (torch.randn(m, k) * torch.exp(torch.randn(m, 1))).to(dtype)
    x[0, :16] = 0
    g = (x.float().abs().amax() / 2688).reshape(1)
    _check_nv(x, g, pad=False, hi_first=hi_first)


@pytest.mark.parametrize("hi_first", [True, False])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_quantize_nvfp4_special_blocks(dtype, hi_first, hip, seed):
    # 16-bit inputs with cols % 64 == 0 take the fast path (one reciprocal per block and
    # a Markstein step per element); blocks with a zero, infinite or NaN amax, and
    # values exactly on E2M1 rounding boundaries, must match the IEEE-division codes.
    m, k = 200, 256
    x = torch.randn(m, k) * torch.exp(torch.randn(m, 1) * 4)
    x[2, :16] = 0.0
    x[3, 16:32] = -0.0
    x[4, 0] = float("nan")
    x[5, 40] = float("inf")
    x[6, 48:64] = float("-inf")
    x[7, :16] = 1e-30
    x[9, 16:32] = 3e25  # amax above the fast scale path's range
    # one block whose amax gives T = g * 6 exactly: every boundary multiple of T/6
    x[8, :16] = torch.tensor([6.0, 0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, -0.25, -0.75, -1.25, -1.75, -2.5, -3.5, -5.0, 0.5])
    x = x.to(dtype)
    finite = x.float().abs().nan_to_num(0.0, 0.0, 0.0)
    g = (finite.amax() / 2688).reshape(1)
    _check_nv(x, g, pad=False, hi_first=hi_first)


@pytest.mark.parametrize("g", [1.0, 1e-30, 1e-40, 0.0, -0.0, -0.01, 1e20, 3.0e-3, float("inf"), float("nan")])
def test_quantize_nvfp4_global_scale_edges(g, hip, seed):
    # global scales outside the fast path's range (zero, subnormal, negative, huge) take
    # the IEEE-division path inside the same kernel.  With g = 0 the all-zero block's
    # 0/0 and with g = inf the infinite block's inf/inf are invalid divisions: x86 gives
    # the negative default NaN, so scale byte 0xFF and negative-NaN codes.
    x = torch.randn(130, 128) * torch.exp(torch.randn(130, 1) * 3)
    x[2, :16] = 0.0
    x[3, 16] = float("inf")
    # with g = 1 this block has T = 1 exactly, so its values sit on the E2M1 rounding
    # boundaries (ties go to the even code)
    x[1, :16] = torch.tensor([6.0, 0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, -0.25, -0.75, -1.25, -1.75, -2.5, -3.5, -5.0, 0.5])
    _check_nv(x.bfloat16(), torch.tensor([g], dtype=torch.float32), pad=False)


@pytest.mark.parametrize("m,k", [(129, 128), (33, 65), (100, 100), (1, 1)])
def test_quantize_nvfp4_padded(m, k, hip, seed):
    x = (torch.randn(m, k) * 4).bfloat16()
    g = (x.float().abs().amax() / 2688).reshape(1)
    _check_nv(x, g, pad=True)


def test_quantize_nvfp4_config5_activation_full(hip):
    import bench

    a, _, ga, _ = bench.make_c5()
    _check_nv(a, ga, pad=False)


def test_nvfp4_hi_first_swap_on_gpu(hip, seed):
    x = (torch.randn(64, 128) * 4).bfloat16().cuda()
    g = (x.float().abs().amax() / 2688).reshape(1)
    qh, sh = ck.quantize_nvfp4(x, g, hi_first=True)
    ql, sl = ck.quantize_nvfp4(x, g, hi_first=False)
    assert torch.equal(ck.swap_nibbles(qh), ql)
    assert torch.equal(bits(sh), bits(sl))


@pytest.mark.parametrize("hi_first", [True, False])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_dequantize_nvfp4(out_dtype, hi_first, hip, seed):
    x = (torch.randn(256, 512) * torch.exp(torch.randn(256, 1))).bfloat16()
    g = (x.float().abs().amax() / 2688).reshape(1)
    q, s = ref.quantize_nvfp4(x, g, hi_first=hi_first)
    want = ref.dequantize_nvfp4(q, g, s, out_dtype, hi_first=hi_first)
    got = ck.dequantize_nvfp4(q.cuda(), g.cuda(), s.cuda(), out_dtype, hi_first=hi_first)
    assert torch.equal(bits(got), bits(want))


@pytest.mark.parametrize("case", range(len(kat.dequantize_nvfp4_cases())))
@pytest.mark.parametrize("hi_first", [True, False])
def test_dequantize_nvfp4_known_answers(case, hi_first, hip):
    """The block total and the element product round in the output dtype."""
    dt, _, g, sbyte, c4, want = kat.dequantize_nvfp4_cases()[case]
    q, s = kat.nvfp4_block(c4, sbyte)
    out = ck.dequantize_nvfp4(q.cuda(), g.cuda(), s.cuda(), dt, hi_first=hi_first)
    assert set((bits(out).int() & 0xFFFF).reshape(-1).tolist()) == {want}


# ------------------------------------------------------------ dynamic scales
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("n", [1, 7, 4096, 1000003, 4096 * 3072])
@pytest.mark.parametrize("divisor", [448.0, 2688.0])
def test_amax_scale_matches_torch(dtype, n, divisor, hip, seed):
    x = (torch.randn(n) * torch.exp(torch.randn(1) * 3)).to(dtype)
    want = ref.default_scale(x, divisor)
    got = ck.amax_scale(x.cuda(), divisor)
    assert got.shape == () and got.dtype == torch.float32
    assert torch.equal(got.cpu().view(torch.int32), want.view(torch.int32))
    # the reference expression itself, evaluated by torch on the device (tensor/fp8.py:57)
    on_device = (torch.amax(x.cuda().abs()) / divisor).float()
    assert torch.equal(got.cpu().view(torch.int32), on_device.cpu().view(torch.int32))


@pytest.mark.parametrize("case", range(len(kat.default_scale_cases())))
def test_amax_scale_known_answers(case, hip):
    x, _, divisor, want = kat.default_scale_cases()[case]
    xs = torch.cat([x, -x / 2, x * 0]).cuda()
    got = ck.amax_scale(xs, divisor)
    assert int(got.view(torch.int32).cpu()) & 0xFFFFFFFF == want


@pytest.mark.parametrize("divisor", [448.0, 57344.0])
def test_amax_scale_tiny_f16_follows_the_device_division(divisor, hip):
    """The f16 amaxes whose quotient torch's CPU and GPU kernels round differently: the
    kernel gives the GPU's (reciprocal-multiply) value, as the oracle does."""
    f16 = torch.arange(0, 0x7C00, dtype=torch.int32).to(torch.int16).view(torch.float16)
    cpu_div = (f16 / divisor).float()
    dev_div = (f16.cuda() / divisor).float().cpu()
    split = f16[cpu_div.view(torch.int32) != dev_div.view(torch.int32)]
    assert 0 < split.numel() < 100
    for v in split:
        x = torch.stack([v, -v]).cuda()
        got = ck.amax_scale(x, divisor).cpu()
        assert torch.equal(got.view(torch.int32), (torch.amax(x.abs()) / divisor).float().cpu().view(torch.int32))
        assert torch.equal(got.view(torch.int32), ref.default_scale(x.cpu(), divisor).view(torch.int32))


@pytest.mark.parametrize("n", [8192 * 5120, 8192 * 5120 + 5])
def test_amax_scale_full_grid(n, hip, seed):
    # enough chunks for every workgroup of the partial pass to run two batches; the
    # largest magnitude sits in the last 16-byte chunk, or in the scalar tail
    x = torch.randn(n).bfloat16()
    x[n - 1] = -977.0
    want = ref.default_scale(x, 2688.0)
    assert torch.equal(ck.amax_scale(x.cuda(), 2688.0).cpu(), want)
    x[n - 1] = 0.5
    x[n // 3] = 611.0
    assert torch.equal(ck.amax_scale(x.cuda(), 2688.0).cpu(), ref.default_scale(x, 2688.0))


def test_amax_scale_misaligned_nan_and_sign(hip, seed):
    x = torch.randn(4099).bfloat16()
    x[1000] = -1234.5  # the amax is taken of |x|
    got = ck.amax_scale(x.cuda()[3:], 448.0)  # a view 6 bytes into the buffer
    assert torch.equal(got.cpu(), ref.default_scale(x[3:], 448.0))
    x[77] = float("nan")
    assert torch.isnan(ck.amax_scale(x.cuda(), 448.0)).item()


@pytest.mark.parametrize("layout", ["TensorCoreFP8Layout", "TensorCoreNVFP4Layout"])
def test_layout_dynamic_scale_uses_the_reference_default(layout, hip, seed):
    from comfy_kitchen.tensor import QuantizedTensor

    x = (torch.randn(256, 512) * 3).bfloat16()
    qt = QuantizedTensor.from_float(x.cuda(), layout)
    want = ref.default_scale(x, 448.0 if layout == "TensorCoreFP8Layout" else 2688.0)
    assert torch.equal(qt._params.scale.reshape(()).cpu(), want)
    if layout == "TensorCoreFP8Layout":
        _fp8_equal(qt._qdata, ref.quantize_per_tensor_fp8(x, want.reshape(1)))
    else:
        q, s = ref.quantize_nvfp4(x, want.reshape(1))
        assert torch.equal(qt._qdata.cpu(), q)
        assert torch.equal(bits(qt._params.block_scale), bits(s))


# ----------------------------------------------------- fused dynamic NVFP4 quantize
def _check_nv_dynamic(x, pad=False, hi_first=True, oracle=True):
    """quantize_nvfp4_dynamic == amax_scale + quantize_nvfp4 on the device, and (oracle=True)
    == the oracle's default_scale + quantize_nvfp4, bit for bit (codes, block scales, scale)."""
    xd = x.cuda()
    q, s, g = ck.quantize_nvfp4_dynamic(xd, 2688.0, pad_16x=pad, hi_first=hi_first)
    assert g.shape == () and g.dtype == torch.float32
    g2 = ck.amax_scale(xd, 2688.0)
    q2, s2 = ck.quantize_nvfp4(xd, g2, pad_16x=pad, hi_first=hi_first)
    assert torch.equal(bits(g), bits(g2)), (g.item(), g2.item())
    assert torch.equal(q, q2), f"{int((q != q2).sum())} code bytes differ from the two-call path"
    assert torch.equal(bits(s), bits(s2)), "block scales differ from the two-call path"
    if oracle:
        want_g = ref.default_scale(x, 2688.0)
        assert torch.equal(bits(g), bits(want_g)), (g.item(), want_g.item())
        want_q, want_s = ref.quantize_nvfp4(x, want_g.reshape(1), pad_16x=pad, hi_first=hi_first)
        assert torch.equal(q.cpu(), want_q) and torch.equal(bits(s), bits(want_s))


@pytest.mark.parametrize("hi_first", [True, False])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("m,k,pad", [(1024, 2048, False), (512, 1024, False), (130, 192, False), (257, 320, False),
                                     (1, 64, False), (16, 1600, False), (33, 65, True), (129, 128, True)])
def test_quantize_nvfp4_dynamic(dtype, m, k, pad, hi_first, hip, seed):
    x = (torch.randn(m, k) * torch.exp(torch.randn(m, 1) * 2)).to(dtype)
    x[0, :16] = 0
    _check_nv_dynamic(x, pad=pad, hi_first=hi_first)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", ["zeros", "nan", "inf", "tiny", "huge"])
def test_quantize_nvfp4_dynamic_special(dtype, case, hip, seed):
    x = torch.randn(256, 512) * torch.exp(torch.randn(256, 1))
    if case == "zeros":
        x.zero_()
    elif case == "nan":
        x[100, 37] = float("nan")
    elif case == "inf":
        x[7, 300] = float("-inf")
    elif case == "tiny":
        x *= 1e-6
    else:
        x *= 1e4 if dtype == torch.float16 else 1e30
    x = x.to(dtype)
    _check_nv_dynamic(x, oracle=case != "nan")  # NaN payloads: compared with the device path only


def test_quantize_nvfp4_dynamic_config5_activation(hip):
    import bench

    a, _, _, _ = bench.make_c5()
    ad = a.cuda()
    q, s, g = ck.quantize_nvfp4_dynamic(ad, 2688.0)
    assert torch.equal(bits(g), bits(ref.default_scale(a, 2688.0)))
    q2, s2 = ck.quantize_nvfp4(ad, g.reshape(1))
    assert torch.equal(q, q2) and torch.equal(bits(s), bits(s2))
    _check_nv(a, g.cpu().reshape(1), pad=False)


@pytest.mark.parametrize("m,k", [(32768, 768), (24576, 960)])
def test_quantize_nvfp4_dynamic_many_partial_words(m, k, hip, seed):
    """Narrow rows (cols < 1024: 256-thread quantize workgroups) with more amax partial
    words than threads, so each thread reduces several of them: the fused path equals
    amax_scale + quantize_nvfp4 on the device, and its scale equals torch's expression
    evaluated on the device (tensor/nvfp4.py:65)."""
    x = (torch.randn(m, k, device="cuda") * torch.exp(torch.randn(m, 1, device="cuda"))).bfloat16()
    x[m // 2, 5] = 30000.0  # the maximum sits deep in the tensor
    q, s, g = ck.quantize_nvfp4_dynamic(x, 2688.0)
    want = (torch.amax(x.abs()) / 2688.0).float()
    assert torch.equal(bits(g), bits(want)), (g.item(), want.item())
    q2, s2 = ck.quantize_nvfp4(x, ck.amax_scale(x, 2688.0))
    assert torch.equal(q, q2) and torch.equal(bits(s), bits(s2))
