"""HIP block-scaled GEMMs vs an fp32 matmul of the dequantized operands.

rel-L2 <= 1e-2 against fp32 matmul of the dequantized operands.  The
kernels multiply the quantized values exactly and accumulate in fp32 MFMAs, so they
are held far tighter: 1e-4 with an fp32 output (the MFMA's internal reduction is not
a sequentially rounded fp32 sum; measured ~1.5e-5), and the output rounding with
bf16/f16 outputs (2^-8 relative per element, well under 1e-2 in L2).
"""
import pytest
import torch

import comfy_kitchen as ck
from oracle import eager_ref as ref

pytestmark = pytest.mark.gpu

# fp32 output: the MFMA reduction is not an fp32-rounded sequential sum (measured ~1.5e-5)
REL_L2 = {torch.float32: 1e-4, torch.float16: 1e-3, torch.bfloat16: 4e-3}


def rel_l2(got: torch.Tensor, want: torch.Tensor) -> float:
    got, want = got.float().cpu(), want.float().cpu()
    return ((got - want).norm() / want.norm().clamp_min(1e-30)).item()


def mx_operands(m, n, k, seed, wscale=0.02):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(m, k, generator=g) * torch.exp(torch.randn(m, 1, generator=g))).bfloat16()
    w = (torch.randn(n, k, generator=g) * wscale).bfloat16()
    qx, sx = ref.quantize_mxfp8(x, pad_32x=(k % 32 != 0))
    qw, sw = ref.quantize_mxfp8(w, pad_32x=(k % 32 != 0))
    return qx, sx, qw, sw


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("m,n,k", [(256, 256, 256), (128, 512, 1024), (512, 256, 3072), (100, 300, 256),
                                   (33, 17, 96), (260, 520, 160), (1, 64, 32), (257, 255, 224)])
def test_scaled_mm_mxfp8_vs_oracle(m, n, k, out_dtype, hip):
    qx, sx, qw, sw = mx_operands(m, n, k, seed=m * 7 + n + k)
    want = ref.scaled_mm_mxfp8_ref(qx, qw, sx, sw, out_dtype=torch.float32)
    got = ck.scaled_mm_mxfp8(qx.cuda(), qw.cuda(), sx.cuda(), sw.cuda(), out_dtype=out_dtype)
    assert got.shape == (m, n) and got.dtype == out_dtype
    assert rel_l2(got, want) <= REL_L2[out_dtype]


def test_scaled_mm_one_round_grid_with_weight_prefetch(hip):
    """256 x 18432 x 3072 runs as 144 half tiles, and the other 112 CUs run workgroups that
    read the weight ahead of the tiles (they write nothing): MXFP8 and per-tensor FP8
    against the oracle on the first and last 1024 output columns (swizzled scale rows of
    whole 128-row blocks slice like the weight)."""
    m, n, k = 256, 18432, 3072
    qx, sx, qw, sw = mx_operands(m, n, k, seed=77)
    got = ck.scaled_mm_mxfp8(qx.cuda(), qw.cuda(), sx.cuda(), sw.cuda(), out_dtype=torch.bfloat16).cpu()
    ta, tb = torch.tensor([0.5]), torch.tensor([3e-3])
    got8 = ck.scaled_mm_fp8(qx.cuda(), qw.cuda(), ta.cuda(), tb.cuda(), out_dtype=torch.bfloat16).cpu()
    for cols in (slice(0, 1024), slice(n - 1024, n)):
        want = ref.scaled_mm_mxfp8_ref(qx, qw[cols], sx, sw[cols], out_dtype=torch.float32)
        assert rel_l2(got[:, cols], want) <= REL_L2[torch.bfloat16]
        want8 = (qx.float() @ qw[cols].float().t()) * (ta * tb)
        assert rel_l2(got8[:, cols], want8) <= REL_L2[torch.bfloat16]


@pytest.mark.parametrize("bias_dtype", [torch.bfloat16, torch.float32, torch.float16])
def test_scaled_mm_mxfp8_bias(bias_dtype, hip):
    qx, sx, qw, sw = mx_operands(192, 384, 512, seed=5)
    bias = (torch.randn(384) * 2).to(bias_dtype)
    want = ref.scaled_mm_mxfp8_ref(qx, qw, sx, sw, bias=bias, out_dtype=torch.float32)
    got = ck.scaled_mm_mxfp8(qx.cuda(), qw.cuda(), sx.cuda(), sw.cuda(), bias=bias.cuda(), out_dtype=torch.float32)
    assert rel_l2(got, want) <= REL_L2[torch.float32]


def test_scaled_mm_mxfp8_extreme_scales(hip):
    """Rows spanning ~2^±40 of magnitude: the E8M0 scales, not the codes, carry the range."""
    g = torch.Generator().manual_seed(11)
    x = torch.randn(128, 512, generator=g) * torch.exp2(torch.randint(-40, 40, (128, 1), generator=g).float())
    w = torch.randn(256, 512, generator=g) * torch.exp2(torch.randint(-20, 20, (256, 16), generator=g).float()
                                                        ).repeat_interleave(32, dim=1)
    qx, sx = ref.quantize_mxfp8(x.bfloat16())
    qw, sw = ref.quantize_mxfp8(w.bfloat16())
    want = ref.scaled_mm_mxfp8_ref(qx, qw, sx, sw, out_dtype=torch.float32)
    got = ck.scaled_mm_mxfp8(qx.cuda(), qw.cuda(), sx.cuda(), sw.cuda(), out_dtype=torch.float32)
    # compare row-normalised: each output row has its own magnitude
    d = (got.cpu() - want) / want.abs().amax(dim=1, keepdim=True).clamp_min(1e-30)
    assert d.abs().max().item() <= 5e-4


@pytest.mark.parametrize("out_dtype,with_bias", [(torch.bfloat16, False), (torch.float16, True), (torch.float32, True)])
def test_scaled_mm_mxfp8_half_tile_tail(out_dtype, with_bias, hip):
    """289 tiles of 256 x 256: 256 run as full tiles, the last 33 as 66 half-width tiles
    (partial ones at the right edge, one wholly past N)."""
    m, n, k = 4352, 4196, 128
    qx, sx, qw, sw = mx_operands(m, n, k, seed=21)
    bias = (torch.randn(n) * 2).float() if with_bias else None
    want = ref.scaled_mm_mxfp8_ref(qx, qw, sx, sw, bias=bias, out_dtype=torch.float32)
    got = ck.scaled_mm_mxfp8(qx.cuda(), qw.cuda(), sx.cuda(), sw.cuda(),
                             bias=None if bias is None else bias.cuda(), out_dtype=out_dtype)
    assert got.shape == (m, n) and got.dtype == out_dtype
    assert rel_l2(got, want) <= REL_L2[out_dtype]
    # The tiles are taken in groups of 6 tile rows, each group column by column: tiles
    # 256..288 lie in the last group (tile rows 12..16) at tile columns 10..16.
    assert rel_l2(got[12 * 256:, 10 * 256:], want[12 * 256:, 10 * 256:]) <= REL_L2[out_dtype]


def test_scaled_mm_mxfp8_config4_full(hip):
    """Config 4 at full size against a GPU fp32 matmul of the (bit-exact) dequantized operands."""
    import bench

    x = bench.make_c3("cuda")
    w = bench.make_c4_weight("cuda")
    qx, sx = ck.quantize_mxfp8(x)
    qw, sw = ck.quantize_mxfp8(w)
    got = ck.scaled_mm_mxfp8(qx, qw, sx, sw)
    dx = ck.dequantize_mxfp8(qx, sx, torch.float32)
    dw = ck.dequantize_mxfp8(qw, sw, torch.float32)
    want = torch.matmul(dx, dw.t().contiguous())
    assert got.shape == (4608, 12288) and got.dtype == torch.bfloat16
    r = ((got.float() - want).norm() / want.norm()).item()
    print(f"config 4 rel-L2 vs fp32 matmul of dequantized operands: {r:.3e}")
    assert r <= 4e-3
    # and a slice against the CPU oracle end to end
    rows = slice(0, 256)
    want_cpu = ref.scaled_mm_mxfp8_ref(qx[rows].cpu(), qw.cpu(), ref.to_blocked(
        ref.from_blocked(sx.cpu().view(torch.uint8), 4608, 96)[rows]).view(torch.float8_e8m0fnu), sw.cpu(),
        out_dtype=torch.float32)
    assert rel_l2(got[rows], want_cpu) <= 4e-3


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("m,n,k", [(1, 4096, 3072), (8, 200, 288), (9, 64, 1024), (16, 1000, 3072), (17, 1000, 3072),
                                   (31, 96, 224), (32, 4096, 64), (33, 130, 5120), (40, 33, 96), (64, 512, 1056),
                                   (2, 33, 32), (48, 18432, 128), (12, 8200, 320), (16, 4096, 3072),
                                   (20, 16400, 256), (30, 9000, 1088), (64, 16448, 320), (50, 12000, 4096),
                                   (63, 3000, 12288), (25, 160, 96), (64, 16384, 544), (36, 24576, 96),
                                   (33, 24600, 4160), (32, 16384, 320), (24, 18432, 544), (20, 32768, 96),
                                   (28, 20000, 4160), (6, 18440, 288), (4, 24576, 3104)])
def test_scaled_mm_mxfp8_skinny(m, n, k, out_dtype, hip):
    """At most 64 activation rows take the skinny kernel (a workgroup per 32 or 64 weight
    rows, K split over its waves; configurations by M, boundaries 8 / 16 / 32 / 64, and from
    9 rows on by N, boundaries 4096 / 8192 / 16384: waves per workgroup, weight tiles, and
    32 or 64 activation rows staged in LDS or loaded as fragments): rows past M, columns
    past N, K % 64 == 32, K past one chunk round and long K."""
    qx, sx, qw, sw = mx_operands(m, n, k, seed=m * 13 + n + k)
    want = ref.scaled_mm_mxfp8_ref(qx, qw, sx, sw, out_dtype=torch.float32)
    got = ck.scaled_mm_mxfp8(qx.cuda(), qw.cuda(), sx.cuda(), sw.cuda(), out_dtype=out_dtype)
    assert got.shape == (m, n) and got.dtype == out_dtype
    assert rel_l2(got, want) <= REL_L2[out_dtype]


@pytest.mark.parametrize("bias_dtype", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("m", [1, 12, 20, 40])
def test_scaled_mm_skinny_bias_and_per_tensor(bias_dtype, m, hip):
    """The skinny kernel's epilogue: bias of each dtype, and the per-tensor FP8 mode
    (ck.scaled_mm_fp8: unit block scales, out = scale_a * scale_b * A B^T + bias)."""
    n, k = 300, 640
    qx, sx, qw, sw = mx_operands(m, n, k, seed=m + 77)
    bias = (torch.randn(n) * 2).to(bias_dtype)
    want = ref.scaled_mm_mxfp8_ref(qx, qw, sx, sw, bias=bias, out_dtype=torch.float32)
    got = ck.scaled_mm_mxfp8(qx.cuda(), qw.cuda(), sx.cuda(), sw.cuda(), bias=bias.cuda(), out_dtype=torch.float32)
    assert rel_l2(got, want) <= REL_L2[torch.float32]
    ta, tb = torch.tensor([0.37]), torch.tensor([1.9e-3])
    want = (qx.float() @ qw.float().t()) * (ta * tb) + bias.float()
    for out_dtype in (torch.float32, torch.bfloat16):
        got = ck.scaled_mm_fp8(qx.cuda(), qw.cuda(), ta.cuda(), tb.cuda(), bias=bias.cuda(), out_dtype=out_dtype)
        assert got.shape == (m, n) and got.dtype == out_dtype
        assert rel_l2(got, want) <= REL_L2[out_dtype]


def _mx_abi(qx, qw, sx, sw, out_dtype, ws):
    """ckh_scaled_mm_mxfp8 through the C ABI with an explicit workspace (None: no split)."""
    import comfy_kitchen.backends.hip as hb

    m, k = qx.shape
    n = qw.shape[0]
    out = torch.empty(m, n, dtype=out_dtype, device="cuda")
    hb._call("ckh_scaled_mm_mxfp8", qx.data_ptr(), qw.data_ptr(), sx.data_ptr(), sw.data_ptr(), None, out.data_ptr(),
             m, n, k, hb.DTYPE_TO_CODE[out_dtype], 0, None if ws is None else ws.data_ptr(),
             0 if ws is None else ws.numel(), torch.cuda.current_stream().cuda_stream)
    return out


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("m,n,k", [(256, 4096, 4096), (300, 2000, 4160), (129, 520, 4128), (65, 18432, 4096),
                                   (512, 3072, 13824), (200, 2000, 2080)])
def test_scaled_mm_mxfp8_split_k(m, n, k, out_dtype, hip):
    """Grids of at most 128 tiles split K over more workgroups into a workspace, and a second
    launch adds the partial tiles (fixed order) and runs the epilogue: against the oracle,
    and against the same call with no workspace (whole-K half tiles), which differs only in
    fp32 summation order.  Covers a last K range shorter than the others (and than one
    group of 4 stages), K % 64 == 32, rows past M and columns past N."""
    import comfy_kitchen.backends.hip as hb

    nbytes = hb._lib.ckh_scaled_mm_workspace_bytes(m, n, k)
    assert nbytes > 0
    qx, sx, qw, sw = mx_operands(m, n, k, seed=m + 5 * n + k)
    want = ref.scaled_mm_mxfp8_ref(qx, qw, sx, sw, out_dtype=torch.float32)
    qx, sx, qw, sw = qx.cuda(), sx.cuda(), qw.cuda(), sw.cuda()
    ws = torch.full((nbytes,), 0xFF, dtype=torch.uint8, device="cuda")  # NaN garbage: every byte is rewritten
    got = _mx_abi(qx, qw, sx, sw, out_dtype, ws)
    assert rel_l2(got, want) <= REL_L2[out_dtype]
    assert torch.equal(got, _mx_abi(qx, qw, sx, sw, out_dtype, ws))  # deterministic
    whole = _mx_abi(qx, qw, sx, sw, out_dtype, None)
    if out_dtype == torch.float32:
        assert rel_l2(got, whole) <= 1e-6
    assert torch.equal(ck.scaled_mm_mxfp8(qx, qw, sx, sw, out_dtype=out_dtype), got)  # the wrapper splits too


@pytest.mark.parametrize("bias_dtype", [torch.bfloat16, torch.float32])
def test_scaled_mm_split_k_bias_and_per_tensor(bias_dtype, hip):
    """The split-K reduce kernel's epilogue: bias, and the per-tensor FP8 mode."""
    m, n, k = 200, 1000, 4096
    qx, sx, qw, sw = mx_operands(m, n, k, seed=31)
    bias = (torch.randn(n) * 2).to(bias_dtype)
    want = ref.scaled_mm_mxfp8_ref(qx, qw, sx, sw, bias=bias, out_dtype=torch.float32)
    got = ck.scaled_mm_mxfp8(qx.cuda(), qw.cuda(), sx.cuda(), sw.cuda(), bias=bias.cuda(), out_dtype=torch.float32)
    assert rel_l2(got, want) <= REL_L2[torch.float32]
    ta, tb = torch.tensor([0.37]), torch.tensor([1.9e-3])
    want = (qx.float() @ qw.float().t()) * (ta * tb) + bias.float()
    for out_dtype in (torch.float32, torch.bfloat16):
        got = ck.scaled_mm_fp8(qx.cuda(), qw.cuda(), ta.cuda(), tb.cuda(), bias=bias.cuda(), out_dtype=out_dtype)
        assert rel_l2(got, want) <= REL_L2[out_dtype]


def test_scaled_mm_workspace_bytes(hip):
    """Only small tile grids with enough K split; big grids, skinny M and short K do not.
    At most 64 tiles split as half tiles (two 128 KB partials per tile and K range)."""
    import comfy_kitchen.backends.hip as hb

    f = hb._lib.ckh_scaled_mm_workspace_bytes
    assert f(256, 13824, 5120) == 54 * 2 * 256 * 256 * 4  # 108 half tiles, 80 stages: 2 ranges of 40
    assert f(256, 5120, 13824) == 20 * 6 * 256 * 256 * 4  # 40 half tiles, 216 stages: 6 ranges of 36
    assert f(256, 32768, 5120) == 0  # 128 tiles, 2 ranges: whole-K half tiles instead
    assert f(256, 18432, 8192) == 72 * 3 * 256 * 256 * 4  # 72 full tiles, 128 stages: 3 ranges of 44
    assert f(256, 9216, 3072) == 36 * 3 * 256 * 256 * 4  # 72 half tiles, 48 stages: 3 ranges of 16
    assert f(4608, 12288, 13824) == 0  # 864 tiles
    assert f(64, 18432, 13824) == 0  # skinny kernel
    assert f(256, 18432, 3072) == 0  # 72 tiles, 48 stages: whole-K half tiles
    assert f(256, 4096, 1984) == 0  # 31 stages
    assert f(0, 4096, 8192) == 0 and f(256, 4096, -1) == 0


def test_scaled_mm_mxfp8_rejects_bad_shapes(hip):
    a = torch.zeros(64, 96, dtype=torch.float8_e4m3fn, device="cuda")
    b = torch.zeros(64, 64, dtype=torch.float8_e4m3fn, device="cuda")
    s = torch.zeros(128, 4, dtype=torch.float8_e8m0fnu, device="cuda")
    with pytest.raises((ValueError, RuntimeError)):
        ck.scaled_mm_mxfp8(a, b, s, s)


# --------------------------------------------------------------------- NVFP4
def nv_operands(m, n, k, seed, wscale=0.02):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g).bfloat16()
    w = (torch.randn(n, k, generator=g) * wscale).bfloat16()
    gx = (x.float().abs().amax() / 2688).reshape(1)
    gw = (w.float().abs().amax() / 2688).reshape(1)
    qx, sx = ref.quantize_nvfp4(x, gx)
    qw, sw = ref.quantize_nvfp4(w, gw)
    return qx, sx, gx, qw, sw, gw


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("m,n,k", [(256, 256, 256), (128, 512, 1024), (512, 256, 5120), (100, 300, 256),
                                   (33, 17, 96), (260, 520, 160), (16, 64, 32), (257, 255, 224)])
def test_scaled_mm_nvfp4_vs_oracle(m, n, k, out_dtype, hip):
    qx, sx, gx, qw, sw, gw = nv_operands(m, n, k, seed=m + 3 * n + k)
    want = ref.scaled_mm_nvfp4_ref(qx, qw, gx, gw, sx, sw, out_dtype=torch.float32)
    got = ck.scaled_mm_nvfp4(qx.cuda(), qw.cuda(), gx.cuda(), gw.cuda(), sx.cuda(), sw.cuda(), out_dtype=out_dtype)
    assert got.shape == (m, n) and got.dtype == out_dtype
    assert rel_l2(got, want) <= REL_L2[out_dtype]


@pytest.mark.parametrize("bias_dtype", [torch.bfloat16, torch.float32])
def test_scaled_mm_nvfp4_bias_and_alpha(bias_dtype, hip):
    qx, sx, gx, qw, sw, gw = nv_operands(192, 384, 512, seed=9)
    bias = (torch.randn(384) * 0.1).to(bias_dtype)
    want = ref.scaled_mm_nvfp4_ref(qx, qw, gx, gw, sx, sw, bias=bias, out_dtype=torch.float32)
    got = ck.scaled_mm_nvfp4(qx.cuda(), qw.cuda(), gx.cuda(), gw.cuda(), sx.cuda(), sw.cuda(), bias=bias.cuda(),
                             out_dtype=torch.float32)
    assert rel_l2(got, want) <= REL_L2[torch.float32]
    # explicit alpha overrides tensor_scale_a * tensor_scale_b
    alpha = (gx * gw * 2).cuda()
    got2 = ck.scaled_mm_nvfp4(qx.cuda(), qw.cuda(), gx.cuda(), gw.cuda(), sx.cuda(), sw.cuda(), out_dtype=torch.float32,
                              alpha=alpha)
    want2 = ref.scaled_mm_nvfp4_ref(qx, qw, gx * 2, gw, sx, sw, out_dtype=torch.float32)
    assert rel_l2(got2, want2) <= REL_L2[torch.float32]


@pytest.mark.parametrize("m", [128, 5])
def test_scaled_mm_nvfp4_hi_first_invariance(m, hip):
    """Packing order does not change the product when both operands share it (tile and
    skinny kernels)."""
    qx, sx, gx, qw, sw, gw = nv_operands(m, 256, 512, seed=2)
    a = ck.scaled_mm_nvfp4(qx.cuda(), qw.cuda(), gx.cuda(), gw.cuda(), sx.cuda(), sw.cuda(), out_dtype=torch.float32)
    b = ck.scaled_mm_nvfp4(ck.swap_nibbles(qx).cuda(), ck.swap_nibbles(qw).cuda(), gx.cuda(), gw.cuda(), sx.cuda(),
                           sw.cuda(), out_dtype=torch.float32)
    assert torch.equal(a, b)


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("m,n,k", [(1, 4096, 3072), (8, 200, 288), (9, 64, 1024), (16, 1000, 3072), (17, 1000, 3072),
                                   (31, 96, 224), (32, 4096, 64), (33, 130, 5120), (40, 33, 96), (64, 512, 1056),
                                   (2, 33, 32), (48, 13824, 128), (3, 160, 1536), (20, 8200, 256), (40, 8192, 96),
                                   (12, 40, 4096), (64, 3000, 5152), (17, 8100, 2080)])
def test_scaled_mm_nvfp4_skinny(m, n, k, out_dtype, hip):
    """At most 64 activation rows take the skinny NVFP4 kernel (a workgroup per 32 or 64
    weight rows, K split over its waves in chunks of 256 elements, two chunks in flight per
    wave; configurations by M (boundaries 8 / 16 / 32 / 64) and, past 16 rows, by N (two weight
    tiles from N = 8192)): rows past M, columns past N, K % 64 == 32 (a half-used scale word),
    fewer chunks than waves, K past one chunk round and long K."""
    qx, sx, gx, qw, sw, gw = nv_operands(m, n, k, seed=m * 13 + n + k)
    want = ref.scaled_mm_nvfp4_ref(qx, qw, gx, gw, sx, sw, out_dtype=torch.float32)
    got = ck.scaled_mm_nvfp4(qx.cuda(), qw.cuda(), gx.cuda(), gw.cuda(), sx.cuda(), sw.cuda(), out_dtype=out_dtype)
    assert got.shape == (m, n) and got.dtype == out_dtype
    assert rel_l2(got, want) <= REL_L2[out_dtype]


@pytest.mark.parametrize("k", [224, 1280, 2304, 2336])
@pytest.mark.parametrize("n", [96, 8200])
@pytest.mark.parametrize("m", [1, 8, 16, 24, 32, 48, 64])
def test_scaled_mm_nvfp4_skinny_chunks_per_wave(m, n, k, hip):
    """Every skinny configuration (by M, and one or two weight tiles by N) with 1, 5, 9 and
    10 chunks of 256 elements, i.e. 4 waves holding 0 to 3 chunks each: the paths from the
    prologue straight to the last step, through one loop iteration, and through the loop
    and the last step.  Each step's wait must cover its own chunk's LDS rows on every one of
    them (the staged activation rows included)."""
    qx, sx, gx, qw, sw, gw = nv_operands(m, n, k, seed=m * 31 + n + k)
    want = ref.scaled_mm_nvfp4_ref(qx, qw, gx, gw, sx, sw, out_dtype=torch.float32)
    got = ck.scaled_mm_nvfp4(qx.cuda(), qw.cuda(), gx.cuda(), gw.cuda(), sx.cuda(), sw.cuda(),
                             out_dtype=torch.float32)
    assert rel_l2(got, want) <= REL_L2[torch.float32]


@pytest.mark.parametrize("bias_dtype", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("m", [1, 12, 20, 40])
def test_scaled_mm_nvfp4_skinny_bias_and_alpha(bias_dtype, m, hip):
    """The skinny NVFP4 epilogue: alpha times the sum, plus bias of each dtype."""
    n, k = 300, 640
    qx, sx, gx, qw, sw, gw = nv_operands(m, n, k, seed=m + 91)
    bias = (torch.randn(n) * 0.1).to(bias_dtype)
    want = ref.scaled_mm_nvfp4_ref(qx, qw, gx, gw, sx, sw, bias=bias, out_dtype=torch.float32)
    got = ck.scaled_mm_nvfp4(qx.cuda(), qw.cuda(), gx.cuda(), gw.cuda(), sx.cuda(), sw.cuda(), bias=bias.cuda(),
                             out_dtype=torch.float32)
    assert rel_l2(got, want) <= REL_L2[torch.float32]


def _nv_abi(qx, qw, gx, gw, sx, sw, out_dtype, ws, bias=None):
    """ckh_scaled_mm_nvfp4 through the C ABI with an explicit workspace (None: no split)."""
    import comfy_kitchen.backends.hip as hb

    m, kb = qx.shape
    n = qw.shape[0]
    alpha = (gx * gw).float().reshape(1)
    out = torch.empty(m, n, dtype=out_dtype, device="cuda")
    hb._call("ckh_scaled_mm_nvfp4", qx.data_ptr(), qw.data_ptr(), sx.data_ptr(), sw.data_ptr(), alpha.data_ptr(),
             None if bias is None else bias.data_ptr(), out.data_ptr(), m, n, 2 * kb, hb.DTYPE_TO_CODE[out_dtype],
             0 if bias is None else hb.DTYPE_TO_CODE[bias.dtype], None if ws is None else ws.data_ptr(),
             0 if ws is None else ws.numel(), torch.cuda.current_stream().cuda_stream)
    return out


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("m,n,k", [(256, 4096, 2048), (300, 2000, 4160), (129, 520, 5152), (65, 13824, 2048),
                                   (300, 8500, 4096)])
def test_scaled_mm_nvfp4_split_k(m, n, k, out_dtype, hip):
    """Small NVFP4 tile grids split K into a workspace, as half tiles (at most 64 tiles) or
    whole tiles (300 x 8500: 68 tiles, 3 ranges) (ranges of ks 256-element groups, odd
    counts and odd starts included, and a last range shorter than the others, down to one
    group; K % 256 != 0, rows past M, columns past N), against the oracle and against the
    unsplit call (fp32 summation order only; an odd group count there too); the reduce
    kernel applies alpha and bias."""
    import comfy_kitchen.backends.hip as hb

    nbytes = hb._lib.ckh_scaled_mm_nvfp4_workspace_bytes(m, n, k)
    assert nbytes > 0
    qx, sx, gx, qw, sw, gw = nv_operands(m, n, k, seed=m + 7 * n + k)
    bias = (torch.randn(n) * 0.1).float()
    want = ref.scaled_mm_nvfp4_ref(qx, qw, gx, gw, sx, sw, bias=bias, out_dtype=torch.float32)
    qx, sx, qw, sw, gx, gw, bias = qx.cuda(), sx.cuda(), qw.cuda(), sw.cuda(), gx.cuda(), gw.cuda(), bias.cuda()
    ws = torch.full((nbytes,), 0xFF, dtype=torch.uint8, device="cuda")
    got = _nv_abi(qx, qw, gx, gw, sx, sw, out_dtype, ws, bias)
    assert rel_l2(got, want) <= REL_L2[out_dtype]
    assert torch.equal(got, _nv_abi(qx, qw, gx, gw, sx, sw, out_dtype, ws, bias))
    if out_dtype == torch.float32:
        assert rel_l2(got, _nv_abi(qx, qw, gx, gw, sx, sw, out_dtype, None, bias)) <= 1e-6
    assert torch.equal(ck.scaled_mm_nvfp4(qx, qw, gx, gw, sx, sw, bias=bias, out_dtype=out_dtype), got)


def test_scaled_mm_nvfp4_workspace_bytes(hip):
    import comfy_kitchen.backends.hip as hb

    f = hb._lib.ckh_scaled_mm_nvfp4_workspace_bytes
    # at most 64 tiles split their column halves: 108 half tiles, 20 groups: 2 ranges of 10
    assert f(256, 13824, 5120) == 54 * 2 * 256 * 256 * 4
    assert f(256, 5120, 13824) == 20 * 6 * 256 * 256 * 4  # 40 half tiles, 54 groups: 6 ranges of 9
    assert f(256, 18432, 8192) == 72 * 3 * 256 * 256 * 4  # 72 whole tiles, 32 groups: 3 ranges of 11
    assert f(256, 32768, 5120) == 0  # 128 tiles: only 2 ranges fit, whole-K half tiles instead
    assert f(256, 18432, 3072) == 0  # 72 tiles, 12 groups: whole tiles split from 16 groups on
    assert f(8192, 13824, 5120) == 0  # 1728 tiles
    assert f(64, 13824, 5120) == 0  # skinny kernel
    assert f(256, 13824, 1024) == 0  # 4 groups
    assert f(0, 4096, 8192) == 0


@pytest.mark.parametrize("out_dtype,with_bias", [(torch.bfloat16, False), (torch.float16, True), (torch.float32, True)])
def test_scaled_mm_nvfp4_half_tile_tail(out_dtype, with_bias, hip):
    """289 tiles of 256 x 256: 256 run as full tiles, the last 33 as 66 half-width tiles
    (partial ones at the right edge, one wholly past N); and a one-round grid without a
    workspace, all of it half tiles."""
    m, n, k = 4352, 4196, 320
    qx, sx, gx, qw, sw, gw = nv_operands(m, n, k, seed=23)
    bias = (torch.randn(n) * 0.1).float() if with_bias else None
    want = ref.scaled_mm_nvfp4_ref(qx, qw, gx, gw, sx, sw, bias=bias, out_dtype=torch.float32)
    got = ck.scaled_mm_nvfp4(qx.cuda(), qw.cuda(), gx.cuda(), gw.cuda(), sx.cuda(), sw.cuda(),
                             bias=None if bias is None else bias.cuda(), out_dtype=out_dtype)
    assert got.shape == (m, n) and got.dtype == out_dtype
    assert rel_l2(got, want) <= REL_L2[out_dtype]
    # The tiles are taken in groups of 6 tile rows, each group column by column: tiles
    # 256..288 lie in the last group (tile rows 12..16) at tile columns 10..16.
    assert rel_l2(got[12 * 256:, 10 * 256:], want[12 * 256:, 10 * 256:]) <= REL_L2[out_dtype]
    # 3 x 5 tiles, no split (K = 1024: 4 groups), as 30 half tiles
    qx, sx, gx, qw, sw, gw = nv_operands(700, 1100, 1024, seed=24)
    want = ref.scaled_mm_nvfp4_ref(qx, qw, gx, gw, sx, sw, out_dtype=torch.float32)
    got = _nv_abi(qx.cuda(), qw.cuda(), gx.cuda(), gw.cuda(), sx.cuda(), sw.cuda(), out_dtype, None)
    assert rel_l2(got, want) <= REL_L2[out_dtype]


def test_scaled_mm_nvfp4_skinny_matches_tile_rows(hip):
    """Rows of a 65-row product (tile kernel) against the same rows computed alone (skinny
    kernel): both sum exact fp16 products in fp32 MFMAs, so they agree to fp32 rounding."""
    qx, sx, gx, qw, sw, gw = nv_operands(65, 512, 2048, seed=44)
    full = ck.scaled_mm_nvfp4(qx.cuda(), qw.cuda(), gx.cuda(), gw.cuda(), sx.cuda(), sw.cuda(), out_dtype=torch.float32)
    part_s = ref.to_blocked(ref.from_blocked(sx.view(torch.uint8), 65, 2048 // 16)[:7].contiguous()).view(
        torch.float8_e4m3fn)
    part = ck.scaled_mm_nvfp4(qx[:7].cuda(), qw.cuda(), gx.cuda(), gw.cuda(), part_s.cuda(), sw.cuda(),
                              out_dtype=torch.float32)
    assert rel_l2(part, full[:7]) <= 1e-5


def test_scaled_mm_nvfp4_config5_full(hip):
    """Config 5 at full size against a GPU fp32 matmul of the dequantized operands."""
    import bench

    a, w, ga, gw = bench.make_c5("cuda")
    qa, sa = ck.quantize_nvfp4(a, ga)
    qw, sw = ck.quantize_nvfp4(w, gw)
    got = ck.scaled_mm_nvfp4(qa, qw, ga, gw, sa, sw)
    da = ck.dequantize_nvfp4(qa, torch.ones_like(ga), sa, torch.float32)  # E2M1 * s8, exact in fp32
    dw = ck.dequantize_nvfp4(qw, torch.ones_like(gw), sw, torch.float32)
    want = torch.matmul(da, dw.t().contiguous()) * (ga * gw)
    assert got.shape == (8192, 13824) and got.dtype == torch.bfloat16
    r = ((got.float() - want).norm() / want.norm()).item()
    print(f"config 5 rel-L2 vs fp32 matmul of dequantized operands: {r:.3e}")
    assert r <= 4e-3
    # and a slice against the CPU oracle end to end: 256 rows of A x 1024 rows of W
    rows, cols = slice(0, 256), slice(0, 1024)

    def rows_of(sc, n, sl):
        return ref.to_blocked(ref.from_blocked(sc.cpu().view(torch.uint8), n, 5120 // 16)[sl].contiguous()).view(
            torch.float8_e4m3fn)

    want_cpu = ref.scaled_mm_nvfp4_ref(qa[rows].cpu(), qw[cols].cpu(), ga.cpu(), gw.cpu(), rows_of(sa, 8192, rows),
                                       rows_of(sw, 13824, cols), out_dtype=torch.float32)
    assert rel_l2(got[rows, cols], want_cpu) <= 4e-3
