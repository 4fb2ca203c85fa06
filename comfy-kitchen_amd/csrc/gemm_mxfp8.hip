// MXFP8 block-scaled GEMM for gfx950 on v_mfma_scale_f32_32x32x64_f8f6f4.
//
//   out[m, n] = sum_k A[m,k] * 2^(sa[m,k/32]-127) * B[n,k] * 2^(sb[n,k/32]-127)  (+ bias[n])
//
// A [M, K] and B [N, K] are E4M3 codes, both K-major (the reference's TN layout);
// sa / sb are E8M0 scales in the 32_4_4 swizzled layout, fed to the MFMA's scale
// operands directly (no dequantization): the four scales of a row for one 128-wide
// K step are one aligned 32-bit word, and the MFMA's opsel picks the byte.
//
// Operand layout of the MFMA (measured): lane l = 32*h + r holds row r; its bytes
// 0..15 are k = 16h..16h+15 and bytes 16..31 are k = 32+16h..32+16h+15 of the 64-wide
// K step; lane-half h supplies the scale of the step's K-block h.  The result lane
// l, register v holds D[8*(v/4) + 4*(l/32) + v%4][l%32].  The weight B is the MFMA's
// first operand and the activation A its second, so each lane ends with 4
// consecutive output columns of one output row (one 8-byte bf16 store).
//
// Tiling: a 256-thread workgroup computes a 256 (m) x 256 (n) tile; its 4 waves
// each own 128 x 128 = 4 x 4 MFMA tiles (256 fp32 accumulators per lane).  K advances
// 128 bytes per stage through double-buffered LDS (2 x 64 KB): global -> registers
// -> LDS, one barrier per stage, next stage's loads in flight during the MFMAs.
// LDS rows are 128 bytes; the 16-byte chunk c of row r is stored at chunk
// c ^ (r & 7) ^ ((r >> 3) & 1): any 8 consecutive rows hit 8 distinct 16-byte bank groups
// and any 16 consecutive rows split 8/8 over both halves of a 256-byte bank row, so
// row-wise writes and 32-row fragment reads are conflict-free whether the LDS
// interleaves 32 or 64 four-byte banks.
//
// Workgroups are dispatched round-robin over the 8 XCDs; the tile index is
// remapped so each XCD walks a contiguous range of tiles (column-major over m), so
// the tiles sharing a weight panel land on the same L2.
#include "ckh_common.h"

namespace ckh {
namespace mx {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));

constexpr int BM = 256, BN = 256, BK = 128, NT = 256;
constexpr int TILE_BYTES = 256 * BK;  // one operand tile in LDS

__device__ __forceinline__ int lds_off(int row, int chunk) { return row * BK + ((chunk ^ ((row & 7) ^ ((row >> 3) & 1))) << 4); }

struct Args {
    const uint8_t* a;   // activation [M, K]
    const uint8_t* b;   // weight [N, K]
    const uint8_t* sa;  // swizzled E8M0 [roundup(M,128), ...]
    const uint8_t* sb;
    const void* bias;
    void* out;
    int M, N, K;
    int ncb;        // scale column blocks: ceil(K/32/4)
    int sa_rows, sb_rows;  // padded scale rows (multiples of 128)
    int tiles_m, tiles_n;
};

// Buffer resource over `bytes` bytes at p: loads at offsets >= bytes return zeros,
// which zero-fills the rows past M / N without branches.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, static_cast<int>(bytes), 0x00020000);
}

// Global -> register prefetch of one stage for one operand: 8 x 16 bytes per thread
// (rows tid/8 + 32*i, 16-byte chunk tid%8).  `off` are the per-row byte offsets
// relative to the tile's first row; a chunk past K gets an offset past the buffer.
__device__ __forceinline__ void load_stage(__amdgpu_buffer_rsrc_t rs, const uint32_t (&off)[8], int k0, int K,
                                           int tid, v4u (&r)[8]) {
    const int k = k0 + (tid & 7) * 16;
    const uint32_t add = k < K ? static_cast<uint32_t>(k) : 0x80000000u;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, off[i] + add, 0, 0);
}

__device__ __forceinline__ void store_stage(uint8_t* __restrict__ lds, int tid, const v4u (&r)[8]) {
    const int chunk = tid & 7;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int row = (tid >> 3) + 32 * i;
        *reinterpret_cast<v4u*>(lds + lds_off(row, chunk)) = r[i];
    }
}

// Scale word of row `row` for the K-step starting at block column k0/32, pre-shifted so
// that byte 0 / byte 2 are this lane-half's scales for MFMA K-substeps 0 / 1.  Rows
// past the padded scale tensor read as 0 through the buffer bounds.
__device__ __forceinline__ uint32_t load_scale(__amdgpu_buffer_rsrc_t rs, int row, int k0, int ncb, int half) {
    const uint32_t w = __builtin_amdgcn_raw_buffer_load_b32(rs, static_cast<uint32_t>(swz_offset(row, k0 >> 5, ncb)), 0, 0);
    return w >> (8 * half);
}

__device__ __forceinline__ v8i load_frag(const uint8_t* __restrict__ lds, int row, int kk, int half) {
    const v4u lo = *reinterpret_cast<const v4u*>(lds + lds_off(row, 4 * kk + half));
    const v4u hi = *reinterpret_cast<const v4u*>(lds + lds_off(row, 4 * kk + 2 + half));
    v8i f;
    f[0] = lo[0]; f[1] = lo[1]; f[2] = lo[2]; f[3] = lo[3];
    f[4] = hi[0]; f[5] = hi[1]; f[6] = hi[2]; f[7] = hi[3];
    return f;
}

template <int OUT>
__device__ __forceinline__ void store4(void* out, int64_t idx, const float (&v)[4]) {
    if constexpr (OUT == CKH_F32) {
        *reinterpret_cast<float4*>(static_cast<float*>(out) + idx) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
        uint32_t w0 = (OUT == CKH_BF16 ? f_to_bf16(v[0]) : f_to_f16(v[0])) |
                      ((OUT == CKH_BF16 ? f_to_bf16(v[1]) : f_to_f16(v[1])) << 16);
        uint32_t w1 = (OUT == CKH_BF16 ? f_to_bf16(v[2]) : f_to_f16(v[2])) |
                      ((OUT == CKH_BF16 ? f_to_bf16(v[3]) : f_to_f16(v[3])) << 16);
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + idx) = make_uint2(w0, w1);
    }
}

template <int OUT>
__device__ __forceinline__ void store1(void* out, int64_t idx, float v) {
    if constexpr (OUT == CKH_F32) static_cast<float*>(out)[idx] = v;
    else static_cast<uint16_t*>(out)[idx] = static_cast<uint16_t>(OUT == CKH_BF16 ? f_to_bf16(v) : f_to_f16(v));
}

template <int BIAS>
__device__ __forceinline__ float bias_at(const void* bias, int n) {
    if constexpr (BIAS < 0) return 0.0f;
    else return load1<BIAS>(bias, n);
}

template <int OUT, int BIAS>
__global__ __launch_bounds__(NT) void gemm_kernel(Args p) {
    __shared__ __attribute__((aligned(16))) uint8_t smem[4 * TILE_BYTES];  // [2 stages][weight, act][tile]

    // XCD-aware tile order: hardware places workgroup i on XCD i % 8.
    const int tiles = p.tiles_m * p.tiles_n;
    int bid = blockIdx.x;
    if ((tiles & 7) == 0) bid = (bid & 7) * (tiles >> 3) + (bid >> 3);
    const int tm = bid % p.tiles_m, tn = bid / p.tiles_m;
    const int m0 = tm * BM, n0 = tn * BN;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;
    const int half = lane >> 5, r32 = lane & 31;

    v16f acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = v16f{};

    const int KT = (p.K + BK - 1) / BK;
    // buffer views of this tile's rows (rows past M / N read as zeros)
    const __amdgpu_buffer_rsrc_t rsb = make_rsrc(p.b + static_cast<int64_t>(n0) * p.K,
                                                static_cast<uint32_t>(min(BN, p.N - n0)) * p.K);
    const __amdgpu_buffer_rsrc_t rsa = make_rsrc(p.a + static_cast<int64_t>(m0) * p.K,
                                                static_cast<uint32_t>(min(BM, p.M - m0)) * p.K);
    const __amdgpu_buffer_rsrc_t rssb = make_rsrc(p.sb, static_cast<uint32_t>(p.sb_rows) * p.ncb * 4);
    const __amdgpu_buffer_rsrc_t rssa = make_rsrc(p.sa, static_cast<uint32_t>(p.sa_rows) * p.ncb * 4);
    uint32_t off[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) off[i] = static_cast<uint32_t>((tid >> 3) + 32 * i) * p.K;
    v4u rb[8], ra[8];
    uint32_t sbw[4], saw[4], sbn[4], san[4];

    load_stage(rsb, off, 0, p.K, tid, rb);
    load_stage(rsa, off, 0, p.K, tid, ra);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        sbw[t] = load_scale(rssb, n0 + wn * 128 + t * 32 + r32, 0, p.ncb, half);
        saw[t] = load_scale(rssa, m0 + wm * 128 + t * 32 + r32, 0, p.ncb, half);
    }
    store_stage(smem, tid, rb);
    store_stage(smem + TILE_BYTES, tid, ra);
    __syncthreads();

    for (int kt = 0; kt < KT; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < KT;
        if (more) {
            const int k1 = (kt + 1) * BK;
            load_stage(rsb, off, k1, p.K, tid, rb);
            load_stage(rsa, off, k1, p.K, tid, ra);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                sbn[t] = load_scale(rssb, n0 + wn * 128 + t * 32 + r32, k1, p.ncb, half);
                san[t] = load_scale(rssa, m0 + wm * 128 + t * 32 + r32, k1, p.ncb, half);
            }
        }
        const uint8_t* lb = smem + cur * 2 * TILE_BYTES;
        const uint8_t* la = lb + TILE_BYTES;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            v8i fa[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) fa[t] = load_frag(la, wm * 128 + t * 32 + r32, kk, half);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const v8i fb = load_frag(lb, wn * 128 + i * 32 + r32, kk, half);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (kk == 0)
                        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fb, fa[j], acc[i][j], 0, 0, 0,
                                                                                    sbw[i], 0, saw[j]);
                    else
                        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fb, fa[j], acc[i][j], 0, 0, 2,
                                                                                    sbw[i], 2, saw[j]);
                }
            }
        }
        if (more) {
            uint8_t* nb = smem + (cur ^ 1) * 2 * TILE_BYTES;
            store_stage(nb, tid, rb);
            store_stage(nb + TILE_BYTES, tid, ra);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                sbw[t] = sbn[t];
                saw[t] = san[t];
            }
        }
        __syncthreads();
    }

    // Epilogue: lane holds out[m][n..n+3] for m = r32-th row of activation tile j and
    // n = 8*g + 4*half (+0..3) of weight tile i.
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int m = m0 + wm * 128 + j * 32 + r32;
        if (m >= p.M) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int n = n0 + wn * 128 + i * 32 + 8 * g + 4 * half;
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = acc[i][j][4 * g + e] + (n + e < p.N ? bias_at<BIAS>(p.bias, n + e) : 0.0f);
                const int64_t idx = static_cast<int64_t>(m) * p.N + n;
                if (n + 3 < p.N && (p.N & 3) == 0) {
                    store4<OUT>(p.out, idx, v);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (n + e < p.N) store1<OUT>(p.out, idx + e, v[e]);
                }
            }
        }
    }
}

}  // namespace mx
}  // namespace ckh

using namespace ckh;

extern "C" int ckh_scaled_mm_mxfp8(const void* a, const void* b, const void* sa, const void* sb, const void* bias,
                                   void* out, int64_t M, int64_t N, int64_t K, int out_code, int bias_code,
                                   uintptr_t stream) {
    CKH_REQUIRE(a && b && sa && sb && out, "scaled_mm_mxfp8: null pointer");
    CKH_REQUIRE(M >= 0 && N >= 0 && K > 0, "scaled_mm_mxfp8: sizes must be M, N >= 0 and K > 0");
    CKH_REQUIRE(K % 32 == 0, "scaled_mm_mxfp8: K (%lld) must be a multiple of 32", (long long)K);
    CKH_REQUIRE(M < (1ll << 31) && N < (1ll << 31) && K < (1ll << 31), "scaled_mm_mxfp8: size too large");
    CKH_REQUIRE(out_code == CKH_F32 || out_code == CKH_F16 || out_code == CKH_BF16,
                "scaled_mm_mxfp8: unsupported output dtype code %d", out_code);
    CKH_REQUIRE(!bias || bias_code == CKH_F32 || bias_code == CKH_F16 || bias_code == CKH_BF16,
                "scaled_mm_mxfp8: unsupported bias dtype code %d", bias_code);
    CKH_REQUIRE(aligned(a, 16) && aligned(b, 16) && aligned(sa, 4) && aligned(sb, 4) && aligned(out, 16),
                "scaled_mm_mxfp8: pointers misaligned");
    CKH_REQUIRE(K % 16 == 0, "scaled_mm_mxfp8: K must keep rows 16-byte aligned");
    if (M == 0 || N == 0) return CKH_OK;
    mx::Args p{};
    p.a = static_cast<const uint8_t*>(a);
    p.b = static_cast<const uint8_t*>(b);
    p.sa = static_cast<const uint8_t*>(sa);
    p.sb = static_cast<const uint8_t*>(sb);
    p.bias = bias;
    p.out = out;
    p.M = static_cast<int>(M);
    p.N = static_cast<int>(N);
    p.K = static_cast<int>(K);
    p.ncb = static_cast<int>(cdiv(K / 32, 4));
    p.sa_rows = static_cast<int>(rup(M, 128));
    p.sb_rows = static_cast<int>(rup(N, 128));
    p.tiles_m = static_cast<int>(cdiv(M, mx::BM));
    p.tiles_n = static_cast<int>(cdiv(N, mx::BN));
    dim3 grid(static_cast<unsigned>(p.tiles_m * p.tiles_n));
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
#define LAUNCH(O, B) hipLaunchKernelGGL((mx::gemm_kernel<O, B>), grid, dim3(mx::NT), 0, st, p)
#define BY_BIAS(O)                                   \
    do {                                             \
        if (!bias) LAUNCH(O, -1);                    \
        else if (bias_code == CKH_F32) LAUNCH(O, CKH_F32); \
        else if (bias_code == CKH_F16) LAUNCH(O, CKH_F16); \
        else LAUNCH(O, CKH_BF16);                    \
    } while (0)
    if (out_code == CKH_BF16) BY_BIAS(CKH_BF16);
    else if (out_code == CKH_F16) BY_BIAS(CKH_F16);
    else BY_BIAS(CKH_F32);
#undef BY_BIAS
#undef LAUNCH
    return check_launch("scaled_mm_mxfp8");
}
