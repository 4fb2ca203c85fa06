// NVFP4 block-scaled GEMM for gfx950.
//
//   out[m, n] = alpha * sum_k E2M1(a[m,k]) * sa[m,k/16] * E2M1(b[n,k]) * sb[n,k/16]  (+ bias[n])
//
// a [M, K/2], b [N, K/2]: packed E2M1 codes, both K-major; sa / sb: E4M3 scales per
// 16 elements in the 32_4_4 swizzled layout; alpha: one fp32 on the device
// (tensor_scale_a * tensor_scale_b).
//
// Exact fold: E2M1 * E4M3 has at most 5 significant bits and lies in [2^-10, 2688],
// so every product value * block scale is an exact fp16.  The global -> LDS stage
// decodes each byte (two E2M1 codes) with v_cvt_scalef32_pk_f16_fp4 and multiplies
// by the block scale with a packed f16 multiply, and the MFMAs (v_mfma_f32_32x32x16_f16) multiply the
// exact fp16 operands with fp32 accumulation; alpha and bias are applied in the
// epilogue.  (An E8M0-scaled FP4 MFMA cannot take E4M3 block scales exactly, and a
// lossy re-encode misses the 1e-2 accuracy bar.)  Nibble order inside a byte does
// not matter: both operands use the same packing, and the dot product is invariant
// under the same permutation of k on both sides.
//
// Tiling matches the MXFP8 kernel: 256 (m) x 256 (n) per 256-thread workgroup, 4 waves
// of 128 x 128, K advancing 64 elements per stage (32 packed bytes per row) through
// double-buffered LDS holding fp16 tiles (128 bytes per row per stage), 16-byte chunk
// c of row r stored at chunk c ^ (r & 7) ^ ((r >> 3) & 1).  MFMA operand layout: lane
// l = 32*h + r holds row r, k = 16*kk + 8*h .. +7 of the 64-wide stage.
#include "ckh_common.h"

namespace ckh {
namespace nv {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));

constexpr int BM = 256, BN = 256, BKE = 64 /* elements */, NT = 256;
constexpr int ROWB = 128;                 // LDS bytes per row per stage (64 fp16)
constexpr int TILE_BYTES = 256 * ROWB;

__device__ __forceinline__ int lds_off(int row, int chunk) { return row * ROWB + ((chunk ^ ((row & 7) ^ ((row >> 3) & 1))) << 4); }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, static_cast<int>(bytes), 0x00020000);
}

struct Args {
    const uint8_t* a;
    const uint8_t* b;
    const uint8_t* sa;
    const uint8_t* sb;
    const float* alpha;
    const void* bias;
    void* out;
    int M, N, K;  // K in elements
    int ncb;      // scale column blocks: ceil(K/16/4)
    int sa_rows, sb_rows;
    int tiles_m, tiles_n;
};

// Per stage each thread owns (row tid>>1 and row 128 + tid>>1) x (16 packed bytes =
// 32 elements = 2 scale blocks, half tid&1 of the 64-element stage).
struct Stage {
    v4u q[2];        // packed codes
    uint32_t s[2];   // the row's scale word for this stage
};

__device__ __forceinline__ void load_stage(__amdgpu_buffer_rsrc_t rs, __amdgpu_buffer_rsrc_t rss, int row0, int Kb,
                                           int k0, int ncb, int tid, Stage& st) {
    const int hh = tid & 1;
    const int kb = k0 / 2 + hh * 16;  // packed byte column
    const uint32_t add = kb < Kb ? static_cast<uint32_t>(kb) : 0x80000000u;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int row = (tid >> 1) + 128 * i;
        st.q[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<uint32_t>(row) * Kb + add, 0, 0);
        st.s[i] = __builtin_amdgcn_raw_buffer_load_b32(
            rss, static_cast<uint32_t>(swz_offset(row0 + row, k0 >> 4, ncb)), 0, 0);
    }
}

// Decode one thread's 2 x 32 elements to fp16 (exact) and write them to LDS.  The
// hardware fp4 -> f16 convert applies only a power-of-two scale, so it decodes with
// scale 1 and the E4M3 block scale (exact in fp16) is applied by a packed f16
// multiply, which is exact for these products.
__device__ __forceinline__ void store_stage(uint8_t* __restrict__ lds, int tid, const Stage& st) {
    const int hh = tid & 1;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int row = (tid >> 1) + 128 * i;
        // the two E4M3 block scales of this half: bytes 2*hh and 2*hh+1 of the word
        const _Float16 s0 = static_cast<_Float16>(e4m3_to_f((st.s[i] >> (16 * hh)) & 0xffu));
        const _Float16 s1 = static_cast<_Float16>(e4m3_to_f((st.s[i] >> (16 * hh + 8)) & 0xffu));
#pragma unroll
        for (int c = 0; c < 4; ++c) {  // 16-byte LDS chunk = 8 fp16 = 4 packed bytes
            const uint32_t w = st.q[i][c];
            const v2h sc = c < 2 ? v2h{s0, s0} : v2h{s1, s1};
            v2h h0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 0) * sc;
            v2h h1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 1) * sc;
            v2h h2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 2) * sc;
            v2h h3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 3) * sc;
            v8h v = {h0[0], h0[1], h1[0], h1[1], h2[0], h2[1], h3[0], h3[1]};
            *reinterpret_cast<v8h*>(lds + lds_off(row, 4 * hh + c)) = v;
        }
    }
}

__device__ __forceinline__ v8h load_frag(const uint8_t* __restrict__ lds, int row, int kk, int half) {
    return *reinterpret_cast<const v8h*>(lds + lds_off(row, 2 * kk + half));
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

    const int tiles = p.tiles_m * p.tiles_n;
    int bid = blockIdx.x;
    if ((tiles & 7) == 0) bid = (bid & 7) * (tiles >> 3) + (bid >> 3);
    const int tm = bid % p.tiles_m, tn = bid / p.tiles_m;
    const int m0 = tm * BM, n0 = tn * BN;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;
    const int half = lane >> 5, r32 = lane & 31;
    const int Kb = p.K / 2;

    const __amdgpu_buffer_rsrc_t rsb = make_rsrc(p.b + static_cast<int64_t>(n0) * Kb,
                                                static_cast<uint32_t>(min(BN, p.N - n0)) * Kb);
    const __amdgpu_buffer_rsrc_t rsa = make_rsrc(p.a + static_cast<int64_t>(m0) * Kb,
                                                static_cast<uint32_t>(min(BM, p.M - m0)) * Kb);
    const __amdgpu_buffer_rsrc_t rssb = make_rsrc(p.sb, static_cast<uint32_t>(p.sb_rows) * p.ncb * 4);
    const __amdgpu_buffer_rsrc_t rssa = make_rsrc(p.sa, static_cast<uint32_t>(p.sa_rows) * p.ncb * 4);

    v16f acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = v16f{};

    const int KT = (p.K + BKE - 1) / BKE;
    Stage sb, sa;
    load_stage(rsb, rssb, n0, Kb, 0, p.ncb, tid, sb);
    load_stage(rsa, rssa, m0, Kb, 0, p.ncb, tid, sa);
    store_stage(smem, tid, sb);
    store_stage(smem + TILE_BYTES, tid, sa);
    __syncthreads();

    for (int kt = 0; kt < KT; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < KT;
        if (more) {
            load_stage(rsb, rssb, n0, Kb, (kt + 1) * BKE, p.ncb, tid, sb);
            load_stage(rsa, rssa, m0, Kb, (kt + 1) * BKE, p.ncb, tid, sa);
        }
        const uint8_t* lb = smem + cur * 2 * TILE_BYTES;
        const uint8_t* la = lb + TILE_BYTES;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            v8h fa[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) fa[t] = load_frag(la, wm * 128 + t * 32 + r32, kk, half);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const v8h fb = load_frag(lb, wn * 128 + i * 32 + r32, kk, half);
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fb, fa[j], acc[i][j], 0, 0, 0);
            }
        }
        if (more) {
            uint8_t* nb = smem + (cur ^ 1) * 2 * TILE_BYTES;
            store_stage(nb, tid, sb);
            store_stage(nb + TILE_BYTES, tid, sa);
        }
        __syncthreads();
    }

    const float alpha = p.alpha[0];
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
                for (int e = 0; e < 4; ++e)
                    v[e] = acc[i][j][4 * g + e] * alpha + (n + e < p.N ? bias_at<BIAS>(p.bias, n + e) : 0.0f);
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

}  // namespace nv
}  // namespace ckh

using namespace ckh;

extern "C" int ckh_scaled_mm_nvfp4(const void* a, const void* b, const void* sa, const void* sb, const void* alpha,
                                   const void* bias, void* out, int64_t M, int64_t N, int64_t K, int out_code,
                                   int bias_code, uintptr_t stream) {
    CKH_REQUIRE(a && b && sa && sb && alpha && out, "scaled_mm_nvfp4: null pointer");
    CKH_REQUIRE(M >= 0 && N >= 0 && K > 0, "scaled_mm_nvfp4: sizes must be M, N >= 0 and K > 0");
    CKH_REQUIRE(K % 32 == 0, "scaled_mm_nvfp4: K (%lld) must be a multiple of 32", (long long)K);
    CKH_REQUIRE(M * (K / 2) < (1ll << 31) && N * (K / 2) < (1ll << 31) && M < (1ll << 30) && N < (1ll << 30),
                "scaled_mm_nvfp4: operand larger than 2 GiB");
    CKH_REQUIRE(out_code == CKH_F32 || out_code == CKH_F16 || out_code == CKH_BF16,
                "scaled_mm_nvfp4: unsupported output dtype code %d", out_code);
    CKH_REQUIRE(!bias || bias_code == CKH_F32 || bias_code == CKH_F16 || bias_code == CKH_BF16,
                "scaled_mm_nvfp4: unsupported bias dtype code %d", bias_code);
    CKH_REQUIRE(aligned(a, 16) && aligned(b, 16) && aligned(sa, 4) && aligned(sb, 4) && aligned(out, 16) &&
                    aligned(alpha, 4),
                "scaled_mm_nvfp4: pointers misaligned");
    if (M == 0 || N == 0) return CKH_OK;
    nv::Args p{};
    p.a = static_cast<const uint8_t*>(a);
    p.b = static_cast<const uint8_t*>(b);
    p.sa = static_cast<const uint8_t*>(sa);
    p.sb = static_cast<const uint8_t*>(sb);
    p.alpha = static_cast<const float*>(alpha);
    p.bias = bias;
    p.out = out;
    p.M = static_cast<int>(M);
    p.N = static_cast<int>(N);
    p.K = static_cast<int>(K);
    p.ncb = static_cast<int>(cdiv(K / 16, 4));
    p.sa_rows = static_cast<int>(rup(M, 128));
    p.sb_rows = static_cast<int>(rup(N, 128));
    p.tiles_m = static_cast<int>(cdiv(M, nv::BM));
    p.tiles_n = static_cast<int>(cdiv(N, nv::BN));
    dim3 grid(static_cast<unsigned>(p.tiles_m * p.tiles_n));
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
#define LAUNCH(O, B) hipLaunchKernelGGL((nv::gemm_kernel<O, B>), grid, dim3(nv::NT), 0, st, p)
#define BY_BIAS(O)                                          \
    do {                                                    \
        if (!bias) LAUNCH(O, -1);                           \
        else if (bias_code == CKH_F32) LAUNCH(O, CKH_F32);  \
        else if (bias_code == CKH_F16) LAUNCH(O, CKH_F16);  \
        else LAUNCH(O, CKH_BF16);                           \
    } while (0)
    if (out_code == CKH_BF16) BY_BIAS(CKH_BF16);
    else if (out_code == CKH_F16) BY_BIAS(CKH_F16);
    else BY_BIAS(CKH_F32);
#undef BY_BIAS
#undef LAUNCH
    return check_launch("scaled_mm_nvfp4");
}
