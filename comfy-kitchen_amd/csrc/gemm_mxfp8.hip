// MXFP8 block-scaled GEMM for gfx950 on v_mfma_scale_f32_32x32x64_f8f6f4.
//
//   out[m, n] = sum_k A[m,k] * 2^(sa[m,k/32]-127) * B[n,k] * 2^(sb[n,k/32]-127)  (+ bias[n])
//
// A [M, K] and B [N, K] are E4M3 codes, both K-major (the reference's TN layout);
// sa / sb are E8M0 scales in the 32_4_4 swizzled layout, fed to the MFMA's scale
// operands directly (no dequantization): the four scales of a row for one 128-wide
// K step are one aligned 32-bit word, and the MFMA's opsel picks the byte.
//
// MFMA operand layout (measured on gfx950): lane l = 32*h + r holds row r; its bytes
// 0..15 are k = 16h..16h+15 and bytes 16..31 are k = 32+16h..32+16h+15 of the 64-wide
// K step; lane-half h supplies the scale of the step's K-block h.  The result lane l,
// register v holds D[8*(v/4) + 4*(l/32) + v%4][l%32].  The weight B is the MFMA's
// first operand and the activation A its second, so each lane ends with 4
// consecutive output columns of one output row.
//
// Tiling: a 256-thread workgroup computes a 256 (m) x 256 (n) tile; its 4 waves each
// own 128 x 128 = 4 x 4 MFMA tiles (256 fp32 accumulators per lane).  K advances 128
// per stage through two LDS buffers (2 x 64 KB).  Global data goes straight to LDS
// with buffer_load_dwordx4 ... lds (no VGPR staging): lane i of a load fills LDS
// bytes [base + 16 i, base + 16 i + 16), so each lane fetches the global chunk that
// belongs at its slot.  Rows past M / N and columns past K lie outside the buffer
// descriptor's range and arrive as zeros.
//
// LDS rows are 128 bytes; logical 16-byte chunk c of row r lives at chunk
// c ^ (r & 7) ^ ((r >> 3) & 1): any 8 consecutive rows use 8 distinct bank groups and
// any 16 split 8/8 over both halves of a 256-byte bank row, so fragment reads (32
// rows at one chunk) are conflict-free for 32- or 64-bank LDS (0 conflicts measured).
//
// Schedule per K stage (one barrier per stage):
//   phase A: 16 MFMAs on fragments F0 (K-substep 0), interleaved with the LDS reads
//            of F1 (substep 1);
//   wait for this wave's LDS reads and stage loads, barrier;
//   phase B: 16 MFMAs on F1, interleaved with the global->LDS loads of stage s+2 into
//            the buffer just finished and the LDS reads of F0 and of the scale words
//            of the next stage.
// The E8M0 scale words travel through LDS as well (1 KB per operand per stage), so no
// global load result is ever waited on inside the loop except at the stage barrier.
// Workgroups are dispatched round-robin over the 8 XCDs; the tile index is remapped
// so each XCD walks a contiguous range of tiles (column-major over m), keeping the
// tiles that share a weight panel on one L2.
#include <type_traits>

#include "ckh_common.h"

namespace ckh {
namespace mx {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int BM = 256, BN = 256, BK = 128, NT = 256;
constexpr int TILE = 256 * BK;   // bytes of one operand tile per stage
constexpr int STILE = 1024;      // bytes of one operand's scale words per stage (256 rows)

// scheduling-group masks of __builtin_amdgcn_sched_group_barrier
constexpr int SG_MFMA = 0x008, SG_DS_READ = 0x100, SG_DS_WRITE = 0x200;

__device__ __forceinline__ int swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, static_cast<int>(bytes), 0x00020000);
}

struct Args {
    const uint8_t* a;   // activation [M, K]
    const uint8_t* b;   // weight [N, K]
    const uint8_t* sa;  // swizzled E8M0, [roundup(M,128), ncb*4]
    const uint8_t* sb;
    const void* bias;
    void* out;
    int M, N, K;
    int ncb;               // scale column blocks: ceil(K/32/4)
    int sa_rows, sb_rows;  // padded scale rows (multiples of 128)
    int tiles_m, tiles_n;
};

// Per-lane state for the direct-to-LDS loads of one operand.  Wave w, load j (0..7)
// covers tile rows R = 64 w + 8 j .. +7; lane i fills row R + i/8, physical chunk
// i%8, i.e. logical chunk (i%8) ^ (i/8) ^ (j&1).
struct Loader {
    __amdgpu_buffer_rsrc_t rs;
    uint32_t base[2];  // byte offset of the lane's chunk for even / odd j, tile-relative, k0 = 0
    int cbyte[2];      // the lane's chunk column in bytes (0..112) for even / odd j
    uint32_t rowstep;  // 8 * K: byte distance between consecutive loads j
    uint32_t row0;     // 64 * wave * K
};

__device__ __forceinline__ Loader make_loader(const uint8_t* tile_base, int valid_rows, int K, int wave, int lane) {
    Loader L;
    L.rs = make_rsrc(tile_base, static_cast<uint32_t>(valid_rows) * K);
    const int rin = lane >> 3, pc = lane & 7;
    L.cbyte[0] = (pc ^ rin) << 4;
    L.cbyte[1] = (pc ^ rin ^ 1) << 4;
    L.base[0] = static_cast<uint32_t>(rin * K + L.cbyte[0]);
    L.base[1] = static_cast<uint32_t>(rin * K + L.cbyte[1]);
    L.rowstep = 8u * K;
    L.row0 = 64u * wave * K;
    return L;
}

// Issue the 8 global->LDS loads of one operand for the stage starting at k0.  A chunk
// past the end of the row (last stage when K % 128 != 0) gets an offset outside the
// descriptor and is written as zeros.
__device__ __forceinline__ void issue_stage(const Loader& L, uint8_t* lds_tile, int wave, int k0, int K) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        uint32_t off = L.base[j & 1] + L.row0 + j * L.rowstep + k0;
        off = (k0 + L.cbyte[j & 1] < K) ? off : 0x80000000u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(L.rs, (lds_void*)(lds_tile + (64 * wave + 8 * j) * BK), 16, off, 0, 0,
                                                 0);
    }
}

// Scale words of a stage: for a 256-row tile and one 128-wide K step they are two
// contiguous 512-byte chunks of the swizzled tensor (rows 128*rb .. +127, block column
// k0/128), chunk (rb * ncb + k0/128).  Wave w copies chunk rb = w & 1 of operand
// w >> 1 (0 = weight, 1 = activation) to LDS with two 4-byte-per-lane DMA loads;
// inside a chunk row r's word sits at (r % 32) * 16 + ((r % 128) / 32) * 4, so a
// lane's words for its four 32-row tiles are one contiguous 16-byte LDS read.
__device__ __forceinline__ void issue_scales(__amdgpu_buffer_rsrc_t rs_b, __amdgpu_buffer_rsrc_t rs_a, int rb0_b,
                                             int rb0_a, int ncb, int k0, int K, uint8_t* lds_stage, int wave,
                                             int lane) {
    const int op = wave >> 1, rb = wave & 1;
    const __amdgpu_buffer_rsrc_t rs = op ? rs_a : rs_b;
    uint32_t chunk = static_cast<uint32_t>(((op ? rb0_a : rb0_b) + rb) * ncb + (k0 >> 7)) * 512u;
    chunk = k0 < K ? chunk : 0x80000000u;  // stages past K: zero scale words
    uint8_t* dst = lds_stage + op * STILE + rb * 512;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)dst, 4, chunk + lane * 4, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(dst + 256), 4, chunk + 256 + lane * 4, 0, 0, 0);
}

struct Frags {
    v8i b[4];  // weight fragments (MFMA operand 0)
    v8i a[4];  // activation fragments (MFMA operand 1)
};

// Byte offsets (within an operand tile) of this lane's two 16-byte halves of a fragment
// for K-substep kk; tile t adds t * 32 rows = t * 4096 bytes.
struct FragAddr {
    uint32_t lo[2], hi[2];  // [kk]
};

__device__ __forceinline__ FragAddr make_frag_addr(int row_base, int lane) {
    const int half = lane >> 5, r32 = lane & 31;
    const int row = row_base + r32;
    const int s = swz(row);
    FragAddr f;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
        f.lo[kk] = static_cast<uint32_t>(row * BK + (((4 * kk + half) ^ s) << 4));
        f.hi[kk] = static_cast<uint32_t>(row * BK + (((4 * kk + 2 + half) ^ s) << 4));
    }
    return f;
}

__device__ __forceinline__ v8i read_frag(const uint8_t* tile, uint32_t lo, uint32_t hi) {
    const v4u x = *reinterpret_cast<const v4u*>(tile + lo);
    const v4u y = *reinterpret_cast<const v4u*>(tile + hi);
    v8i f;
    f[0] = x[0]; f[1] = x[1]; f[2] = x[2]; f[3] = x[3];
    f[4] = y[0]; f[5] = y[1]; f[6] = y[2]; f[7] = y[3];
    return f;
}

__device__ __forceinline__ void read_frags(Frags& F, const uint8_t* tb, const uint8_t* ta, const FragAddr& fb,
                                           const FragAddr& fa, int kk) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        F.b[t] = read_frag(tb + t * 32 * BK, fb.lo[kk], fb.hi[kk]);
        F.a[t] = read_frag(ta + t * 32 * BK, fa.lo[kk], fa.hi[kk]);
    }
}

template <int OPSEL>
__device__ __forceinline__ void mfma16(v16f (&acc)[4][4], const Frags& F, const uint32_t (&sb)[4],
                                       const uint32_t (&sa)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(F.b[i], F.a[j], acc[i][j], 0, 0, OPSEL, sb[i],
                                                                        OPSEL, sa[j]);
}

template <int OUT>
__device__ __forceinline__ void store4(void* out, int64_t idx, const float (&v)[4]) {
    if constexpr (OUT == CKH_F32) {
        *reinterpret_cast<float4*>(static_cast<float*>(out) + idx) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
        uint32_t w0 = (OUT == CKH_BF16 ? f_to_bf16_rne(v[0]) : f_to_f16(v[0])) |
                      ((OUT == CKH_BF16 ? f_to_bf16_rne(v[1]) : f_to_f16(v[1])) << 16);
        uint32_t w1 = (OUT == CKH_BF16 ? f_to_bf16_rne(v[2]) : f_to_f16(v[2])) |
                      ((OUT == CKH_BF16 ? f_to_bf16_rne(v[3]) : f_to_f16(v[3])) << 16);
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + idx) = make_uint2(w0, w1);
    }
}

template <int OUT>
__device__ __forceinline__ void store1(void* out, int64_t idx, float v) {
    if constexpr (OUT == CKH_F32) static_cast<float*>(out)[idx] = v;
    else static_cast<uint16_t*>(out)[idx] = static_cast<uint16_t>(OUT == CKH_BF16 ? f_to_bf16_rne(v) : f_to_f16(v));
}

template <int BIAS>
__device__ __forceinline__ float bias_at(const void* bias, int n) {
    if constexpr (BIAS < 0) return 0.0f;
    else return load1<BIAS>(bias, n);
}

template <int OUT, int BIAS>
__global__ __launch_bounds__(NT) void gemm_kernel(Args p) {
    // One LDS array per buffer parity, so the compiler can prove that the DMA writes of
    // one stage never alias the fragment reads of the other and waits only at barriers.
    __shared__ __attribute__((aligned(1024))) uint8_t smem0[2 * TILE];  // [weight, act][TILE]
    __shared__ __attribute__((aligned(1024))) uint8_t smem1[2 * TILE];
    __shared__ __attribute__((aligned(16))) uint8_t sscale0[2 * STILE];  // [weight, act][1 KB]
    __shared__ __attribute__((aligned(16))) uint8_t sscale1[2 * STILE];

    const int tiles = p.tiles_m * p.tiles_n;
    int bid = blockIdx.x;
    if ((tiles & 7) == 0) bid = (bid & 7) * (tiles >> 3) + (bid >> 3);
    const int tm = bid % p.tiles_m, tn = bid / p.tiles_m;
    const int m0 = tm * BM, n0 = tn * BN;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
    const int wm = wave & 1, wn = wave >> 1;
    const int half = lane >> 5, r32 = lane & 31;

    const Loader LB = make_loader(p.b + static_cast<int64_t>(n0) * p.K, min(BN, p.N - n0), p.K, wave, lane);
    const Loader LA = make_loader(p.a + static_cast<int64_t>(m0) * p.K, min(BM, p.M - m0), p.K, wave, lane);
    const __amdgpu_buffer_rsrc_t rssb = make_rsrc(p.sb, static_cast<uint32_t>(p.sb_rows) * p.ncb * 4);
    const __amdgpu_buffer_rsrc_t rssa = make_rsrc(p.sa, static_cast<uint32_t>(p.sa_rows) * p.ncb * 4);
    const FragAddr fab = make_frag_addr(wn * 128, lane);
    const FragAddr faa = make_frag_addr(wm * 128, lane);
    const int KT = (p.K + BK - 1) / BK;

    v16f acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = v16f{};

    auto buf = [&](auto par_c) -> uint8_t* { return decltype(par_c)::value ? smem1 : smem0; };
    auto sbuf = [&](auto par_c) -> uint8_t* { return decltype(par_c)::value ? sscale1 : sscale0; };
    auto issue = [&](auto par_c, int s) {
        uint8_t* b = buf(par_c);
        issue_stage(LB, b, wave, s * BK, p.K);
        issue_stage(LA, b + TILE, wave, s * BK, p.K);
        issue_scales(rssb, rssa, n0 >> 7, m0 >> 7, p.ncb, s * BK, p.K, sbuf(par_c), wave, lane);
    };
    // this lane's 4 scale words (tiles t = 0..3) of each operand for a stage, shifted so
    // byte 0 / byte 2 are the lane-half's scales for K-substeps 0 / 1
    const int hs = 8 * half;
    auto read_scales = [&](auto par_c, uint32_t (&sb)[4], uint32_t (&sa)[4]) {
        const uint8_t* st = sbuf(par_c);
        const v4u wb = *reinterpret_cast<const v4u*>(st + wn * 512 + r32 * 16);
        const v4u wa = *reinterpret_cast<const v4u*>(st + STILE + wm * 512 + r32 * 16);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            sb[t] = wb[t] >> hs;
            sa[t] = wa[t] >> hs;
        }
    };

    uint32_t scb[4], sca[4];
    Frags F0, F1;
    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;

    // One K stage held in buffer PAR: the stage's MFMAs, the reads of the next stage's
    // F0 and scale words, and the loads of the stage after next into this buffer.  Every
    // stage runs the same branch-free body; stages at or past K load as zeros, so the
    // stage count is padded to even and the loop needs no tail variants.
    auto stage = [&](auto par_c, int kt) {
        using Other = std::integral_constant<int, 1 - decltype(par_c)::value>;
        const uint8_t* tb = buf(par_c);
        const uint8_t* ta = tb + TILE;
        // ---- phase A: MFMAs on F0, LDS reads of F1
        read_frags(F1, tb, ta, fab, faa, 1);
        mfma16<0>(acc, F0, scb, sca);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
            __builtin_amdgcn_sched_group_barrier(SG_DS_READ, 1, 0);
        }
        // stage kt+1 resident everywhere; every wave done reading stage kt
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        // ---- phase B: MFMAs on F1, loads of stage kt+2, LDS reads of F0 (stage kt+1)
        uint32_t nb[4], na[4];
        issue(par_c, kt + 2);
        read_frags(F0, buf(Other{}), buf(Other{}) + TILE, fab, faa, 0);
        read_scales(Other{}, nb, na);
        mfma16<2>(acc, F1, scb, sca);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
            __builtin_amdgcn_sched_group_barrier(SG_DS_WRITE, 1, 0);
            __builtin_amdgcn_sched_group_barrier(SG_DS_READ, 1, 0);
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            scb[t] = nb[t];
            sca[t] = na[t];
        }
    };

    // prologue: stage 0 resident, stage 1 in flight, F0 and stage-0 scales read
    issue(P0{}, 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    issue(P1{}, 1);
    read_frags(F0, smem0, smem0 + TILE, fab, faa, 0);
    read_scales(P0{}, scb, sca);

    // stages in pairs: even stages in buffer 0, odd in buffer 1
    for (int kt = 0; kt < KT; kt += 2) {
        stage(P0{}, kt);
        stage(P1{}, kt + 1);
    }
    __builtin_amdgcn_s_waitcnt(0);  // drain the loads issued past the last stage

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
                for (int e = 0; e < 4; ++e)
                    v[e] = acc[i][j][4 * g + e] + (n + e < p.N ? bias_at<BIAS>(p.bias, n + e) : 0.0f);
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
    CKH_REQUIRE(M * K < (1ll << 31) && N * K < (1ll << 31) && K < (1ll << 24),
                "scaled_mm_mxfp8: operand larger than 2 GiB");
    CKH_REQUIRE(out_code == CKH_F32 || out_code == CKH_F16 || out_code == CKH_BF16,
                "scaled_mm_mxfp8: unsupported output dtype code %d", out_code);
    CKH_REQUIRE(!bias || bias_code == CKH_F32 || bias_code == CKH_F16 || bias_code == CKH_BF16,
                "scaled_mm_mxfp8: unsupported bias dtype code %d", bias_code);
    CKH_REQUIRE(aligned(a, 16) && aligned(b, 16) && aligned(sa, 4) && aligned(sb, 4) && aligned(out, 16),
                "scaled_mm_mxfp8: pointers misaligned");
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
#define BY_BIAS(O)                                         \
    do {                                                   \
        if (!bias) LAUNCH(O, -1);                          \
        else if (bias_code == CKH_F32) LAUNCH(O, CKH_F32); \
        else if (bias_code == CKH_F16) LAUNCH(O, CKH_F16); \
        else LAUNCH(O, CKH_BF16);                          \
    } while (0)
    if (out_code == CKH_BF16) BY_BIAS(CKH_BF16);
    else if (out_code == CKH_F16) BY_BIAS(CKH_F16);
    else BY_BIAS(CKH_F32);
#undef BY_BIAS
#undef LAUNCH
    return check_launch("scaled_mm_mxfp8");
}
