// MXFP8 block-scaled GEMM for gfx950 on v_mfma_scale_f32_32x32x64_f8f6f4.
//
//   out[m, n] = sum_k A[m,k] * 2^(sa[m,k/32]-127) * B[n,k] * 2^(sb[n,k/32]-127)  (+ bias[n])
//
// A [M, K] and B [N, K] are E4M3 codes, both K-major (the reference's TN layout);
// sa / sb are E8M0 scales in the 32_4_4 swizzled layout, fed to the MFMA's scale
// operands directly (no dequantization): the four scales of a row for a 128-wide K
// block are one aligned 32-bit word, and the MFMA's opsel picks the byte.
//
// MFMA operand layout (measured on gfx950): lane l = 32*h + r holds row r; its bytes
// 0..15 are k = 16h..16h+15 and bytes 16..31 are k = 32+16h..32+16h+15 of the 64-wide
// K step; lane-half h supplies the scale of the step's K-block h.  The result lane l,
// register v holds D[8*(v/4) + 4*(l/32) + v%4][l%32].  The weight B is the MFMA's
// first operand and the activation A its second, so each lane ends with 4
// consecutive output columns of one output row.
//
// Tiling: a 256-thread workgroup computes a 256 (m) x 256 (n) tile; its 4 waves each
// own 128 x 128 = 4 x 4 MFMA tiles (256 fp32 accumulators per lane).  K advances 64
// per stage (one MFMA K-step, 16 MFMAs per wave) through 4 LDS buffers of 34 KB.
// Global data goes straight to LDS with buffer_load_dwordx4 ... lds (no VGPR
// staging): lane i of a load fills LDS bytes [base + 16 i, base + 16 i + 16), so each
// lane fetches the global chunk that belongs at its slot.  Rows past M / N, columns
// past K and stages past the end lie outside the buffer descriptors' ranges and
// arrive as zeros, so every stage runs the same branch-free code.
//
// Pipeline: at stage t (after its barrier) the fragments of t are already in
// registers, so buffer t%4 is free and receives the loads of stage t+4; the LDS
// reads of stage t+1's fragments and scale words overlap stage t's 16 MFMAs.  The
// barrier of stage t waits only until this wave's loads of stage t+1 have landed
// (vmcnt <= 20: the 10 loads each of stages t+2 and t+3 stay in flight), giving the
// global loads three stages (~3000 MFMA cycles) of latency cover.
//
// LDS rows are 64 bytes; logical 16-byte chunk c of row r lives at chunk
// c ^ ((r >> 1) & 3) ^ ((r >> 3) & 1), which makes a 32-row fragment read (one chunk
// of 32 consecutive rows) conflict-free for both 32- and 64-bank LDS layouts.
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

constexpr int BM = 256, BN = 256, BK = 64, NT = 256, NBUF = 4;
constexpr int TILE = 256 * BK;  // bytes of one operand tile per stage (16 KB)
constexpr int STILE = 1024;     // bytes of one operand's scale words per stage (256 rows)
constexpr int LOADS_PER_STAGE = 10;  // per wave: 4 + 4 data, 2 scale DMA loads

// s_waitcnt immediates (gfx9 encoding): vmcnt in [3:0] and [15:14], expcnt [6:4],
// lgkmcnt [11:8].  expcnt is left unconstrained (7).
constexpr int waitcnt_vm_lgkm0(int vm) { return (vm & 15) | (7 << 4) | ((vm >> 4) << 14); }

// Workgroup barrier after an explicit s_waitcnt.  __syncthreads() would add a release
// fence, i.e. vmcnt(0), draining the prefetched stages; here each wave has already
// waited for exactly what the barrier must publish (its DMA loads of the next stage,
// its LDS reads of the buffer about to be refilled), LDS is one coherent array per CU,
// and the empty asm statements keep the compiler from moving memory operations across.
template <int WAITCNT>
__device__ __forceinline__ void stage_barrier() {
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(WAITCNT);
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
}

// scheduling-group masks of __builtin_amdgcn_sched_group_barrier
constexpr int SG_MFMA = 0x008, SG_DS_READ = 0x100, SG_DS_WRITE = 0x200;

__device__ __forceinline__ int swz(int row) { return ((row >> 1) & 3) ^ ((row >> 3) & 1); }

// Buffer descriptor over [p, p + bytes).  The inputs are wave-uniform by construction;
// reading them through readfirstlane keeps the descriptor in SGPRs (a descriptor the
// compiler believes divergent turns every load into a per-lane loop).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a >> 32));
    void* up = reinterpret_cast<void*>((static_cast<uint64_t>(hi) << 32) | lo);
    return __builtin_amdgcn_make_buffer_rsrc(up, 0, static_cast<int>(__builtin_amdgcn_readfirstlane(bytes)),
                                             0x00020000);
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

// Direct-to-LDS loads of one operand.  Wave w, load j (0..3) covers tile rows
// R = 64 w + 16 j .. +15 (1 KB of LDS); lane i fills row R + i/4, physical chunk i%4,
// which holds logical chunk (i%4) ^ swz(row), and swz(row) depends only on i.
struct Loader {
    __amdgpu_buffer_rsrc_t rs;
    uint32_t base;     // lane's byte offset within rows R.. (k0 = 0)
    int cbyte;         // lane's chunk column in bytes (0..48)
    uint32_t rowstep;  // 16 * K: byte distance between consecutive loads j
    uint32_t row0;     // 64 * wave * K
};

__device__ __forceinline__ Loader make_loader(const uint8_t* tile_base, int valid_rows, int K, int wave, int lane) {
    Loader L;
    L.rs = make_rsrc(tile_base, static_cast<uint32_t>(max(valid_rows, 0)) * K);
    const int row = lane >> 2;  // row within a 16-row load (R is a multiple of 16)
    L.cbyte = ((lane & 3) ^ swz(row)) << 4;
    L.base = static_cast<uint32_t>(row * K + L.cbyte);
    L.rowstep = 16u * K;
    L.row0 = 64u * wave * K;
    return L;
}

__device__ __forceinline__ void issue_stage(const Loader& L, uint8_t* lds_tile, int wave, int k0, int K) {
    const uint32_t add = (k0 + L.cbyte < K) ? static_cast<uint32_t>(k0) : 0x80000000u;  // past K: zeros
#pragma unroll
    for (int j = 0; j < 4; ++j)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(L.rs, (lds_void*)(lds_tile + (64 * wave + 16 * j) * BK), 16,
                                                 L.base + L.row0 + j * L.rowstep + add, 0, 0, 0);
}

// Scale words of a stage: for a 256-row tile and one 128-wide K block they are two
// contiguous 512-byte chunks of the swizzled tensor (rows 128*rb .. +127), chunk
// (rb * ncb + k0/128).  Wave w copies chunk rb = w & 1 of operand w >> 1 (0 = weight,
// 1 = activation) with two 4-byte-per-lane DMA loads.  Inside a chunk row r's word
// sits at (r % 32) * 16 + ((r % 128) / 32) * 4, so a lane's words for its four 32-row
// tiles are one contiguous 16-byte LDS read.
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

// Byte offsets (within an operand tile) of this lane's two 16-byte fragment halves
// (chunks h and 2 + h); tile t adds t * 32 rows = t * 2048 bytes.
struct FragAddr {
    uint32_t lo, hi;
};

__device__ __forceinline__ FragAddr make_frag_addr(int row_base, int lane) {
    const int half = lane >> 5, r32 = lane & 31;
    const int row = row_base + r32;
    const int s = swz(row);
    return FragAddr{static_cast<uint32_t>(row * BK + ((half ^ s) << 4)),
                    static_cast<uint32_t>(row * BK + (((2 + half) ^ s) << 4))};
}

__device__ __forceinline__ v8i read_frag(const uint8_t* tile, const FragAddr& f) {
    const v4u x = *reinterpret_cast<const v4u*>(tile + f.lo);
    const v4u y = *reinterpret_cast<const v4u*>(tile + f.hi);
    v8i r;
    r[0] = x[0]; r[1] = x[1]; r[2] = x[2]; r[3] = x[3];
    r[4] = y[0]; r[5] = y[1]; r[6] = y[2]; r[7] = y[3];
    return r;
}

__device__ __forceinline__ void read_frags(Frags& F, const uint8_t* stage_buf, const FragAddr& fb,
                                           const FragAddr& fa) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        F.b[t] = read_frag(stage_buf + t * 32 * BK, fb);
        F.a[t] = read_frag(stage_buf + TILE + t * 32 * BK, fa);
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
    // One LDS array per buffer, indexed at compile time, so the compiler can prove the
    // in-flight DMA writes never alias the fragment reads and adds no waits of its own.
    __shared__ __attribute__((aligned(1024))) uint8_t buf0[2 * TILE + 2 * STILE];
    __shared__ __attribute__((aligned(1024))) uint8_t buf1[2 * TILE + 2 * STILE];
    __shared__ __attribute__((aligned(1024))) uint8_t buf2[2 * TILE + 2 * STILE];
    __shared__ __attribute__((aligned(1024))) uint8_t buf3[2 * TILE + 2 * STILE];

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

    auto buf = [&](auto b_c) -> uint8_t* {
        constexpr int B = decltype(b_c)::value & 3;
        return B == 0 ? buf0 : B == 1 ? buf1 : B == 2 ? buf2 : buf3;
    };
    auto issue = [&](auto b_c, int s) {
        uint8_t* b = buf(b_c);
        issue_stage(LB, b, wave, s * BK, p.K);
        issue_stage(LA, b + TILE, wave, s * BK, p.K);
        issue_scales(rssb, rssa, n0 >> 7, m0 >> 7, p.ncb, s * BK, p.K, b + 2 * TILE, wave, lane);
    };
    // this lane's 4 scale words (tiles t = 0..3) of each operand for a stage, shifted so
    // byte 0 / byte 2 are the lane-half's scales of the even / odd 64-wide stage
    const int hs = 8 * half;
    auto read_scales = [&](auto b_c, uint32_t (&sb)[4], uint32_t (&sa)[4]) {
        const uint8_t* st = buf(b_c) + 2 * TILE;
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

    // Stage t held in buffer B = t % 4 (compile-time): fragments F (stage t) are in
    // registers; read stage t+1 into G while issuing stage t+4 into buffer B.
    auto stage = [&](auto b_c, int t, Frags& F, Frags& G) {
        constexpr int B = decltype(b_c)::value;
        using Next = std::integral_constant<int, (B + 1) & 3>;
        stage_barrier<waitcnt_vm_lgkm0(2 * LOADS_PER_STAGE)>();
        uint32_t nb[4], na[4];
        issue(b_c, t + NBUF);
        read_frags(G, buf(Next{}), fab, faa);
        read_scales(Next{}, nb, na);
        if constexpr ((B & 1) == 0) mfma16<0>(acc, F, scb, sca);
        else mfma16<2>(acc, F, scb, sca);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
            __builtin_amdgcn_sched_group_barrier(SG_DS_READ, 2, 0);
            __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
            __builtin_amdgcn_sched_group_barrier(SG_DS_WRITE, 1, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            scb[i] = nb[i];
            sca[i] = na[i];
        }
    };

    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
    using B2 = std::integral_constant<int, 2>;
    using B3 = std::integral_constant<int, 3>;

    // prologue: stages 0..3 in flight, stage 0 resident and read
    issue(B0{}, 0);
    issue(B1{}, 1);
    issue(B2{}, 2);
    issue(B3{}, 3);
    stage_barrier<waitcnt_vm_lgkm0(3 * LOADS_PER_STAGE)>();
    read_frags(F0, buf0, fab, faa);
    read_scales(B0{}, scb, sca);

    // stages in groups of 4 (buffer index = stage % 4); stages past K are all zeros
    for (int t = 0; t < KT; t += 4) {
        stage(B0{}, t, F0, F1);
        stage(B1{}, t + 1, F1, F0);
        stage(B2{}, t + 2, F0, F1);
        stage(B3{}, t + 3, F1, F0);
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
