// NVFP4 block-scaled GEMM for gfx950.
//
//   out[m, n] = alpha * sum_k E2M1(a[m,k]) * sa[m,k/16] * E2M1(b[n,k]) * sb[n,k/16]  (+ bias[n])
//
// a [M, K/2], b [N, K/2]: packed E2M1 codes, both K-major; sa / sb: E4M3 scales per
// 16 elements in the 32_4_4 swizzled layout; alpha: one fp32 on the device
// (tensor_scale_a * tensor_scale_b).
//
// Arithmetic.  The gfx950 block-scaled MFMAs take only power-of-two (E8M0) scales, and
// E2M1 * E4M3 needs up to 6 significant bits, so no FP8/FP6/FP4 element format holds
// the scaled values exactly.  Each E2M1 code times its E4M3 block scale is an exact
// fp16 (magnitudes in [2^-10, 2688]), so the operands are decoded to fp16 in registers
// (v_cvt_scalef32_pk_f16_fp4 with scale 1, then a packed multiply by the block scale,
// itself converted with v_cvt_scalef32_pk_f16_fp8) and multiplied with
// v_mfma_f32_32x32x16_f16 (fp32 accumulation); alpha and bias are applied in the
// epilogue.  Any consistent assignment of k to MFMA lanes gives the same dot product,
// so both operands use the same one and nibble order inside a byte does not matter.
//
// Tiling: a 256-thread workgroup computes a 256 (m) x 256 (n) tile, 4 waves of
// 128 x 128 (4 x 4 MFMA tiles, 256 fp32 accumulators per lane).  A stage is 64 K
// elements: 32 packed bytes per row and one 32-bit word of four block scales per row.
// Packed codes and scale words go to LDS unchanged (4x less LDS traffic than fp16
// tiles) in groups of 4 stages (one 128-byte line per row), double-buffered, by
// buffer_load_dwordx4 ... lds: 18 direct-to-LDS loads per wave per group, one barrier
// per group, and a whole group (~8000 MFMA cycles) of latency cover.  A last round of
// tiles at most half full, and the split-K of a grid of at most 64 tiles, run 256 x 128
// column halves instead (each wave 128 x 64; the same body with NW = 2 weight tiles per
// wave): twice the workgroups for the CUs the grid would leave idle.
//
// Within a stage each lane needs, per 32-row tile, 16 bytes (32 codes: k = 32h ..
// 32h+31 of the stage for lane half h, of which MFMA substep kk uses bytes 4kk..4kk+3)
// and the tile row's scale word (blocks 2h and 2h+1 are its); one ds_read_b128 each.
// Each of a substep's 16 MFMAs sits in a slot of its own (sched_barrier) with 1/16 of
// the next substep's decode (two converts, two packed multiplies), and in the first
// substep one of the next stage's 10 LDS reads and, in the last stage of a group, one
// of the 18 loads of the group after next.  A 32-cycle f16 MFMA hides about 8 such
// VALU instructions; left to itself the compiler clustered the decode between runs of
// back-to-back MFMAs, which kept the matrix cores 60% busy instead of 77%.
//
// LDS rows are 128 bytes (a group); logical 16-byte chunk c of row r is stored at
// chunk c ^ (r & 7) ^ ((r >> 3) & 1), so any 16 consecutive rows of a fragment read
// hit distinct banks of the 64-bank LDS (measured: no bank conflicts; with c ^ (r & 7)
// rows r and r + 8 collided).  Workgroups walk the tiles XCD-contiguously in grouped
// order, as in the MXFP8 kernel.
#include <type_traits>
#include <utility>

#include "ckh_common.h"
#include "quant_math.h"
#include "skinny.h"

namespace ckh {
namespace nv {

using ckh::v8h;
using ckh::v2h;
typedef float v16f __attribute__((ext_vector_type(16)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int BM = 256, BN = 256, NT = 256;
constexpr int SKB = 32;                     // packed bytes per row per stage (64 elements)
constexpr int GS = 4;                       // stages per group
constexpr int GKB = SKB * GS;               // bytes per row per group: one 128-byte line
constexpr int TILE = 256 * GKB;             // one operand's codes per group (32 KB)
constexpr int STILE = 256 * 4 * GS;         // one operand's scale words per group (4 KB)
constexpr int GBUF = 2 * TILE + 2 * STILE;  // one group buffer: b codes, a codes, b scales, a scales
constexpr int EPI_ROW = 520;                // bytes of one staged 16-bit output row (512 + 8 pad)
static_assert(128 * EPI_ROW <= GBUF, "half the output tile must fit one group buffer");
// direct-to-LDS loads per wave per group of a 256 x 64 NW tile: 2 NW weight-code loads,
// 8 activation-code loads, 2 scale loads (18 for full tiles, 14 for half tiles)
constexpr int loads_per_group(int NW) { return 2 * NW + 8 + 2; }

// fn(integral_constant<int, K>) for each K in order
template <typename Fn, int... K>
__device__ __forceinline__ void for_each_index(Fn&& fn, std::integer_sequence<int, K...>) {
    (fn(std::integral_constant<int, K>{}), ...);
}

// s_waitcnt immediate: vmcnt in [3:0] and [15:14], expcnt [6:4] (left at 7), lgkmcnt 0
constexpr int waitcnt_vm_lgkm0(int vm) { return (vm & 15) | (7 << 4) | ((vm >> 4) << 14); }

// Barrier after an explicit wait; the empty asm statements keep memory operations from
// moving across (a __syncthreads() fence would also drain the prefetched group).
template <int WAITCNT>
__device__ __forceinline__ void group_barrier() {
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(WAITCNT);
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
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
    int ncb;      // scale word columns: ceil(K/16/4)
    int sa_rows, sb_rows;
    int tiles_m, tiles_n;
    int n_full;  // workgroups [0, n_full) compute full tiles 0 .. n_full-1 (grouped order)
    int n_half;  // workgroups n_full + 2 i, +1 compute the two column halves of tile n_full + i
    // split-K mode (gemm_split_kernel): workgroup U * splits + s computes groups
    // [s * ks, min((s + 1) * ks, NG)) of tile (or half tile) U and writes its fp32 partial
    int splits, ks;
    float* part;
};

// fp32 values of one partial tile in the workspace (256 x 256, or two 256 x 128 halves)
constexpr int kPartTile = BM * BN;

// Direct-to-LDS loads of one operand's group.  Wave w, load j (0..7) covers rows
// R = 64 w + 8 j .. +7 (1 KB of LDS; 32 w + 8 j, j = 0..3, for a 128-row half tile);
// lane i fills row R + i/8, physical chunk i%8, which holds logical chunk
// (i%8) ^ (i/8) ^ (j & 1) (R is a multiple of 8, and bit 3 of the row is j's lowest bit).
struct Loader {
    __amdgpu_buffer_rsrc_t rs;
    uint32_t voff;     // lane's byte offset for j = 0 and group 0
    int cbyte;         // 16 * logical chunk for even j
    uint32_t cdelta;   // byte offset of odd j's chunk relative to even j's (+-16)
    uint32_t rowstep;  // 8 rows
};

__device__ __forceinline__ Loader make_loader(const uint8_t* tile_base, int valid_rows, int Kb, int wave, int lane,
                                             int rows_per_wave = 64) {
    Loader L;
    L.rs = buffer_rsrc(tile_base, static_cast<uint32_t>(max(valid_rows, 0)) * Kb);
    const int row = rows_per_wave * wave + (lane >> 3);
    L.cbyte = ((lane & 7) ^ (lane >> 3)) << 4;
    L.cdelta = static_cast<uint32_t>((L.cbyte ^ 16) - L.cbyte);
    L.voff = static_cast<uint32_t>(row * Kb + L.cbyte);
    L.rowstep = 8u * Kb;
    return L;
}

// Load j (0..7, or 0..3 for 32 rows per wave) of issue_codes alone.  With 32 rows per
// wave, R = 32 w + 8 j still has bit 3 equal to j's lowest bit.
template <int RPW = 64>
__device__ __forceinline__ void issue_code_part(const Loader& L, uint8_t* dst, int wave, int kb0, int Kb, int j) {
    const int cb = (j & 1) ? (L.cbyte ^ 16) : L.cbyte;
    const uint32_t add = (kb0 + cb < Kb) ? static_cast<uint32_t>(kb0) : 0x80000000u;  // past K: zeros
    __builtin_amdgcn_raw_ptr_buffer_load_lds(L.rs, (lds_void*)(dst + (RPW * wave + 8 * j) * GKB), 16,
                                             L.voff + j * L.rowstep + ((j & 1) ? L.cdelta : 0) + add, 0, 0, 0);
}

template <int RPW = 64>
__device__ __forceinline__ void issue_codes(const Loader& L, uint8_t* dst, int wave, int kb0, int Kb) {
#pragma unroll
    for (int j = 0; j < RPW / 8; ++j) issue_code_part<RPW>(L, dst, wave, kb0, Kb, j);
}

// Scale words of a group: for a 256-row tile, 128-row block rb and word column c, the
// 512-byte chunk ((rb0 + rb) * ncb + c) of the swizzled tensor; the 4 columns of a group
// are contiguous, so each block's group is one 2 KB run.  Wave w copies block rb = w & 1
// of operand w >> 1 (0 = weight, 1 = activation): 2 loads of 1 KB.  Columns from cend on
// (the last, or the end of a split's K range) and blocks past the padded rows arrive as
// zeros.  Inside a chunk row r's
// word sits at (r % 32) * 16 + ((r % 128) / 32) * 4.
__device__ __forceinline__ void issue_scales(__amdgpu_buffer_rsrc_t rs_b, __amdgpu_buffer_rsrc_t rs_a, int rb0_b,
                                             int rb0_a, int ncb, int cend, int g, uint8_t* sdst, int wave, int lane,
                                             int q0 = 0, int q1 = 2) {
    const int op = wave >> 1, rb = wave & 1;
    const __amdgpu_buffer_rsrc_t rs = op ? rs_a : rs_b;
    const int base = (op ? rb0_a : rb0_b) + rb;
#pragma unroll
    for (int q = q0; q < q1; ++q) {
        const int col = GS * g + 2 * q + (lane >> 5);
        const uint32_t off =
            col < cend ? static_cast<uint32_t>((base * ncb + col) * 512 + (lane & 31) * 16) : 0x80000000u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(sdst + op * STILE + rb * 2048 + q * 1024), 16, off,
                                                 0, 0, 0);
    }
}

// One stage's raw operands for this lane: per tile 16 code bytes + the scale word.
struct Raw {
    v4u b[4], a[4];
    v4u wb, wa;  // scale words of tiles 0..3
};

// Decoded fp16 operands of one MFMA substep.
struct Dec {
    v8h b[4], a[4];
};


template <int OUT>
__device__ __forceinline__ uint32_t pack2(float x, float y) {
    return (OUT == CKH_BF16 ? f_to_bf16_rne(x) : f_to_f16(x)) |
           ((OUT == CKH_BF16 ? f_to_bf16_rne(y) : f_to_f16(y)) << 16);
}

template <int OUT>
__device__ __forceinline__ void store4(void* out, int64_t idx, const float (&v)[4]) {
    if constexpr (OUT == CKH_F32) {
        *reinterpret_cast<float4*>(static_cast<float*>(out) + idx) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + idx) =
            make_uint2(pack2<OUT>(v[0], v[1]), pack2<OUT>(v[2], v[3]));
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

// NW: 32-column MFMA tiles per wave along n: 4 for 256 x 256 workgroup tiles, 2 for the
// 256 x 128 column halves of a tile (each wave 128 x 64: 8 MFMAs per substep instead of
// 16, with 6 of the 8 operand tiles decoded).
template <int OUT, int BIAS, int NW, bool SPLIT = false>
__device__ __forceinline__ void gemm_tile(const Args& p, int bid, uint8_t* lds0, uint8_t* lds1) {
    constexpr int TBN = 64 * NW;         // tile width along n
    constexpr int RPW = TBN / 4;         // weight rows loaded per wave
    constexpr int SLOTS = 4 * NW;        // MFMAs per wave per substep
    constexpr int NREAD = NW + 6;        // LDS reads per wave per stage
    constexpr int NDEC = 2 * NW + 8;     // decode parts per substep
    constexpr int NLD = loads_per_group(NW);
    // Workgroups are dispatched round-robin over the 8 XCDs; full tiles are remapped so
    // each XCD walks a contiguous range of tiles (in grouped order).  Half tiles give tile
    // L's two column halves to consecutive workgroups.  Split-K workgroups take tile (or
    // half tile) bid / splits, K range bid % splits.
    const int split = SPLIT ? bid % p.splits : 0;
    if (SPLIT) bid /= p.splits;
    else if (NW == 4 && (p.n_full & 7) == 0) bid = (bid & 7) * (p.n_full >> 3) + (bid >> 3);
    const int L = (NW == 4) ? bid : (SPLIT ? 0 : p.n_full) + (bid >> 1);
    int tm, tn;
    grouped_tile(L, p.tiles_m, p.tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN + (NW == 4 ? 0 : (bid & 1) * TBN);
    if (n0 >= p.N) return;  // a half tile wholly past N (uniform over the workgroup)

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave & 1, wn = wave >> 1;
    const int half = lane >> 5, r32 = lane & 31;
    const int Kb = p.K / 2;

    const Loader LB = make_loader(p.b + static_cast<int64_t>(n0) * Kb, min(TBN, p.N - n0), Kb, wave, lane, RPW);
    const Loader LA = make_loader(p.a + static_cast<int64_t>(m0) * Kb, min(BM, p.M - m0), Kb, wave, lane);
    const __amdgpu_buffer_rsrc_t rssb = buffer_rsrc(p.sb, static_cast<uint32_t>(p.sb_rows) * p.ncb * 4);
    const __amdgpu_buffer_rsrc_t rssa = buffer_rsrc(p.sa, static_cast<uint32_t>(p.sa_rows) * p.ncb * 4);
    const int NG = (Kb + GKB - 1) / GKB;  // groups of 256 elements
    // this workgroup's groups [gb, ge), the code bytes and scale-word columns they cover:
    // loads past them read zeros
    const int gb = SPLIT ? split * p.ks : 0;
    const int ge = SPLIT ? min(gb + p.ks, NG) : NG;
    const int kend = SPLIT ? min(ge * GKB, Kb) : Kb;
    const int cend = SPLIT ? min(p.ncb, ge * GS) : p.ncb;

    v16f acc[NW][4];
#pragma unroll
    for (int i = 0; i < NW; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = v16f{};

    auto gbuf = [&](auto g_c) -> uint8_t* { return (decltype(g_c)::value & 1) ? lds1 : lds0; };
    auto issue_group = [&](auto g_c, int g) {
        uint8_t* d = gbuf(g_c);
        issue_codes<RPW>(LB, d, wave, g * GKB, kend);
        issue_codes(LA, d + TILE, wave, g * GKB, kend);
        issue_scales(rssb, rssa, n0 >> 7, m0 >> 7, p.ncb, cend, g, d + 2 * TILE, wave, lane);
    };
    // load I (0..NLD-1) of issue_group: weight codes 0..2NW-1, then 8 activation codes,
    // then the 2 scale loads (a half tile's wave also copies the scale words of the 128
    // weight rows after its own, which it does not read, so that every wave issues the same
    // number of loads)
    auto issue_part = [&](auto g_c, int g, auto i_c) {
        constexpr int I = decltype(i_c)::value;
        uint8_t* d = gbuf(g_c);
        if constexpr (I < 2 * NW) issue_code_part<RPW>(LB, d, wave, g * GKB, kend, I);
        else if constexpr (I < 2 * NW + 8) issue_code_part(LA, d + TILE, wave, g * GKB, kend, I - 2 * NW);
        else issue_scales(rssb, rssa, n0 >> 7, m0 >> 7, p.ncb, cend, g, d + 2 * TILE, wave, lane, I - 2 * NW - 8,
                          I - 2 * NW - 7);
    };

    // lane's fragment and scale-word addresses inside a group buffer
    const int x7 = (r32 & 7) ^ ((r32 >> 3) & 1);
    const uint32_t frow_b = static_cast<uint32_t>((wn * 32 * NW + r32) * GKB);
    const uint32_t frow_a = static_cast<uint32_t>(TILE + (wm * 128 + r32) * GKB);
    // (a half tile's weight rows are one 128-row block, whose word (r % 128) / 32 is this
    // wave's tile 2 wn + i: the two words at byte 8 wn of the lane's 16)
    const uint32_t sw_b = static_cast<uint32_t>(2 * TILE + (NW == 4 ? wn * 2048 : 8 * wn) + r32 * 16);
    const uint32_t sw_a = static_cast<uint32_t>(2 * TILE + STILE + wm * 2048 + r32 * 16);
    // One of the NREAD LDS reads of a stage's raw operands: weight tiles 0..NW-1,
    // activation tiles NW..NW+3, scale words NW+4 (weight) and NW+5 (activation).
    auto read_part = [&](const uint8_t* gb, auto s_c, auto i_c, Raw& R) {
        constexpr int S = decltype(s_c)::value, I = decltype(i_c)::value;
        const uint32_t chunk = static_cast<uint32_t>(((2 * S + half) ^ x7) << 4);
        if constexpr (I < NW) {
            R.b[I] = *reinterpret_cast<const v4u*>(gb + frow_b + I * 32 * GKB + chunk);
        } else if constexpr (I < NW + 4) {
            R.a[I - NW] = *reinterpret_cast<const v4u*>(gb + frow_a + (I - NW) * 32 * GKB + chunk);
        } else if constexpr (I == NW + 4) {
            if constexpr (NW == 4) {
                R.wb = *reinterpret_cast<const v4u*>(gb + sw_b + S * 512);
            } else {
                const uint2 w = *reinterpret_cast<const uint2*>(gb + sw_b + S * 512);
                R.wb[0] = w.x;
                R.wb[1] = w.y;
            }
        } else {
            R.wa = *reinterpret_cast<const v4u*>(gb + sw_a + S * 512);
        }
    };
    const int sh = 16 * half;
    // Part P (0..NDEC-1) of decoding substep KK of R into D (dword KK of each tile, block
    // 2h + KK/2): half P & 1 of weight tile P / 2 (P < 2 NW) or of activation tile
    // P / 2 - NW, i.e. two converts and two scale multiplies.
    auto decode_part = [&](const Raw& R, auto kk_c, auto p_c, Dec& D) {
        constexpr int KK = decltype(kk_c)::value, P = decltype(p_c)::value;
        constexpr bool A = P >= 2 * NW;
        constexpr int t = A ? (P - 2 * NW) >> 1 : P >> 1, h = P & 1;
        const v2h pr = scale_pair(A ? R.wa[t] : R.wb[t], sh);
        const v2h sc = KK < 2 ? v2h{pr[0], pr[0]} : v2h{pr[1], pr[1]};
        const uint32_t w = A ? R.a[t][KK] : R.b[t][KK];
        const v2h e0 = decode2<2 * h>(w, sc);
        const v2h e1 = decode2<2 * h + 1>(w, sc);
        v8h& d = A ? D.a[t] : D.b[t];
        d[4 * h] = e0[0];
        d[4 * h + 1] = e0[1];
        d[4 * h + 2] = e1[0];
        d[4 * h + 3] = e1[1];
    };
    // The SLOTS MFMAs of one substep on Dc, each in a slot of its own with its share of the
    // decode of (Rd, KKd) into Dn (one part each for full tiles; half tiles add the last 4
    // parts to the even slots) and, per the flags, one LDS read of the next stage and one
    // load of the group after next (LD 1: loads 0..SLOTS-1, LD 2: the rest); the slots keep
    // the decode's VALU work spread between the MFMAs (the compiler would otherwise cluster
    // it).
    auto substep = [&](const Dec& Dc, const Raw& Rd, auto kkd_c, Dec& Dn, auto rd_c, const uint8_t* nb, auto sn_c,
                       Raw& Rn, auto ld_c, auto lg_c, int lg) {
        constexpr int RD = decltype(rd_c)::value, LD = decltype(ld_c)::value;
        for_each_index([&](auto i_c) {
            constexpr int i = decltype(i_c)::value;
            acc[i >> 2][i & 3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(Dc.b[i >> 2], Dc.a[i & 3], acc[i >> 2][i & 3],
                                                                        0, 0, 0);
            decode_part(Rd, kkd_c, i_c, Dn);
            if constexpr (NDEC > SLOTS && (i & 1) == 0)
                decode_part(Rd, kkd_c, std::integral_constant<int, SLOTS + i / 2>{}, Dn);
            if constexpr (RD && i < NREAD) read_part(nb, sn_c, i_c, Rn);
            if constexpr (LD == 1) issue_part(lg_c, lg, i_c);
            if constexpr (LD == 2 && i < NLD - SLOTS) issue_part(lg_c, lg, std::integral_constant<int, SLOTS + i>{});
            __builtin_amdgcn_sched_barrier(0);
        }, std::make_integer_sequence<int, SLOTS>{});
    };
    Raw R0, R1;
    Dec D0, D1;
    using G0 = std::integral_constant<int, 0>;
    using G1 = std::integral_constant<int, 1>;
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    using S2 = std::integral_constant<int, 2>;
    using S3 = std::integral_constant<int, 3>;
    using K0 = std::integral_constant<int, 0>;
    using K1 = std::integral_constant<int, 1>;
    using K2 = std::integral_constant<int, 2>;
    using K3 = std::integral_constant<int, 3>;

    // One stage: the MFMAs of substeps 0..3 on R (each substep decoded one ahead), the
    // next stage's raw operands read into Rn during substep 1, and substep 0 of Rn
    // decoded during substep 3.  Before the last stage of a group reads the next group,
    // that group must be resident: wait for this wave's loads, barrier (after which no
    // wave reads group g's buffer any more), then refill that buffer with group g + 2.
    auto stage = [&](auto g_c, auto s_c, int g, Raw& R, Raw& Rn) {
        constexpr int G = decltype(g_c)::value, S = decltype(s_c)::value;
        using GN = std::integral_constant<int, (S == GS - 1) ? (G ^ 1) : G>;
        using SN = std::integral_constant<int, (S + 1) % GS>;
        using T = std::integral_constant<int, 1>;
        using F = std::integral_constant<int, 0>;
        using L1 = std::integral_constant<int, (S == GS - 1) ? 1 : 0>;
        using L2 = std::integral_constant<int, (S == GS - 1) ? 2 : 0>;
        if constexpr (S == GS - 1) group_barrier<waitcnt_vm_lgkm0(0)>();
        substep(D0, R, K1{}, D1, T{}, gbuf(GN{}), SN{}, Rn, L1{}, g_c, g + 2);
        substep(D1, R, K2{}, D0, F{}, gbuf(GN{}), SN{}, Rn, L2{}, g_c, g + 2);
        substep(D0, R, K3{}, D1, F{}, gbuf(GN{}), SN{}, Rn, F{}, g_c, g + 2);
        substep(D1, Rn, K0{}, D0, F{}, gbuf(GN{}), SN{}, Rn, F{}, g_c, g + 2);
    };

    // prologue: groups 0 and 1 in flight, group 0 resident, stage 0 read and decoded
    issue_group(G0{}, gb);
    issue_group(G1{}, gb + 1);
    group_barrier<waitcnt_vm_lgkm0(NLD)>();
    for_each_index([&](auto i_c) { read_part(lds0, S0{}, i_c, R0); }, std::make_integer_sequence<int, NREAD>{});
    for_each_index([&](auto p_c) { decode_part(R0, K0{}, p_c, D0); }, std::make_integer_sequence<int, NDEC>{});

    // groups in pairs (buffer = (group - gb) % 2); an odd count ends after the first group of
    // its last pair (the second, past the range, was loaded as zeros and is not computed)
    int g = gb;
    for (; g + 1 < ge; g += 2) {
        stage(G0{}, S0{}, g, R0, R1);
        stage(G0{}, S1{}, g, R1, R0);
        stage(G0{}, S2{}, g, R0, R1);
        stage(G0{}, S3{}, g, R1, R0);
        stage(G1{}, S0{}, g + 1, R0, R1);
        stage(G1{}, S1{}, g + 1, R1, R0);
        stage(G1{}, S2{}, g + 1, R0, R1);
        stage(G1{}, S3{}, g + 1, R1, R0);
    }
    if (g < ge) {
        stage(G0{}, S0{}, g, R0, R1);
        stage(G0{}, S1{}, g, R1, R0);
        stage(G0{}, S2{}, g, R0, R1);
        stage(G0{}, S3{}, g, R1, R0);
    }
    // the loads of the groups past the end still write LDS, which the epilogue reuses
    __builtin_amdgcn_s_waitcnt(0);
    if constexpr (SPLIT) {
        // The raw fp32 accumulators go to the workspace in register order: float4 g of
        // MFMA tile (i, j) of wave w, lane l at ((w * 4 NW + 4 i + j) * 4 + g) * 64 + l, so
        // every store instruction writes 1 KB contiguously.  The reduce kernel adds the
        // splits and runs the epilogue.
        constexpr int kPart = BM * TBN;  // fp32 values of one partial (half) tile
        float4* dst = reinterpret_cast<float4*>(p.part) + (static_cast<int64_t>(bid) * p.splits + split) * (kPart / 4) +
                      wave * (kPart / 16) + lane;
#pragma unroll
        for (int i = 0; i < NW; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int g = 0; g < 4; ++g)
                    dst[((4 * i + j) * 4 + g) * 64] =
                        make_float4(acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]);
        return;
    }
    __syncthreads();

    // Epilogue: lane holds out[m][n..n+3] for m = r32-th row of activation tile j and
    // n = 8*gg + 4*half (+0..3) of weight tile i; times alpha, plus bias.
    const float alpha = p.alpha[0];
    auto value = [&](float a, int n) { return a * alpha + (n < p.N ? bias_at<BIAS>(p.bias, n) : 0.0f); };
    if constexpr (OUT != CKH_F32) {
        // Stage the 16-bit tile in LDS as 256 rows of EPI_ROW bytes (rows 0..127 in
        // buffer 0, 128..255 in buffer 1; the 520-byte pitch spreads a fragment's 32 rows
        // over distinct bank pairs), then each wave stores 64 whole rows, 8 bytes per lane:
        // one 512-byte row per instruction (full tiles) or two 256-byte rows (half tiles).
        auto row_ptr = [&](int r) -> uint8_t* { return r < 128 ? lds0 + r * EPI_ROW : lds1 + (r - 128) * EPI_ROW; };
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint8_t* rowp = row_ptr(wm * 128 + j * 32 + r32);
#pragma unroll
            for (int i = 0; i < NW; ++i) {
#pragma unroll
                for (int gg = 0; gg < 4; ++gg) {
                    const int nl = wn * 32 * NW + i * 32 + 8 * gg + 4 * half;
                    const int n = n0 + nl;
                    *reinterpret_cast<uint2*>(rowp + nl * 2) =
                        make_uint2(pack2<OUT>(value(acc[i][j][4 * gg], n), value(acc[i][j][4 * gg + 1], n + 1)),
                                   pack2<OUT>(value(acc[i][j][4 * gg + 2], n + 2), value(acc[i][j][4 * gg + 3], n + 3)));
                }
            }
        }
        __syncthreads();
        constexpr int LPR = TBN / 4;   // lanes per output row, 8 bytes (4 values) each
        constexpr int RPI = 64 / LPR;  // rows per store instruction
        const int lr = lane % LPR, lrow = lane / LPR;
        const int n = n0 + 4 * lr;
        const bool vec = (p.N & 3) == 0 && n + 4 <= p.N;
        const int rows = min(64, p.M - (m0 + wave * 64)) - lrow;
        uint16_t* orow = static_cast<uint16_t*>(p.out) + static_cast<int64_t>(m0 + wave * 64 + lrow) * p.N + n;
#pragma unroll 8
        for (int rl = 0; rl < 64; rl += RPI) {
            const uint2 d = *reinterpret_cast<const uint2*>(row_ptr(wave * 64 + rl + lrow) + lr * 8);
            if (rl >= rows) break;
            uint16_t* o = orow + static_cast<int64_t>(rl) * p.N;
            if (vec) {
                st_stream8(o, d);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (n + e < p.N) o[e] = static_cast<uint16_t>((e < 2 ? d.x : d.y) >> (16 * (e & 1)));
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int m = m0 + wm * 128 + j * 32 + r32;
            if (m >= p.M) continue;
#pragma unroll
            for (int i = 0; i < NW; ++i) {
#pragma unroll
                for (int gg = 0; gg < 4; ++gg) {
                    const int n = n0 + wn * 32 * NW + i * 32 + 8 * gg + 4 * half;
                    float v[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = value(acc[i][j][4 * gg + e], n + e);
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
}

template <int OUT, int BIAS>
__global__ __launch_bounds__(NT) void gemm_kernel(Args p) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds0[GBUF];
    __shared__ __attribute__((aligned(1024))) uint8_t lds1[GBUF];
    const int b = blockIdx.x;
    if (b < p.n_full) gemm_tile<OUT, BIAS, 4>(p, b, lds0, lds1);
    else gemm_tile<OUT, BIAS, 2>(p, b - p.n_full, lds0, lds1);
}

// Split-K, first launch: each workgroup one K range of one 256 x 256 tile (NW = 4) or
// 256 x 128 half tile (NW = 2), partial sums to the workspace (alpha and bias are applied
// by the reduce kernel).
template <int NW>
__global__ __launch_bounds__(NT) void gemm_split_kernel(Args p) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds0[GBUF];
    __shared__ __attribute__((aligned(1024))) uint8_t lds1[GBUF];
    gemm_tile<CKH_F32, -1, NW, true>(p, blockIdx.x, lds0, lds1);
}

// Split-K, second launch: thread q adds float4 q % U of unit q / U (U = 4096 NW float4 of
// a tile or half tile) over the splits in split order, times alpha, plus bias, and stores
// out[m][n .. n + 3] (the register mapping of the tile epilogue).
template <int OUT, int BIAS, int NW>
__global__ __launch_bounds__(256) void gemm_reduce_kernel(Args p) {
    constexpr int kUnit = BM * 64 * NW / 4;  // float4 of one partial (half) tile
    constexpr int kLog = NW == 4 ? 14 : 13;
    static_assert(kUnit == 1 << kLog, "unit size");
    const int64_t q = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int U = static_cast<int>(q >> kLog);
    if (U >= p.tiles_m * p.tiles_n * (4 / NW)) return;
    const int rest = static_cast<int>(q & (kUnit - 1));
    const int wave = rest >> (kLog - 2), ij = (rest >> 8) & (4 * NW - 1), g = (rest >> 6) & 3, lane = rest & 63;
    const int i = ij >> 2, j = ij & 3;
    const float4* src = reinterpret_cast<const float4*>(p.part) + static_cast<int64_t>(U) * p.splits * kUnit + rest;
    float4 v = src[0];
    for (int s = 1; s < p.splits; ++s) {
        const float4 w = src[static_cast<int64_t>(s) * kUnit];
        v.x += w.x;
        v.y += w.y;
        v.z += w.z;
        v.w += w.w;
    }
    const int L = NW == 4 ? U : U >> 1;
    int tm, tn;
    grouped_tile(L, p.tiles_m, p.tiles_n, tm, tn);
    const int m = tm * BM + (wave & 1) * 128 + j * 32 + (lane & 31);
    const int n = tn * BN + (NW == 4 ? 0 : (U & 1) * 128) + (wave >> 1) * 32 * NW + i * 32 + 8 * g + 4 * (lane >> 5);
    if (m >= p.M || n >= p.N) return;
    const float alpha = p.alpha[0];
    const float s4[4] = {v.x, v.y, v.z, v.w};
    float o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = s4[e] * alpha + (n + e < p.N ? bias_at<BIAS>(p.bias, n + e) : 0.0f);
    const int64_t idx = static_cast<int64_t>(m) * p.N + n;
    if (n + 3 < p.N && (p.N & 3) == 0) {
        store4<OUT>(p.out, idx, o);
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (n + e < p.N) store1<OUT>(p.out, idx + e, o[e]);
    }
}

}  // namespace nv

// ------------------------------------------------------------ skinny activations
// GEMMs with few activation rows (M <= 64) stream the weight once and are bound by HBM
// bandwidth on it; the 256 x 256 tiles above would give them only N / 256 workgroups.  A
// workgroup owns 32 or 64 weight rows and all of K; its waves split K in chunks of 128 code
// bytes per row (256 elements: 4 stages of 64, 4 scale words per row), chunk c to wave
// c % WV, and each wave keeps two chunks in flight: its weight rows go to one of two LDS
// buffers by whole-line direct-to-LDS loads, scale words and activation codes to registers,
// and the loads of chunk i + 2 are issued as soon as chunk i's LDS reads are done.
//
// Operands are decoded to fp16 as in the tile kernel (lane l = 32 h + r: row r, code bytes
// 16 h .. 16 h + 15 of each 32-byte stage, dword kk for MFMA substep kk, whose block scale is
// byte 2 h + kk / 2 of the row's scale word) and multiplied with v_mfma_f32_32x32x16_f16.
// With M <= 16 most of a 32-row MFMA operand is padding, so the activation (AR = 8 or 16
// rows) is decoded once per chunk by the whole wave, 32 elements a lane, into an fp16 area
// of LDS, and its fragments are read from there; lanes of rows past AR read a zero row.
// Larger M decode their activation fragments in registers, each feeding NT MFMAs.  At the
// end the K partials meet in LDS and each wave adds and stores its share of the tile, times
// alpha, plus bias.  Rows past M or N, bytes past K and scale columns past the last read as
// zeros.
namespace nvsk {

using namespace ckh::sk;
using ckh::v8h;
using ckh::v2h;
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kStages = kCb / 32;    // 64-element stages (and scale words of a row) per chunk: 4
constexpr int kApitch = 2 * 2 * kCb + 16;  // bytes of one decoded fp16 activation row (+16 pad)

struct Args {
    const uint8_t* a;
    const uint8_t* b;
    const uint8_t* sa;
    const uint8_t* sb;
    const float* alpha;
    const void* bias;
    void* out;
    int M, N, K;           // K in elements
    int ncb;               // scale word columns: ceil(K/16/4)
    int sa_rows, sb_rows;  // padded scale rows (multiples of 128)
};

// One chunk's register-held operands.
template <int NT, int MT, int AR, int AS>
struct Regs {
    uint32_t swb[kStages][NT];  // weight scale words, one per stage
    // AR > 0: the lane's 32 activation elements (row 8 s + lane / 8, 16-byte chunk lane % 8)
    // of each group s of 8 rows, and their scale words
    v4u ac[AR > 0 ? AR / 8 : 1];
    uint32_t aw[AR > 0 ? AR / 8 : 1];
    // AR == 0: the tiles' scale words and, unless the activation codes are staged in LDS
    // (AS > 0), 16 activation code bytes per stage and tile
    v4u al[AR > 0 || AS > 0 ? 1 : MT][kStages];
    uint32_t swa[kStages][AR > 0 ? 1 : MT];
};

// Pin a chunk's registers at this point: the empty asm "modifies" them, so nothing computed
// from them (e.g. a scale pair) can be hoisted into an earlier step, where it would make the
// compiler wait for that chunk's loads.
template <int NT, int MT, int AR, int AS>
__device__ __forceinline__ void pin(Regs<NT, MT, AR, AS>& R) {
#pragma unroll
    for (int j = 0; j < kStages; ++j) {
#pragma unroll
        for (int u = 0; u < NT; ++u) __asm__ volatile("" : "+v"(R.swb[j][u]));
    }
    if constexpr (AR > 0) {
#pragma unroll
        for (int s = 0; s < AR / 8; ++s) __asm__ volatile("" : "+v"(R.ac[s]), "+v"(R.aw[s]));
    } else {
#pragma unroll
        for (int j = 0; j < kStages; ++j) {
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                __asm__ volatile("" : "+v"(R.swa[j][t]));
                if constexpr (AS == 0) __asm__ volatile("" : "+v"(R.al[t][j]));
            }
        }
    }
}

// Vector-memory instructions issue() makes per chunk (for the vmcnt waits): direct-to-LDS
// loads (weight rows, staged activation rows) and loads into registers (scale words,
// activation codes).
template <int NT, int AS>
constexpr int lds_loads_per_chunk() {
    return 4 * NT + AS / 8;
}
template <int MT, int AR, int AS>
constexpr int reg_loads_per_chunk() {
    return kStages + (AR > 0 ? 2 * (AR / 8) : kStages + (AS > 0 ? 0 : MT * kStages));
}

__device__ __forceinline__ v2h bcast(_Float16 x) { return v2h{x, x}; }

// WV: waves per workgroup, each taking every WV-th K chunk.
// NT: 32-row weight tiles per workgroup (1 or 2).
// MT: 32-row activation tiles (M <= 32 MT).
// AR: activation rows decoded once per chunk into LDS (8 or 16, >= M, MT = 1), or 0: the
// activation fragments are decoded in registers.
// D: chunks in flight per wave (LDS weight buffers).
// AS (AR = 0): activation rows (32 MT) whose codes are staged in LDS with the weight rows by
// whole-line loads, or 0: each lane loads its own 16-byte code pieces.
template <int OUT, int BIAS, int WV, int NT, int MT, int AR, int D, int AS>
__device__ __forceinline__ void skinny_tile(const Args& p) {
    static_assert(AR == 0 || (MT == 1 && AR % 8 == 0 && AR <= 16), "decoded activation: 8 or 16 rows");
    static_assert(AS == 0 || (AR == 0 && AS == 32 * MT), "staged activation codes: whole tiles");
    static_assert(16 % WV == 0, "each wave stores 16 / WV accumulator registers");
    static_assert(NT <= 2 && MT <= 2, "scale words of at most two tiles per load");
    constexpr int WR = 32 * NT;                                   // weight rows of the workgroup
    constexpr int WB = (WR + AS) * kCb;                           // one staged chunk (weight, activation)
    constexpr int WST = D * WB + (AR > 0 ? AR * kApitch : 0);     // LDS per wave
    constexpr int ZERO = AR > 0 ? kApitch : 0;                    // the zero activation row
    constexpr int RED = WV * NT * MT * 16 * 64 * 4;
    constexpr int LDS = WV * WST + ZERO > RED ? WV * WST + ZERO : RED;
    // a step's wait: chunk i's register loads and the later chunks' direct-to-LDS loads
    // may stay in flight (see the step below)
    constexpr int VM = reg_loads_per_chunk<MT, AR, AS>() + (D - 1) * lds_loads_per_chunk<NT, AS>();
    static_assert(VM < 64, "vmcnt range");
    __shared__ __attribute__((aligned(1024))) uint8_t lds[LDS];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h = lane >> 5, r = lane & 31;
    const int n0 = xcd_group(blockIdx.x, gridDim.x) * WR;
    const int Kb = p.K / 2;  // code bytes per row

    const __amdgpu_buffer_rsrc_t rb =
        buffer_rsrc(p.b + static_cast<int64_t>(n0) * Kb, static_cast<uint32_t>(min(WR, p.N - n0)) * Kb);
    __amdgpu_buffer_rsrc_t ra[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t)
        ra[t] = buffer_rsrc(p.a + static_cast<int64_t>(32 * t) * Kb,
                            static_cast<uint32_t>(max(0, min(32, p.M - 32 * t))) * Kb);
    const __amdgpu_buffer_rsrc_t ras = buffer_rsrc(p.a, static_cast<uint32_t>(max(0, min(AS, p.M))) * Kb);
    const __amdgpu_buffer_rsrc_t rsb = buffer_rsrc(p.sb, static_cast<uint32_t>(p.sb_rows) * p.ncb * 4);
    const __amdgpu_buffer_rsrc_t rsa = buffer_rsrc(p.sa, static_cast<uint32_t>(p.sa_rows) * p.ncb * 4);
    // Scale word of row r of the workgroup's first weight tile in word column c: swizzled
    // offset ((row/128 * ncb + c) * 32 + row%32) * 16 + ((row%128)/32) * 4; the second tile's
    // word follows it (n0 is a multiple of 64 when NT = 2).  Activation row i (< 128):
    // (i%32) * 16 + (i/32) * 4.
    const uint32_t sb_row = weight_word_offset(n0, r, p.ncb);
    const int NC = (Kb + kCb - 1) / kCb;

    uint8_t* wbuf = lds + wave * WST;           // this wave's D weight buffers
    uint8_t* actf = wbuf + D * WB;              // its decoded activation rows (AR > 0)
    uint8_t* zrow = lds + WV * WST;             // zero row shared by the workgroup (AR > 0)
    if constexpr (AR > 0) {
        for (int i = threadIdx.x; i < kApitch / 4; i += 64 * WV) reinterpret_cast<uint32_t*>(zrow)[i] = 0u;
        __syncthreads();
    }

    // (the lambdas are forced inline: an outlined step would keep R in scratch memory)
    auto issue = [&](int c, uint8_t* buf, Regs<NT, MT, AR, AS>& R) __attribute__((always_inline)) {
        const int b0 = c * kCb;  // first code byte of the chunk
        // the direct-to-LDS loads first; the empty asm keeps the register loads after them
        stage_rows<4 * NT, kAuxNontemporal>(rb, buf, Kb, b0, lane);
        if constexpr (AS > 0) stage_rows<AS / 8, 0>(ras, buf + WR * kCb, Kb, b0, lane);
        __asm__ volatile("" ::: "memory");
#pragma unroll
        for (int j = 0; j < kStages; ++j) {
            const int col = c * kStages + j;
            const uint32_t co = col < p.ncb ? static_cast<uint32_t>(col * 512) : 0x80000000u;
            load_words<NT>(rsb, sb_row + co, R.swb[j]);
        }
        if constexpr (AR > 0) {
            const int q = lane & 7;
#pragma unroll
            for (int s = 0; s < AR / 8; ++s) {
                const int row = 8 * s + (lane >> 3);
                const int k = b0 + 16 * q;
                R.ac[s] = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(
                                                      ra[0], k < Kb ? static_cast<uint32_t>(row * Kb + k) : 0x80000000u,
                                                      0, 0));
                const int col = c * kStages + (q >> 1);
                R.aw[s] = __builtin_amdgcn_raw_buffer_load_b32(
                    rsa, col < p.ncb ? static_cast<uint32_t>(col * 512 + row * 16) : 0x80000000u, 0, 0);
            }
        } else {
#pragma unroll
            for (int j = 0; j < kStages; ++j) {
                const int col = c * kStages + j;
                const uint32_t co = col < p.ncb ? static_cast<uint32_t>(col * 512) : 0x80000000u;
                load_words<MT>(rsa, r * 16 + co, R.swa[j]);
            }
            if constexpr (AS == 0) {
#pragma unroll
                for (int t = 0; t < MT; ++t)
#pragma unroll
                    for (int j = 0; j < kStages; ++j) {
                        const int k = b0 + 32 * j + 16 * h;
                        R.al[t][j] = __builtin_bit_cast(
                            v4u, __builtin_amdgcn_raw_buffer_load_b128(
                                     ra[t], k < Kb ? static_cast<uint32_t>(r * Kb + k) : 0x80000000u, 0, 0));
                    }
            }
        }
    };

    v16f acc[NT][MT];
#pragma unroll
    for (int u = 0; u < NT; ++u)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[u][t] = v16f{};

    // lane's fragment addresses: weight row r of tile u, logical chunk 2 j + h; decoded
    // activation row r (or the zero row), bytes 128 j + 64 h + 16 kk
    const uint32_t wrow = static_cast<uint32_t>(r * kCb);
    const uint32_t wsw = swz8(r);
    const uint8_t* abase = (AR > 0 && r < AR ? actf + r * kApitch : zrow) + 64 * h;

    auto compute = [&](const uint8_t* buf, const Regs<NT, MT, AR, AS>& R) __attribute__((always_inline)) {
        if constexpr (AR > 0) {
            // decode the chunk's activation rows: lane's 32 elements are blocks 2 q, 2 q + 1 of
            // the chunk (bytes 2 (q % 2), +1 of word q / 2)
            const int q = lane & 7;
#pragma unroll
            for (int s = 0; s < AR / 8; ++s) {
                const v2h sp = scale_pair(R.aw[s], 16 * (q & 1));
                uint8_t* dst = actf + (8 * s + (lane >> 3)) * kApitch + q * 64;
                *reinterpret_cast<v8h*>(dst) = decode8(R.ac[s][0], bcast(sp[0]));
                *reinterpret_cast<v8h*>(dst + 16) = decode8(R.ac[s][1], bcast(sp[0]));
                *reinterpret_cast<v8h*>(dst + 32) = decode8(R.ac[s][2], bcast(sp[1]));
                *reinterpret_cast<v8h*>(dst + 48) = decode8(R.ac[s][3], bcast(sp[1]));
            }
        }
#pragma unroll
        for (int j = 0; j < kStages; ++j) {
            v4u cb[NT];
            v2h pb[NT];
#pragma unroll
            for (int u = 0; u < NT; ++u) {
                cb[u] = *reinterpret_cast<const v4u*>(buf + u * 32 * kCb + wrow + (((2 * j + h) ^ wsw) << 4));
                pb[u] = scale_pair(R.swb[j][u], 16 * h);
            }
            v2h pa[MT];
            v4u ca[MT];
            if constexpr (AR == 0) {
#pragma unroll
                for (int t = 0; t < MT; ++t) {
                    pa[t] = scale_pair(R.swa[j][t], 16 * h);
                    ca[t] = AS > 0 ? staged_chunk(buf + WR * kCb, 32 * t + r, 2 * j + h) : R.al[t][j];
                }
            }
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                v8h da[MT];
#pragma unroll
                for (int t = 0; t < MT; ++t) {
                    if constexpr (AR > 0) da[t] = *reinterpret_cast<const v8h*>(abase + 128 * j + 16 * kk);
                    else da[t] = decode8(ca[t][kk], bcast(pa[t][kk >> 1]));
                }
#pragma unroll
                for (int u = 0; u < NT; ++u) {
                    const v8h db = decode8(cb[u][kk], bcast(pb[u][kk >> 1]));
#pragma unroll
                    for (int t = 0; t < MT; ++t)
                        acc[u][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(db, da[t], acc[u][t], 0, 0, 0);
                }
            }
        }
    };

    // This wave's chunks c_i = wave + i WV, i < n.  Chunks i .. i + D - 1 are in flight while
    // chunk i is computed (buffer i % D, registers R[i % D]).  Every step issues the loads
    // of chunk i + D, past the end too (they read nothing and write zeros to its own
    // buffer).  The wait before chunk i counts only loads that are issued after chunk i's
    // direct-to-LDS loads on every path: chunk i's own register loads (read right after the
    // wait, and kept behind its LDS loads by issue()) and the D - 1 later chunks' LDS loads,
    // which write memory and so stay where they are.  The later chunks' register loads do
    // not count: the compiler may move them into the blocks that read them, so on a path
    // that never reads them (the prologue straight to the last steps) they are not issued.
    // The compiler waits for the registers itself.
    const int n = wave < NC ? (NC - wave + WV - 1) / WV : 0;
    Regs<NT, MT, AR, AS> R[D];
    nv::for_each_index([&](auto d_c) {
        constexpr int d = decltype(d_c)::value;
        issue(wave + d * WV, wbuf + d * WB, R[d]);
    }, std::make_integer_sequence<int, D>{});
    auto step = [&](int i, auto d_c) __attribute__((always_inline)) {
        constexpr int d = decltype(d_c)::value;
        wait<waitcnt_vm_lgkm0(VM)>();  // chunk i's LDS rows have landed
        pin(R[d]);
        compute(wbuf + d * WB, R[d]);
        // the loads of chunk i + D overwrite this buffer: every read of it is done
        wait<waitcnt_vm_lgkm0(63)>();
        issue(wave + (i + D) * WV, wbuf + d * WB, R[d]);
    };
    int i = 0;
    for (; i + D - 1 < n; i += D)
        nv::for_each_index([&](auto d_c) { step(i + decltype(d_c)::value, d_c); }, std::make_integer_sequence<int, D>{});
    // the last n % D chunks
    nv::for_each_index([&](auto d_c) {
        if (i + decltype(d_c)::value < n) step(i + decltype(d_c)::value, d_c);
    }, std::make_integer_sequence<int, D - 1>{});
    wait<waitcnt_vm_lgkm0(0)>();  // the trailing loads write LDS, which is reused below

    // the K partials of each 32 x 32 tile meet in LDS (reusing the staging area); wave w adds
    // and stores registers RPW w .. RPW w + RPW - 1 (columns n0 + 32 u + 8 (v / 4) + 4 h + v % 4
    // of row m = 32 t + r)
    constexpr int RPW = 16 / WV;
    __syncthreads();
    float (*red)[NT][MT][16][64] = reinterpret_cast<float (*)[NT][MT][16][64]>(lds);
#pragma unroll
    for (int u = 0; u < NT; ++u)
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int v = 0; v < 16; ++v) red[wave][u][t][v][lane] = acc[u][t][v];
    __syncthreads();
    const float alpha = p.alpha[0];
    // registers v .. v + G - 1 of a group hold consecutive columns (G <= 4, v % G == 0)
    constexpr int G = RPW < 4 ? RPW : 4;
    const int v0 = RPW * wave;
#pragma unroll
    for (int u = 0; u < NT; ++u) {
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const int m = 32 * t + r;
#pragma unroll
            for (int g0 = 0; g0 < RPW; g0 += G) {
                const int vb = v0 + g0;
                const int n = n0 + 32 * u + 8 * (vb >> 2) + 4 * h + (vb & 3);
                float v[G];
#pragma unroll
                for (int e = 0; e < G; ++e) {
                    float s = 0.0f;
#pragma unroll
                    for (int w = 0; w < WV; ++w) s += red[w][u][t][vb + e][lane];
                    v[e] = s * alpha + (n + e < p.N ? nv::bias_at<BIAS>(p.bias, n + e) : 0.0f);
                }
                if (m >= p.M) continue;
                const int64_t idx = static_cast<int64_t>(m) * p.N + n;
                if constexpr (G == 4) {
                    if (n + 3 < p.N && (p.N & 3) == 0) {
                        nv::store4<OUT>(p.out, idx, v);
                        continue;
                    }
                }
#pragma unroll
                for (int e = 0; e < G; ++e)
                    if (n + e < p.N) nv::store1<OUT>(p.out, idx + e, v[e]);
            }
        }
    }
}

template <int OUT, int BIAS, int WV, int NT, int MT, int AR, int D, int AS>
__global__ __launch_bounds__(64 * WV) void gemm_skinny_kernel(Args p) {
    skinny_tile<OUT, BIAS, WV, NT, MT, AR, D, AS>(p);
}

// Eight waves share the SIMDs in pairs (the LDS holds one such workgroup per CU), so each
// wave may have half the register file; left to that budget the compiler spends all 256
// registers (the four-wave form needs fewer than 100) and spills some.  A limit of 128
// keeps it in registers: the attribute's count is doubled on this architecture (one file
// holds a wave's vector and accumulation registers), so 64 asks for 128.
template <int OUT, int BIAS, int NT, int MT, int AR, int D, int AS>
__global__ __launch_bounds__(512) __attribute__((amdgpu_num_vgpr(64))) void gemm_skinny_kernel8(Args p) {
    skinny_tile<OUT, BIAS, 8, NT, MT, AR, D, AS>(p);
}

}  // namespace nvsk
}  // namespace ckh

using namespace ckh;

namespace {

// Activations of at most kNvSkinnyMaxM rows take the skinny kernel (nvsk::gemm_skinny_kernel).
constexpr int kNvSkinnyMaxM = 64;

// Split-K: a grid of at most 128 tiles (half the CUs) with at least kNvMinSplitK groups of
// 256 elements runs S K ranges of every tile (each of ks groups, the last one fewer, at
// least kNvMinSplitGroups) as S times as many workgroups, at most 256, which write fp32
// partial tiles to the caller's workspace; a second launch adds them.  A group costs about
// 4 us of MFMA time per tile and a partial tile's round trip about as much as one group.
// Ranges of an odd number of groups end mid-pair (measured against ranges rounded up to an
// even count, same process: M = 256, N = 13824, K = 5120, four ranges of 5 instead of 6, 6,
// 6, 2: 48.7 against 53.8 us; M = 300, N = 2000, K = 4160 35.0 against 39.6; M = 2048, N =
// 4096, K = 5376 84.6 against 90.1).  Minimum range lengths of 2, 3, 6 and 8 groups
// measured no better than 4 over six shapes (2: 300 x 2000 x 4160 30.9 against 34.4 us but
// 256 x 3072 x 12288 36.5 against 35.4; 8: up to 40% slower).  Grids of at most
// kNvHalfSplitTiles tiles split their 256 x 128 column halves instead (twice the units,
// half the ranges: less partial traffic per unit of work), also in ranges of at least
// kNvMinSplitGroups (3 measured 2-4% faster on three shapes but 16% slower on 512 x 3072 x
// 3072; 2 slower on four of five).  Grids of 65-128 tiles split whole tiles only into three
// ranges or more and from kNvMinSplitKFull groups on; otherwise they run as one round of
// whole-K half tiles, which write no partials (same process, split against half tiles: two
// ranges, 256 x 32768 x 5120 86.0 against 73.8 us, 2048 x 4096 x 5376 86.6 against 74.4,
// 384 x 12288 x 6144 74.3 against 71.8; three ranges of 4 groups, 256 x 18432 x 3072 44.6
// against 39.8; three of 11 and 7, 256 x 18432 x 8192 77.4 against 90.9 and 512 x 8704 x
// 5120 55.7 against 59.5).
constexpr int kNvSlots = 256;
constexpr int kNvMinSplitK = 8;
constexpr int kNvMinSplitKFull = 16;
constexpr int kNvMinSplitGroups = 4;
constexpr int kNvHalfSplitTiles = 64;
// A last round of at most this many tiles runs them as half tiles (see ckh_scaled_mm_nvfp4).
constexpr int kNvHalfTail = kNvSlots / 2;

struct NvSplitPlan {
    int S = 1;   // K ranges (1: no split)
    int ks = 0;  // groups per range
    int nw = 4;  // 4: full tiles, 2: half tiles
};

NvSplitPlan nv_split_plan(int64_t M, int64_t N, int64_t K) {
    NvSplitPlan sp;
    if (M <= kNvSkinnyMaxM) return sp;
    const int tiles = static_cast<int>(cdiv(M, nv::BM) * cdiv(N, nv::BN));
    const int NG = static_cast<int>(cdiv(K / 2, nv::GKB));
    const bool half = tiles <= kNvHalfSplitTiles;
    if (tiles > kNvSlots / 2 || NG < (half ? kNvMinSplitK : kNvMinSplitKFull)) return sp;
    const int units = half ? 2 * tiles : tiles;
    const int S = min(kNvSlots / units, NG / kNvMinSplitGroups);
    if (S < (half ? 2 : 3)) return sp;
    sp.ks = static_cast<int>(cdiv(NG, S));
    sp.S = static_cast<int>(cdiv(NG, sp.ks));
    sp.nw = half ? 2 : 4;
    return sp;
}

// one partial tile (or two partial half tiles) per tile and K range
int64_t nv_split_workspace_bytes(int64_t M, int64_t N, int64_t K) {
    const NvSplitPlan sp = nv_split_plan(M, N, K);
    if (sp.S < 2) return 0;
    return cdiv(M, nv::BM) * cdiv(N, nv::BN) * sp.S * static_cast<int64_t>(nv::kPartTile) * 4;
}

template <int NW>
void launch_nv_split(const nv::Args& p, int out_code, int bias_code, bool has_bias, hipStream_t st) {
    const int units = p.tiles_m * p.tiles_n * (4 / NW);
    hipLaunchKernelGGL(nv::gemm_split_kernel<NW>, dim3(static_cast<unsigned>(units * p.splits)), dim3(nv::NT), 0, st,
                       p);
    const dim3 g2(static_cast<unsigned>(units * (nv::BM * 64 * NW / 4 / 256)));
#define LAUNCH(O, B) hipLaunchKernelGGL((nv::gemm_reduce_kernel<O, B, NW>), g2, dim3(256), 0, st, p)
#define BY_BIAS(O)                                         \
    do {                                                   \
        if (!has_bias) LAUNCH(O, -1);                      \
        else if (bias_code == CKH_F32) LAUNCH(O, CKH_F32); \
        else if (bias_code == CKH_F16) LAUNCH(O, CKH_F16); \
        else LAUNCH(O, CKH_BF16);                          \
    } while (0)
    if (out_code == CKH_BF16) BY_BIAS(CKH_BF16);
    else if (out_code == CKH_F16) BY_BIAS(CKH_F16);
    else BY_BIAS(CKH_F32);
#undef BY_BIAS
#undef LAUNCH
}

int launch_nv_skinny(const nv::Args& q, int out_code, int bias_code, bool has_bias, hipStream_t st) {
    nvsk::Args p{};
    p.a = q.a; p.b = q.b; p.sa = q.sa; p.sb = q.sb; p.alpha = q.alpha; p.bias = q.bias; p.out = q.out;
    p.M = q.M; p.N = q.N; p.K = q.K; p.ncb = q.ncb; p.sa_rows = q.sa_rows; p.sb_rows = q.sb_rows;
    // Per activation size: waves per workgroup, weight tiles per workgroup, activation tiles,
    // activation rows decoded to LDS, chunks in flight per wave.  Measured (graph-timed, K = 5120,
    // N = 13824): M = 1 12.5 us, M = 8 13.0 us, M = 16 16.0 us; 8 waves, 3 chunks in flight, or
    // activation fragments decoded in registers were 10-20% slower at M <= 8.  With fewer than
    // 256 workgroups (N < 8192) 8 waves per workgroup pay instead (same process, against 4):
    // M = 16, N = 5120, K = 13824 18.8 against 22.1 us; M = 16, N = 3072, K = 12288 17.0
    // against 20.0; M = 1, N = 5120, K = 5120 8.1 against 8.8 (for the staged 32-row
    // activation 8 waves measured 9-11% slower).  For M > 16 two
    // weight tiles per workgroup halve the activation decoding per weight byte, which pays
    // while N gives enough workgroups (M = 64: N = 13824 19.4 against 24.8 us with one tile;
    // N = 5120, K = 13824 27.5 against 32.4 us with two).  With one tile (N < 8192) the
    // activation codes are staged in LDS by whole-line loads rather than loaded by each lane
    // (M = 32, N = 5120, K = 5120 10.0 against 10.4 us; M = 64, N = 3072, K = 12288 22.3
    // against 24.7; M = 64, N = 5120, K = 13824 25.1 against 26.6); with two tiles that
    // measured no better (19.6 against 19.5 us at M = 64, N = 13824).
    const bool two = q.N >= 8192;
#define LAUNCH(O, B, WV, NT, MT, AR, D, AS)                                                       \
    do {                                                                                          \
        if constexpr (WV == 8)                                                                    \
            hipLaunchKernelGGL((nvsk::gemm_skinny_kernel8<O, B, NT, MT, AR, D, AS>),              \
                               dim3(static_cast<unsigned>(cdiv(q.N, 32 * NT))), dim3(512), 0, st, p); \
        else                                                                                      \
            hipLaunchKernelGGL((nvsk::gemm_skinny_kernel<O, B, WV, NT, MT, AR, D, AS>),           \
                               dim3(static_cast<unsigned>(cdiv(q.N, 32 * NT))), dim3(64 * WV), 0, st, p); \
    } while (0)
#define BY_MT(O, B)                                                \
    do {                                                           \
        if (p.M <= 8 && two) LAUNCH(O, B, 4, 1, 1, 8, 2, 0);       \
        else if (p.M <= 8) LAUNCH(O, B, 8, 1, 1, 8, 2, 0);         \
        else if (p.M <= 16 && two) LAUNCH(O, B, 4, 1, 1, 16, 2, 0); \
        else if (p.M <= 16) LAUNCH(O, B, 8, 1, 1, 16, 2, 0);       \
        else if (p.M <= 32 && two) LAUNCH(O, B, 4, 2, 1, 0, 2, 0); \
        else if (p.M <= 32) LAUNCH(O, B, 4, 1, 1, 0, 2, 32);       \
        else if (two) LAUNCH(O, B, 4, 2, 2, 0, 2, 0);              \
        else LAUNCH(O, B, 4, 1, 2, 0, 2, 64);                      \
    } while (0)
#define BY_BIAS(O)                                          \
    do {                                                    \
        if (!has_bias) BY_MT(O, -1);                        \
        else if (bias_code == CKH_F32) BY_MT(O, CKH_F32);   \
        else if (bias_code == CKH_F16) BY_MT(O, CKH_F16);   \
        else BY_MT(O, CKH_BF16);                            \
    } while (0)
    if (out_code == CKH_BF16) BY_BIAS(CKH_BF16);
    else if (out_code == CKH_F16) BY_BIAS(CKH_F16);
    else BY_BIAS(CKH_F32);
#undef BY_BIAS
#undef BY_MT
#undef LAUNCH
    return check_launch("scaled_mm_nvfp4");
}

}  // namespace

extern "C" int64_t ckh_scaled_mm_nvfp4_workspace_bytes(int64_t M, int64_t N, int64_t K) {
    if (M <= 0 || N <= 0 || K <= 0 || M >= (1ll << 30) || N >= (1ll << 30) || K >= (1ll << 31)) return 0;
    return nv_split_workspace_bytes(M, N, K);
}

extern "C" int ckh_scaled_mm_nvfp4(const void* a, const void* b, const void* sa, const void* sb, const void* alpha,
                                   const void* bias, void* out, int64_t M, int64_t N, int64_t K, int out_code,
                                   int bias_code, void* workspace, int64_t workspace_bytes, uintptr_t stream) {
    CKH_REQUIRE(a && b && sa && sb && alpha && out, "scaled_mm_nvfp4: null pointer");
    CKH_REQUIRE(M >= 0 && N >= 0 && K > 0, "scaled_mm_nvfp4: sizes must be M, N >= 0 and K > 0");
    CKH_REQUIRE(K % 32 == 0, "scaled_mm_nvfp4: K (%lld) must be a multiple of 32", (long long)K);
    CKH_REQUIRE(M * (K / 2) < (1ll << 31) && N * (K / 2) < (1ll << 31) && M < (1ll << 30) && N < (1ll << 30),
                "scaled_mm_nvfp4: operand larger than 2 GiB");
    CKH_REQUIRE(out_code == CKH_F32 || out_code == CKH_F16 || out_code == CKH_BF16,
                "scaled_mm_nvfp4: unsupported output dtype code %d", out_code);
    CKH_REQUIRE(!bias || bias_code == CKH_F32 || bias_code == CKH_F16 || bias_code == CKH_BF16,
                "scaled_mm_nvfp4: unsupported bias dtype code %d", bias_code);
    CKH_REQUIRE(aligned(a, 16) && aligned(b, 16) && aligned(sa, 16) && aligned(sb, 16) && aligned(out, 16) &&
                    aligned(alpha, 4) && (!workspace || aligned(workspace, 16)),
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
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (p.M <= kNvSkinnyMaxM) return launch_nv_skinny(p, out_code, bias_code, bias != nullptr, st);
    const NvSplitPlan sp = nv_split_plan(M, N, K);
    if (sp.S > 1 && workspace && workspace_bytes >= nv_split_workspace_bytes(M, N, K)) {
        p.splits = sp.S;
        p.ks = sp.ks;
        p.part = static_cast<float*>(workspace);
        if (sp.nw == 2) launch_nv_split<2>(p, out_code, bias_code, bias != nullptr, st);
        else launch_nv_split<4>(p, out_code, bias_code, bias != nullptr, st);
        return check_launch("scaled_mm_nvfp4");
    }
    // The tiles run one per CU in rounds.  When the last round would be at most half full,
    // its tiles run as twice as many 256 x 128 half tiles in the same grid (a grid of one
    // round with no split-K workspace runs all of its tiles so).
    const int tiles = p.tiles_m * p.tiles_n;
    const int tail = tiles > kNvSlots ? tiles % kNvSlots : tiles;
    p.n_half = (tail > 0 && tail <= kNvHalfTail) ? tail : 0;
    p.n_full = tiles - p.n_half;
    dim3 grid(static_cast<unsigned>(p.n_full + 2 * p.n_half));
#define LAUNCH(O, B) hipLaunchKernelGGL((nv::gemm_kernel<O, B>), grid, dim3(nv::NT), 0, st, p)
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
    return check_launch("scaled_mm_nvfp4");
}
