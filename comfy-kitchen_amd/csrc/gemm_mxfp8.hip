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
// Rows past M / N, columns past K and stages past the end lie outside the buffer
// descriptors' ranges and load as zeros, so every stage runs the same branch-free code.
//
// Pipeline: at stage t (after its barrier) the fragments of t are already in
// registers; the LDS reads of stage t+1's fragments overlap stage t's 16 MFMAs.
// Activation fragments are double-buffered (each is used by all of a stage's MFMA rows);
// each weight fragment is read into its own registers right after its last MFMA of the
// stage; with 32 fewer live VGPRs the block-scaled kernels do not spill (2 VGPRs still
// do in some per-tensor instantiations).  Each wave loads its own E8M0 scale words (16
// bytes per operand and 128-wide K block) straight into registers two stages ahead.
// Global data moves in pairs of stages through registers: one load
// instruction brings whole 128-byte lines (both stages' halves of 8 rows).  An even
// stage t writes the staged weight pair t+2, t+3 to LDS and loads the activation pair
// t+4, t+5; the odd stage after it writes that pair and loads the next weight pair, so
// each load has one stage (~1000 MFMA cycles) to arrive.  (Keeping each operand's
// registers for two stages instead makes both staged sets loop-carried, and the
// compiler then drains every load each stage.)  Register staging rather than direct-to-LDS
// loads because each buffer_load ... lds instruction holds up the issuing wave's MFMA
// stream for ~22 cycles on gfx950, while plain loads and ds_writes hide under the MFMAs.
// Each barrier waits for LDS traffic only; the compiler's vmcnt waits guard the staged
// registers.
//
// LDS rows are 64 bytes; logical 16-byte chunk c of row r lives at chunk
// c ^ ((r >> 1) & 3) ^ ((r >> 3) & 1), which makes a 32-row fragment read (one chunk
// of 32 consecutive rows) conflict-free for both 32- and 64-bank LDS layouts.
// Workgroups are dispatched round-robin over the 8 XCDs; the tile index is remapped
// so each XCD walks a contiguous range of tiles in grouped order (grouped_tile), so the
// tiles an XCD runs at once share few operand panels in its L2.  Tiles run one per CU
// in rounds; when the last round would be at most half full, its tiles run as 256 x 128
// half tiles (2 MFMA columns per wave, 8-slot stages) on twice as many CUs, in the same
// grid after the full tiles.
#include <type_traits>
#include <utility>

#include "ckh_common.h"
#include "skinny.h"

namespace ckh {
namespace mx {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

constexpr int BM = 256, BN = 256, BK = 64, NT = 256;
constexpr int TILE = 256 * BK;  // bytes of one operand tile per stage (16 KB)
// One stage buffer: weight tile, activation tile, room for the epilogue's 64-row output
// slab, and 64 bytes of padding.  LDS banks repeat every 128 bytes; a staged store writes
// row r of buffers s and s + 1 from 8 neighbouring lanes (64 bytes each), which the
// padding puts in opposite halves of the bank cycle (measured conflict-free; without it
// every store conflicts 2-way).
constexpr int BUF = 2 * TILE + 2048 + 64;
// Bytes of one staged 16-bit output row (512 + 16 pad, rows 16-byte aligned).  The 8-byte
// staging writes of this layout are where the kernel's LDS bank conflicts come from (0.88 of
// 0.93 M conflict cycles per C4 call); 16-byte writes after a v_permlane32_swap of the
// lane halves remove them but measured the same time (bit-identical), so the conflicts are
// off the critical path and the simpler writes stay.
constexpr int EPI_ROW = 528;
static_assert(64 * EPI_ROW <= BUF, "an output slab must fit one stage buffer");

// s_waitcnt immediates (gfx9 encoding): vmcnt in [3:0] and [15:14], expcnt [6:4],
// lgkmcnt [11:8].  expcnt is left unconstrained (7).
constexpr int waitcnt_vm_lgkm0(int vm) { return (vm & 15) | (7 << 4) | ((vm >> 4) << 14); }
constexpr int WAIT_LGKM0 = waitcnt_vm_lgkm0(63);  // LDS only; global loads stay in flight

// Workgroup barrier after an explicit s_waitcnt.  __syncthreads() would add a release
// fence, i.e. vmcnt(0), draining the prefetched stages; here each wave has already
// waited for exactly what the barrier must publish (its LDS writes and reads), LDS is
// one coherent array per CU, and the empty asm statements keep the compiler from
// moving memory operations across.
template <int WAITCNT>
__device__ __forceinline__ void stage_barrier() {
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(WAITCNT);
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
}

// fn(integral_constant<int, K>) for each K in order
template <typename Fn, int... K>
__device__ __forceinline__ void for_each_index(Fn&& fn, std::integer_sequence<int, K...>) {
    (fn(std::integral_constant<int, K>{}), ...);
}

__device__ __forceinline__ int swz(int row) { return ((row >> 1) & 3) ^ ((row >> 3) & 1); }

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
    int tiles_m, tiles_n;  // 256 x 256 tile grid
    int n_full;            // workgroups [0, n_full) compute full tiles 0 .. n_full-1 (linear, grouped order)
    int n_half;            // workgroups n_full + 2 i, +1 compute the two column halves of tile n_full + i
    int n_pref;            // the workgroups after those read the weight ahead (prefetch_weight)
    // per-tensor mode only: the two fp32 tensor scales (device), applied in the epilogue
    const float* tsa;
    const float* tsb;
    // split-K mode (gemm_split_kernel): workgroup L * splits + s computes stages
    // [s * ks, min((s + 1) * ks, KT)) of tile L and writes its fp32 partial tile to part
    int splits, ks;
    float* part;
};

// fp32 values of one partial tile in the workspace (256 x 256)
constexpr int kPartTile = BM * BN;

// Register-staged loads of one operand for a pair of stages (s, s + 1), i.e. K bytes
// [k0, k0 + 128) of the tile's 256 (or 128) rows.  Wave w, load j (0..7, or 0..3)
// covers rows R = 64 w + 8 j .. +7 (R = 32 w + 8 j for 128 rows): lane i fetches 16-byte chunk c = i % 8 of row R + i / 8, so each
// 8 lanes read one whole 128-byte line (with all CUs loading, half-line requests reach
// only ~70% of the L2 throughput of whole lines).  Chunks 0..3 go to stage s's buffer,
// 4..7 to stage s + 1's, at physical chunk (c % 4) ^ swz(row); swz(row + 8) = swz(row) ^ 1.
struct Loader {
    __amdgpu_buffer_rsrc_t rs;
    uint32_t voff;      // lane's global byte offset for j = 0, k0 = 0
    uint32_t rowstep;   // 8 * K: global distance between consecutive loads j
    int cbyte;          // 16 * c
    uint32_t lds_even;  // lane's LDS offset within a stage tile for j = 0 (even j adds 512 j)
    uint32_t lds_odd;   // the same for odd j (before adding 512 j)
    bool hi;            // chunk belongs to stage s + 1
};

__device__ __forceinline__ Loader make_loader(const uint8_t* tile_base, int valid_rows, int K, int wave, int lane,
                                             int rows_per_wave = 64) {
    Loader L;
    L.rs = buffer_rsrc(tile_base, static_cast<uint32_t>(max(valid_rows, 0)) * K);
    const int row = rows_per_wave * wave + (lane >> 3), c = lane & 7;
    L.cbyte = c << 4;
    L.voff = static_cast<uint32_t>(row * K + L.cbyte);
    L.rowstep = 8u * K;
    L.lds_even = static_cast<uint32_t>(row * BK + (((c & 3) ^ swz(row)) << 4));
    L.lds_odd = static_cast<uint32_t>(row * BK + (((c & 3) ^ swz(row) ^ 1) << 4));
    L.hi = c >= 4;
    return L;
}

// Offset added to a lane's global address for the pair at k0: past K the lane reads
// zeros from outside the descriptor's range.
__device__ __forceinline__ uint32_t pair_add(const Loader& L, int k0, int K) {
    return (k0 + L.cbyte < K) ? static_cast<uint32_t>(k0) : 0x80000000u;
}

template <int J>
__device__ __forceinline__ void load_piece(const Loader& L, v4u (&x)[8], uint32_t add) {
    x[J] = __builtin_amdgcn_raw_buffer_load_b128(L.rs, L.voff + J * L.rowstep + add, 0, 0);
}

template <int J>
__device__ __forceinline__ void store_piece(const Loader& L, const v4u (&x)[8], uint8_t* tx, uint8_t* ty) {
    uint8_t* t = L.hi ? ty : tx;
    *reinterpret_cast<v4u*>(t + ((J & 1) ? L.lds_odd : L.lds_even) + 512 * J) = x[J];
}

template <int... J>
__device__ __forceinline__ void load_pair(const Loader& L, v4u (&x)[8], int k0, int K,
                                          std::integer_sequence<int, J...>) {
    const uint32_t add = pair_add(L, k0, K);
    (load_piece<J>(L, x, add), ...);
}

template <int NP = 8>
__device__ __forceinline__ void load_pair(const Loader& L, v4u (&x)[8], int k0, int K) {
    load_pair(L, x, k0, K, std::make_integer_sequence<int, NP>{});
}

template <int... J>
__device__ __forceinline__ void store_pair(const Loader& L, const v4u (&x)[8], uint8_t* tx, uint8_t* ty,
                                           std::integer_sequence<int, J...>) {
    (store_piece<J>(L, x, tx, ty), ...);
}

template <int NP = 8>
__device__ __forceinline__ void store_pair(const Loader& L, const v4u (&x)[8], uint8_t* tx, uint8_t* ty) {
    store_pair(L, x, tx, ty, std::make_integer_sequence<int, NP>{});
}

// activation fragments of one stage (MFMA operand 1); the weight fragments (operand 0)
// live in one v8i[NW] array
struct Frags {
    v8i a[4];
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

template <int NW>
__device__ __forceinline__ void read_frags(Frags& F, v8i (&FB)[NW], const uint8_t* stage_buf, const FragAddr& fb,
                                           const FragAddr& fa) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        if (t < NW) FB[t] = read_frag(stage_buf + t * 32 * BK, fb);
        F.a[t] = read_frag(stage_buf + TILE + t * 32 * BK, fa);
    }
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

// Two floats to two 16-bit values (RNE) in one v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32, low
// half first.  `opaque` keeps an fp32 product or sum feeding the convert from being fused
// into a single-rounding mixed-precision instruction.
template <int OUT, bool HIDE>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    if constexpr (HIDE) {
        a = opaque(a);
        b = opaque(b);
    }
    const v2f v = {a, b};
    if constexpr (OUT == CKH_BF16) return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, v2bf));
    else return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, v2h));
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

// UNIT: per-tensor FP8 (TensorCoreFP8Layout): no block scales (every MFMA scale byte is
// E8M0 127 = 1.0) and out = tsa * tsb * (A B^T) + bias.
// NW: 32-column MFMA tiles per wave along n: 4 for 256 x 256 workgroup tiles, 2 for the
// 256 x 128 half tiles that finish a grid whose last round would leave most CUs idle.
// bid: the workgroup's index among the workgroups of its kind (full or half tiles).
//
// Stage buffers 0, 1 and 2, 3 live in two arrays.  Every stage reads fragments from one
// array and writes staged data into the other, so the compiler knows they never alias
// and may interleave the two freely; within an array, per-lane addresses of different
// buffers differ only by immediates.
template <int OUT, int BIAS, bool UNIT, int NW, bool SPLIT = false>
__device__ __forceinline__ void gemm_tile(const Args& p, int bid, uint8_t* lds01, uint8_t* lds23) {
    constexpr int TBN = 64 * NW;  // tile width along n
    constexpr int PB = TBN / 32;  // staged weight loads per lane per pair of stages
    constexpr int SLOTS = 4 * NW;  // MFMAs per wave per stage

    // Workgroups are dispatched round-robin over the 8 XCDs; full tiles are remapped so
    // each XCD walks a contiguous range of tiles (in grouped order).  Half tiles give
    // tile L's two column halves to consecutive workgroups.  Split-K workgroups take tile
    // (or half tile) bid / splits, K range bid % splits.
    const int KT = (p.K + BK - 1) / BK;
    const int split = SPLIT ? bid % p.splits : 0;
    if (SPLIT) bid /= p.splits;
    else if (NW == 4 && (p.n_full & 7) == 0) bid = (bid & 7) * (p.n_full >> 3) + (bid >> 3);
    // this workgroup's stages [t0, t1) (t0 a multiple of 4), the bytes of K they cover and
    // the 128-wide scale blocks: loads past them read zeros
    const int t0 = SPLIT ? split * p.ks : 0;
    const int t1 = SPLIT ? min(t0 + p.ks, KT) : KT;
    const int kend = SPLIT ? min(t1 * BK, p.K) : p.K;
    const int pend = SPLIT ? min(p.ncb, (t1 + 1) / 2) : p.ncb;
    const int L = (NW == 4) ? bid : (SPLIT ? 0 : p.n_full) + (bid >> 1);
    int tm, tn;
    grouped_tile(L, p.tiles_m, p.tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN + (NW == 4 ? 0 : (bid & 1) * TBN);
    if (n0 >= p.N) return;  // a half tile wholly past N (uniform over the workgroup)

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
    const int wm = wave & 1, wn = wave >> 1;
    const int half = lane >> 5, r32 = lane & 31;

    const Loader LB = make_loader(p.b + static_cast<int64_t>(n0) * p.K, min(TBN, p.N - n0), p.K, wave, lane, TBN / 4);
    const Loader LA = make_loader(p.a + static_cast<int64_t>(m0) * p.K, min(BM, p.M - m0), p.K, wave, lane);
    constexpr bool DS = !UNIT;  // block scales (per-tensor mode: E8M0 127 throughout)
    const __amdgpu_buffer_rsrc_t rssb = buffer_rsrc(p.sb, static_cast<uint32_t>(p.sb_rows) * p.ncb * 4);
    const __amdgpu_buffer_rsrc_t rssa = buffer_rsrc(p.sa, static_cast<uint32_t>(p.sa_rows) * p.ncb * 4);
    const FragAddr fab = make_frag_addr(wn * 32 * NW, lane);
    const FragAddr faa = make_frag_addr(wm * 128, lane);

    v16f acc[NW][4];
#pragma unroll
    for (int i = 0; i < NW; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = v16f{};

    auto buf = [&](auto b_c) -> uint8_t* {
        constexpr int B = decltype(b_c)::value & 3;
        return (B < 2 ? lds01 : lds23) + (B & 1) * BUF;
    };
    // Register staging: a pair of stages of one operand at a time.
    v4u SB[8], SA[8];
    auto load_b = [&](int s) { load_pair<PB>(LB, SB, s * BK, kend); };
    // Scale words: a lane's 4 words for its wave's 4 32-row tiles of an operand and one
    // 128-wide K block (pair of stages) are 16 contiguous bytes of the swizzled tensor, at
    // chunk ((row128 / 128) * ncb + pair) * 512 + r32 * 16 for the tiles' 128-row block
    // row128.  Each wave loads its own into registers two stages ahead of use (staging them
    // through LDS with the operands, shared by the workgroup, measured 1.3-1.8% slower on
    // every shape, bit-identical).
    const uint32_t dsb_off = static_cast<uint32_t>(((n0 >> 7) + (NW == 4 ? wn : 0)) * p.ncb * 512 + r32 * 16);
    const uint32_t dsa_off = static_cast<uint32_t>(((m0 >> 7) + wm) * p.ncb * 512 + r32 * 16);
    v4u DWB, DWA;  // words of the next pair not yet consumed
    auto load_dscales = [&](int pair) {
        const uint32_t po = pair < pend ? static_cast<uint32_t>(pair * 512) : 0x80000000u;
        DWB = __builtin_amdgcn_raw_buffer_load_b128(rssb, dsb_off + po, 0, 0);
        DWA = __builtin_amdgcn_raw_buffer_load_b128(rssa, dsa_off + po, 0, 0);
    };
    auto load_a = [&](int s) { load_pair(LA, SA, s * BK, kend); };
    auto store_a = [&](auto x_c, auto y_c) { store_pair(LA, SA, buf(x_c) + TILE, buf(y_c) + TILE); };
    // this lane's 4 scale words (tiles t = 0..3) of each operand for a stage, shifted so
    // byte 0 / byte 2 are the lane-half's scales of the even / odd 64-wide stage
    const int hs = 8 * half;
    // the first of this wave's weight tiles in its 16-byte scale chunk (half tiles: 2 of 4)
    const int sbt = NW == 4 ? 0 : 2 * wn;
    uint32_t scb[4], sca[4];
    Frags F0, F1;
    v8i FB[NW];

    // Stage t held in buffer B = t % 4 (compile-time): activation fragments F and the
    // weight fragments FB (stage t) are in registers; read stage t+1 into G and, each
    // after its last MFMA here (slot 4i + 3), into FB[i].  A pair of stages (s, s+1), s
    // even, moves in two halves: the activation pair is loaded at stage s-4 and written to
    // LDS at s-3, the weight pair loaded at s-3 and written at s-2.  Each write targets
    // buffers whose previous stages were read before the current barrier.  An odd stage
    // shifts the next pair's scale words into place (slot SLOTS - 4) and loads the pair
    // after it (slot SLOTS - 3).
    //
    // The stage is scheduled by hand in 16 slots, one MFMA each (sched_barrier keeps
    // the order): the next stage's fragments in the order the next stage uses them, and
    // in slots 0..7 one staged chunk written to LDS followed by the load that refills its
    // registers, which therefore has a whole stage to arrive.  (Double-
    // buffering the weight fragments too gave the same times, bit-identical, but spilled
    // 2-3 VGPRs.)
    auto stage = [&](auto b_c, int t, Frags& F, Frags& G) {
        constexpr int B = decltype(b_c)::value;
        constexpr bool EVEN = (B & 1) == 0;
        constexpr int OPSEL = EVEN ? 0 : 2;
        using Next = std::integral_constant<int, (B + 1) & 3>;
        using P2 = std::integral_constant<int, (B + 2) & 3>;
        using P3 = std::integral_constant<int, (B + 3) & 3>;
        stage_barrier<WAIT_LGKM0>();
        const uint8_t* nx = buf(Next{});
        uint8_t* wx = EVEN ? buf(P2{}) : buf(P3{}) + TILE;
        uint8_t* wy = EVEN ? buf(P3{}) : buf(b_c) + TILE;
        const uint32_t add = EVEN ? pair_add(LA, (t + 4) * BK, kend) : pair_add(LB, (t + 3) * BK, kend);
        uint32_t nb[4], na[4];
        if constexpr (UNIT) {
#pragma unroll
            for (int u = 0; u < 4; ++u) nb[u] = na[u] = 0x7f7f7f7fu;
        } else if constexpr (EVEN) {  // the next stage is in this stage's pair: same words
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                nb[u] = scb[u];
                na[u] = sca[u];
            }
        }
        auto slot = [&](auto k_c) {
            constexpr int k = decltype(k_c)::value;
            constexpr int i = k / 4, j = k % 4;
            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(FB[i], F.a[j], acc[i][j], 0, 0, OPSEL, scb[i],
                                                                        OPSEL, sca[j]);
            if constexpr (k == 1) G.a[0] = read_frag(nx + TILE, faa);
            if constexpr (k >= 3 && k <= 5) G.a[k - 2] = read_frag(nx + TILE + (k - 2) * 32 * BK, faa);
            if constexpr (k % 4 == 3 && k / 4 < NW) FB[k / 4] = read_frag(nx + (k / 4) * 32 * BK, fab);
            if constexpr (k < 8) {
                if constexpr (EVEN) {
                    if constexpr (k < PB) store_piece<k>(LB, SB, wx, wy);
                    load_piece<k>(LA, SA, add);
                } else {
                    store_piece<k>(LA, SA, wx, wy);
                    if constexpr (k < PB) load_piece<k>(LB, SB, add);
                }
            }
            if constexpr (k == SLOTS - 4 && DS && !EVEN) {
                // the next stage opens pair (t + 1) / 2: its words, then pair (t + 1) / 2 + 1's load
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    nb[u] = (NW == 4 ? DWB[u] : (sbt ? DWB[2 + (u & 1)] : DWB[u & 1])) >> hs;
                    na[u] = DWA[u] >> hs;
                }
            }
            if constexpr (k == SLOTS - 3 && DS && !EVEN) load_dscales((t + 1) / 2 + 1);
            __builtin_amdgcn_sched_barrier(0);
        };
        for_each_index(slot, std::make_integer_sequence<int, SLOTS>{});
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            scb[u] = nb[u];
            sca[u] = na[u];
        }
    };

    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
    using B2 = std::integral_constant<int, 2>;
    using B3 = std::integral_constant<int, 3>;

    // prologue: stages 0..3 resident except the weight half of 2, 3 (staged in SB for
    // stage 0 to write), stage 0 read.  All four pairs are loaded before the first LDS
    // write, so the prologue waits out one memory latency rather than two.
    {
        v4u XA[8], XB[8];
        load_a(t0);
        load_pair<PB>(LB, XB, t0 * BK, kend);
        if constexpr (DS) load_dscales(t0 / 2);
        load_pair(LA, XA, (t0 + 2) * BK, kend);
        load_b(t0 + 2);
        store_a(B0{}, B1{});
        store_pair<PB>(LB, XB, buf(B0{}), buf(B1{}));
        store_pair(LA, XA, buf(B2{}) + TILE, buf(B3{}) + TILE);
    }
    stage_barrier<WAIT_LGKM0>();
    read_frags(F0, FB, lds01, fab, faa);
    if constexpr (DS) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            scb[u] = (NW == 4 ? DWB[u] : (sbt ? DWB[2 + (u & 1)] : DWB[u & 1])) >> hs;
            sca[u] = DWA[u] >> hs;
        }
        load_dscales(t0 / 2 + 1);
    } else {
#pragma unroll
        for (int u = 0; u < 4; ++u) scb[u] = sca[u] = 0x7f7f7f7fu;
    }

    // stages in groups of 4 (buffer index = stage % 4); stages past K are all zeros
    for (int t = t0; t < t1; t += 4) {
        stage(B0{}, t, F0, F1);
        stage(B1{}, t + 1, F1, F0);
        stage(B2{}, t + 2, F0, F1);
        stage(B3{}, t + 3, F1, F0);
    }
    if constexpr (SPLIT) {
        __builtin_amdgcn_s_waitcnt(0);  // prefetches past this range (zeros) have landed
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
    // the epilogue reuses the LDS buffers
    __syncthreads();

    // Epilogue: lane holds out[m][n..n+3] for m = r32-th row of activation tile j and
    // n = 8*g + 4*half (+0..3) of weight tile i.
    const float alpha = UNIT ? p.tsa[0] * p.tsb[0] : 1.0f;
    // With neither a tensor scale nor a bias the accumulator is the output value.
    constexpr bool ARITH = UNIT || BIAS >= 0;
    auto value = [&](float a, int n) {
        if constexpr (UNIT) a *= alpha;
        if constexpr (BIAS >= 0) a += n < p.N ? bias_at<BIAS>(p.bias, n) : 0.0f;
        return a;
    };
    if constexpr (OUT != CKH_F32) {
        // 16-bit output: stage the tile in LDS as 256 rows of 512 bytes, the 64-row slab
        // q in buffer q, converting two values per instruction.  Then each wave stores
        // whole rows of its slab, 16 bytes per lane: two 512-byte rows per instruction
        // (NW = 4) or four 256-byte rows (NW = 2).
        auto slab = [&](int q) -> uint8_t* { return (q < 2 ? lds01 : lds23) + (q & 1) * BUF; };
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint8_t* rowp = slab(wm * 2 + (j >> 1)) + ((j & 1) * 32 + r32) * EPI_ROW;
#pragma unroll
            for (int i = 0; i < NW; ++i) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int nl = wn * 32 * NW + i * 32 + 8 * g + 4 * half;
                    const int n = n0 + nl;
                    const v16f& a = acc[i][j];
                    const uint32_t w0 = pack2<OUT, ARITH>(value(a[4 * g], n), value(a[4 * g + 1], n + 1));
                    const uint32_t w1 = pack2<OUT, ARITH>(value(a[4 * g + 2], n + 2), value(a[4 * g + 3], n + 3));
                    *reinterpret_cast<uint2*>(rowp + nl * 2) = make_uint2(w0, w1);
                }
            }
        }
        __syncthreads();
        constexpr int LPR = TBN / 8;  // lanes per output row, 16 bytes (8 values) each
        constexpr int RPI = 64 / LPR;  // rows per store instruction
        const int lr = lane % LPR, lrow = lane / LPR;
        const uint8_t* src = slab(wave) + lrow * EPI_ROW + lr * 16;
        const int n = n0 + 8 * lr;
        const bool vec = (p.N & 7) == 0 && n + 8 <= p.N;
        uint16_t* orow = static_cast<uint16_t*>(p.out) + static_cast<int64_t>(m0 + wave * 64 + lrow) * p.N + n;
        const int rows = min(64, p.M - (m0 + wave * 64)) - lrow;
#pragma unroll 8
        for (int rl = 0; rl < 64; rl += RPI) {
            const v4u d = *reinterpret_cast<const v4u*>(src + rl * EPI_ROW);
            if (rl >= rows) break;
            uint16_t* o = orow + static_cast<int64_t>(rl) * p.N;
            if (vec) {
                __builtin_nontemporal_store(d, reinterpret_cast<v4u*>(o));
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    if (n + e < p.N) o[e] = static_cast<uint16_t>(d[e >> 1] >> (16 * (e & 1)));
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
                for (int g = 0; g < 4; ++g) {
                    const int n = n0 + wn * 32 * NW + i * 32 + 8 * g + 4 * half;
                    float v[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = value(acc[i][j][4 * g + e], n + e);
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

// A grid of one round (fewer tiles than CUs) leaves CUs idle, and its tiles wait on HBM
// for every weight byte: the weight streams through once, and a tile's loads run only a
// few stages ahead of its MFMAs.  Workgroups on the idle CUs (one per CU: the tile
// kernel's LDS fills a CU) therefore read the weight ahead of the tiles, so that the
// tiles' own loads find it in the memory-side cache (256 MB): first the weight's scale
// words, then its codes from K byte kPrefSkip on (the tiles' prologue loads the bytes
// before that itself) in pieces of kPiece bytes, one K range of every row, then the next
// range, in the order the tiles consume them.  A wave loads a piece with one 16-byte load
// per lane (8 whole lines per instruction) and discards it; the waves of the n_pref
// workgroups take kPrefBatch consecutive pieces each in turn, so that together they
// sweep the ranges in K order.  The loads stay inside the operands (a piece past the end
// of a row reads nothing).  Measured (graph-timed, rotated operands, same process):
// 256 x 18432 x 3072 31.8 -> 30.3 us, 512 x 18432 x 3072 41.3 -> 39.6, 1024 x 3072 x 3072
// 21.7 -> 21.5.  The gain is bounded by what the cache gives at all: with the weight
// read completely beforehand by a separate grid, the 256-row GEMM still took 27.9 us
// against 32.0 cold and 22.4 with the same operands as the call before.  Loading one
// dword per 64-byte sector instead, or 256-byte K ranges, measured the same or slower.
constexpr int kPiece = 1024;
constexpr int kPrefSkip = 4 * BK;
constexpr int kPrefBatch = 32;

template <bool UNIT>
__device__ __forceinline__ void prefetch_weight(const Args& p, int w) {
    const int lane = threadIdx.x & 63;
    const uint32_t gw = static_cast<uint32_t>(w) * (NT / 64) + (threadIdx.x >> 6);  // wave among all
    const uint32_t stride = static_cast<uint32_t>(p.n_pref) * (NT / 64) * kPrefBatch;
    v4u x = {0u, 0u, 0u, 0u};
    if constexpr (!UNIT) {
        const uint32_t sb_bytes = static_cast<uint32_t>(p.sb_rows) * p.ncb * 4;
        const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(p.sb, sb_bytes);
        const uint32_t pieces = (sb_bytes + kPiece - 1) / kPiece;
        for (uint32_t base = gw * kPrefBatch; base < pieces; base += stride) {
            v4u v[kPrefBatch];
#pragma unroll
            for (int j = 0; j < kPrefBatch; ++j)
                v[j] = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(
                                                   rs, (base + j) * kPiece + lane * 16u, 0, 0));
#pragma unroll
            for (int j = 0; j < kPrefBatch; ++j) x ^= v[j];
        }
    }
    const uint32_t Kb = static_cast<uint32_t>(p.K);  // code bytes per weight row
    const uint32_t N = static_cast<uint32_t>(p.N);
    const uint32_t ranges = Kb > kPrefSkip ? (Kb - kPrefSkip + kPiece - 1) / kPiece : 0;
    const uint32_t pieces = ranges * N;
    const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(p.b, N * Kb);
    for (uint32_t base = gw * kPrefBatch; base < pieces; base += stride) {
        v4u v[kPrefBatch];
#pragma unroll
        for (int j = 0; j < kPrefBatch; ++j) {
            const uint32_t q = base + j;
            const uint32_t c = q / N, n = q - c * N;
            const uint32_t k = kPrefSkip + c * kPiece + lane * 16u;
            const uint32_t off = q < pieces && k < Kb ? n * Kb + k : 0x80000000u;
            v[j] = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(rb, off, 0, 0));
        }
#pragma unroll
        for (int j = 0; j < kPrefBatch; ++j) x ^= v[j];
    }
    __asm__ volatile("" ::"v"(x));  // the loads are kept; their values are not used
}

// One grid runs both kinds of workgroup: the full tiles first, then (when the last
// round of full tiles would be at most half full) that round's tiles as half tiles.
// The dispatcher starts half-tile workgroups on CUs as their last full tile ends, so
// the tail overlaps the uneven end of the previous round instead of waiting for a
// second launch.  A grid of one round ends with the weight-prefetch workgroups.
template <int OUT, int BIAS, bool UNIT>
__global__ __launch_bounds__(NT) void gemm_kernel(Args p) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds01[2 * BUF];
    __shared__ __attribute__((aligned(1024))) uint8_t lds23[2 * BUF];
    const int b = blockIdx.x;
    if (b < p.n_full) gemm_tile<OUT, BIAS, UNIT, 4>(p, b, lds01, lds23);
    else if (b < p.n_full + 2 * p.n_half) gemm_tile<OUT, BIAS, UNIT, 2>(p, b - p.n_full, lds01, lds23);
    else prefetch_weight<UNIT>(p, b - p.n_full - 2 * p.n_half);
}

// Split-K, first launch: each workgroup one K range of one 256 x 256 tile (NW = 4) or
// 256 x 128 half tile (NW = 2), partial sums to the workspace (no output, bias or tensor
// scale here).
template <bool UNIT, int NW>
__global__ __launch_bounds__(NT) void gemm_split_kernel(Args p) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds01[2 * BUF];
    __shared__ __attribute__((aligned(1024))) uint8_t lds23[2 * BUF];
    gemm_tile<CKH_F32, -1, UNIT, NW, true>(p, blockIdx.x, lds01, lds23);
}

// Split-K, second launch: thread q adds float4 q % U of unit q / U (U = 4096 NW float4 of a
// tile or half tile) over the splits in split order (the sum does not depend on which
// workgroup finished first), then applies the tensor scale and bias and stores
// out[m][n .. n + 3] (the register mapping of the tile kernel's epilogue).
template <int OUT, int BIAS, bool UNIT, int NW>
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
    const int L = NW == 4 ? U : U >> 1;
    const float4* src = reinterpret_cast<const float4*>(p.part) + static_cast<int64_t>(U) * p.splits * kUnit + rest;
    float4 v = src[0];
    for (int s = 1; s < p.splits; ++s) {
        const float4 w = src[static_cast<int64_t>(s) * kUnit];
        v.x += w.x;
        v.y += w.y;
        v.z += w.z;
        v.w += w.w;
    }
    int tm, tn;
    grouped_tile(L, p.tiles_m, p.tiles_n, tm, tn);
    const int m = tm * BM + (wave & 1) * 128 + j * 32 + (lane & 31);
    const int n = tn * BN + (NW == 4 ? 0 : (U & 1) * 128) + (wave >> 1) * 32 * NW + i * 32 + 8 * g + 4 * (lane >> 5);
    if (m >= p.M || n >= p.N) return;
    float o[4] = {v.x, v.y, v.z, v.w};
    const float alpha = UNIT ? p.tsa[0] * p.tsb[0] : 1.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        if constexpr (UNIT) o[e] *= alpha;
        if constexpr (BIAS >= 0) o[e] += n + e < p.N ? bias_at<BIAS>(p.bias, n + e) : 0.0f;
        // kept from being fused with the narrowing into one mixed-precision rounding
        if constexpr (UNIT || BIAS >= 0) o[e] = opaque(o[e]);
    }
    const int64_t idx = static_cast<int64_t>(m) * p.N + n;
    if (n + 3 < p.N && (p.N & 3) == 0) {
        store4<OUT>(p.out, idx, o);
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (n + e < p.N) store1<OUT>(p.out, idx + e, o[e]);
    }
}

}  // namespace mx

// ------------------------------------------------------------ skinny activations
// GEMMs with few activation rows (M <= 64: batch-size-1 modulation and projection linears)
// read every weight byte once and do little arithmetic per byte, so they are bound by HBM
// bandwidth on the weight, not by the matrix cores.  The 256 x 256 tiles above would give
// such a GEMM only N / 256 workgroups.  Here a workgroup owns 32 or 64 weight rows and all of
// K (N / 32 = 576 workgroups for N = 18432, several resident per CU), and its waves split
// the K steps in chunks of 4 (256 bytes of each row), chunk c to wave c % WV.  A wave stages
// its chunk of weight rows (and, for M <= 16, of activation rows) in its own LDS area with
// direct-to-LDS loads in which every instruction reads 8 whole 128-byte lines, then reads
// its MFMA fragments from there: loading the fragments straight from memory asks for 32-byte
// pieces of 32 lines per instruction and measured 18.9 against 15.1 us at M = 1,
// N = 18432, K = 3072.  The weight loads are nontemporal; the activation, read by every
// workgroup, stays cached.  At the end the K partials meet in LDS and each wave adds and
// stores its share of the tile.  Operand layout and scale selection are the tile kernel's
// (lane l = 32 h + r: row r, bytes k0 + 16 h and k0 + 32 + 16 h; scale word shifted by
// 8 h, opsel 0 / 2 for even / odd steps of a 128-wide scale block).  Rows past M or N and
// bytes past K lie outside the buffer descriptors and load as zeros.
namespace mxsk {

using namespace ckh::sk;

constexpr int kSkRow = 256;              // staged bytes per row and chunk
constexpr int kSkCpr = kSkRow / 16;      // 16-byte chunks per staged row
constexpr int kSkRpl = 1024 / kSkRow;    // staged rows per direct-to-LDS load (1 KB)

// Staging layout: row r of a chunk is 256 bytes; logical 16-byte chunk c sits at physical
// chunk c ^ (r % 16).  LDS banks repeat every 256 bytes, so a fragment read (16 lanes = 16
// consecutive rows, one logical chunk) hits 16 distinct 16-byte bank groups.
__device__ __forceinline__ uint32_t sk_swz(int r) { return static_cast<uint32_t>(r & (kSkCpr - 1)); }

// Direct-to-LDS whole-line loads of rows [0, NQ * kSkRpl) of a chunk: load q writes 1 KB,
// rows kSkRpl q .. , lane i to row kSkRpl q + i / kSkCpr, physical chunk i % kSkCpr, so each
// load reads 8 whole 128-byte lines.  Bytes past K, and rows outside the descriptor, arrive
// as zeros.
template <int NQ, int AUX>
__device__ __forceinline__ void stage_rows256(__amdgpu_buffer_rsrc_t rs, uint8_t* dst, int K, int kbase, int lane) {
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        const int row = kSkRpl * q + lane / kSkCpr;
        const int k = kbase + static_cast<int>(((lane % kSkCpr) ^ sk_swz(row)) << 4);
        const uint32_t off = k < K ? static_cast<uint32_t>(row * K + k) : 0x80000000u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(dst + q * 1024), 16, off, 0, 0, AUX);
    }
}

// Logical 16-byte chunk c of staged row r.
__device__ __forceinline__ v4u staged_chunk256(const uint8_t* st, int r, int c) {
    return *reinterpret_cast<const v4u*>(st + r * kSkRow + ((static_cast<uint32_t>(c) ^ sk_swz(r)) << 4));
}

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kSkChunk = kSkRow / 64;    // K steps (64 bytes) per wave per chunk: two scale words

struct Args {
    const uint8_t* a;
    const uint8_t* b;
    const uint8_t* sa;
    const uint8_t* sb;
    const void* bias;
    void* out;
    int M, N, K;
    int ncb;               // scale column blocks: ceil(K/32/4)
    int sa_rows, sb_rows;  // padded scale rows (multiples of 128)
    const float* tsa;      // per-tensor mode: the two fp32 tensor scales (device)
    const float* tsb;
};

// This lane's MFMA operand for step j of the staged chunk: row r, logical chunks 4 j + h and
// 4 j + 2 + h (bytes k0 + 16 h and k0 + 32 + 16 h of the step).
__device__ __forceinline__ v8i staged_frag(const uint8_t* st, int r, int h, int j) {
    const v4u x = staged_chunk256(st, r, 4 * j + h);
    const v4u y = staged_chunk256(st, r, 4 * j + 2 + h);
    return v8i{(int)x[0], (int)x[1], (int)x[2], (int)x[3], (int)y[0], (int)y[1], (int)y[2], (int)y[3]};
}

// Offset of this lane's piece p (0, 1) of the step at k0 for a direct (unstaged) operand
// load: bytes k0 + 32 p + 16 h of its row; past K it reads zeros.
__device__ __forceinline__ uint32_t piece_off(uint32_t row_off, int k0, int p, int h, int K) {
    const int k = k0 + 32 * p + 16 * h;
    return k < K ? row_off + static_cast<uint32_t>(k) : 0x80000000u;
}

// One chunk's register-held operands: scale words and (unstaged activation) fragments.
template <int MT, int NT>
struct SkRegs {
    uint32_t swb[NT][kSkChunk / 2], swa[MT][kSkChunk / 2];
    v4u al[MT][kSkChunk][2];
};

// WV: waves per workgroup, each taking every WV-th K chunk.
// NT: 32-row weight tiles per workgroup (1 or 2); each activation fragment feeds NT MFMAs.
// MT: 32-row activation tiles (M <= 32 MT).
// AR: activation rows staged through LDS like the weight (8 or 16, >= M, one M-tile), or 0:
// the activation's fragments are loaded straight into registers.
template <int OUT, int BIAS, bool UNIT, int WV, int NT, int MT, int AR>
__global__ __launch_bounds__(64 * WV) void gemm_skinny_kernel(Args p) {
    static_assert(AR == 0 || (AR % kSkRpl == 0 && AR <= 32 * MT && AR > 32 * (MT - 1)),
                  "staged activation rows: within the MT tiles, a multiple of the rows per load");
    static_assert(16 % WV == 0, "each wave stores 16 / WV accumulator registers");
    constexpr int WR = 32 * NT;                   // weight rows of the workgroup
    constexpr int WST = (WR + AR) * kSkRow;       // staged bytes per wave
    constexpr int RED = WV * NT * MT * 16 * 64 * 4;
    constexpr int LDS = WV * WST > RED ? WV * WST : RED;
    __shared__ __attribute__((aligned(1024))) uint8_t stage[LDS];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h = lane >> 5, r = lane & 31;
    const int n0 = xcd_group(blockIdx.x, gridDim.x) * WR;

    const __amdgpu_buffer_rsrc_t rb =
        buffer_rsrc(p.b + static_cast<int64_t>(n0) * p.K, static_cast<uint32_t>(min(WR, p.N - n0)) * p.K);
    __amdgpu_buffer_rsrc_t ra[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t)
        ra[t] = buffer_rsrc(p.a + static_cast<int64_t>(32 * t) * p.K,
                            static_cast<uint32_t>(max(0, min(32, p.M - 32 * t))) * p.K);
    // the staged activation rows (AR > 0): rows past M read as zeros
    const __amdgpu_buffer_rsrc_t ras = buffer_rsrc(p.a, static_cast<uint32_t>(max(0, min(AR, p.M))) * p.K);
    // per-tensor mode: no scale tensors (zero-sized descriptors, never loaded)
    const __amdgpu_buffer_rsrc_t rsb = buffer_rsrc(p.sb, UNIT ? 0u : static_cast<uint32_t>(p.sb_rows) * p.ncb * 4);
    const __amdgpu_buffer_rsrc_t rsa = buffer_rsrc(p.sa, UNIT ? 0u : static_cast<uint32_t>(p.sa_rows) * p.ncb * 4);
    const uint32_t row_off = static_cast<uint32_t>(r * p.K);
    // scale word of row r (of the 32-row group) in column block cb: swizzled offset
    // ((row/128 * ncb + cb) * 32 + row%32) * 16 + ((row%128)/32) * 4
    uint32_t sb_row[NT];
#pragma unroll
    for (int u = 0; u < NT; ++u) {
        const int nu = n0 + 32 * u;
        sb_row[u] = static_cast<uint32_t>((nu >> 7) * p.ncb * 512 + r * 16 + ((nu & 127) >> 5) * 4);
    }
    const uint32_t sa_row = static_cast<uint32_t>(r * 16);  // activation rows 32 t + r: + 4 t
    const int KT = (p.K + 63) / 64;
    const int NC = (KT + kSkChunk - 1) / kSkChunk;

    // issue chunk c's loads: weight (and staged activation) rows to LDS buffer `buf`, scale
    // words and unstaged activation fragments to R
    uint8_t* stb = stage + wave * WST;  // this wave's staged rows: weight, then activation
    auto issue = [&](int c, SkRegs<MT, NT>& R) {
        const int s0 = c * kSkChunk;
        // the weight is read once (nontemporal); the activation, which every workgroup
        // reads, stays cached
        stage_rows256<WR / kSkRpl, kAuxNontemporal>(rb, stb, p.K, s0 * 64, lane);
        if constexpr (AR > 0) stage_rows256<AR / kSkRpl, 0>(ras, stb + WR * kSkRow, p.K, s0 * 64, lane);
        if constexpr (!UNIT) {
#pragma unroll
            for (int u = 0; u < kSkChunk / 2; ++u) {
                const int cb = (s0 >> 1) + u;  // 128-wide scale block of steps s0 + 2u, s0 + 2u + 1
                const uint32_t cbo = cb < p.ncb ? static_cast<uint32_t>(cb * 512) : 0x80000000u;
#pragma unroll
                for (int v = 0; v < NT; ++v)
                    R.swb[v][u] = __builtin_amdgcn_raw_buffer_load_b32(rsb, sb_row[v] + cbo, 0, 0);
#pragma unroll
                for (int t = 0; t < MT; ++t)
                    R.swa[t][u] = __builtin_amdgcn_raw_buffer_load_b32(rsa, sa_row + t * 4 + cbo, 0, 0);
            }
        }
        if constexpr (AR == 0) {
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int j = 0; j < kSkChunk; ++j)
#pragma unroll
                    for (int q = 0; q < 2; ++q)
                        R.al[t][j][q] = __builtin_amdgcn_raw_buffer_load_b128(
                            ra[t], piece_off(row_off, (s0 + j) * 64, q, h, p.K), 0, 0);
        }
    };

    v16f acc[NT][MT];
#pragma unroll
    for (int u = 0; u < NT; ++u)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[u][t] = v16f{};

    // this wave's chunks: c = wave, wave + WV, ...; the staged rows are the wave's own, so
    // waiting for its own loads is enough (no barrier)
    SkRegs<MT, NT> cur;
    if (wave < NC) issue(wave, cur);
    for (int c = wave; c < NC; c += WV) {
        __asm__ volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
        __asm__ volatile("" ::: "memory");
#pragma unroll
        for (int j = 0; j < kSkChunk; ++j) {
            v8i fa[MT];
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                if constexpr (AR > 0) {
                    const int row = 32 * t + r;
                    fa[t] = staged_frag(stb + WR * kSkRow, row < AR ? row : 0, h, j);
                    if (row >= AR) fa[t] = v8i{};
                } else {
                    const v4u u = cur.al[t][j][0], w = cur.al[t][j][1];
                    fa[t] = v8i{(int)u[0], (int)u[1], (int)u[2], (int)u[3], (int)w[0], (int)w[1], (int)w[2], (int)w[3]};
                }
            }
#pragma unroll
            for (int u = 0; u < NT; ++u) {
                const v8i fb = staged_frag(stb + u * 32 * kSkRow, r, h, j);
                const uint32_t sbv = UNIT ? 0x7f7f7f7fu : cur.swb[u][j >> 1] >> (8 * h);
#pragma unroll
                for (int t = 0; t < MT; ++t) {
                    const uint32_t sav = UNIT ? 0x7f7f7f7fu : cur.swa[t][j >> 1] >> (8 * h);
                    if (j & 1)
                        acc[u][t] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fb, fa[t], acc[u][t], 0, 0, 2, sbv, 2, sav);
                    else
                        acc[u][t] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fb, fa[t], acc[u][t], 0, 0, 0, sbv, 0, sav);
                }
            }
        }
        // the next chunk's loads overwrite the staged rows: every fragment read is done
        __asm__ volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(63));
        __asm__ volatile("" ::: "memory");
        if (c + WV < NC) issue(c + WV, cur);
    }

    // the K partials of each 32 x 32 tile meet in LDS (reusing the staging area); wave w adds
    // and stores registers RPW w .. RPW w + RPW - 1 (columns n0 + 32 u + 8 (v / 4) + 4 h + v % 4
    // of row m = 32 t + r)
    constexpr int RPW = 16 / WV;
    __syncthreads();
    float (*red)[NT][MT][16][64] = reinterpret_cast<float (*)[NT][MT][16][64]>(stage);
#pragma unroll
    for (int u = 0; u < NT; ++u)
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int v = 0; v < 16; ++v) red[wave][u][t][v][lane] = acc[u][t][v];
    __syncthreads();
    const float alpha = UNIT ? p.tsa[0] * p.tsb[0] : 1.0f;
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
                    if constexpr (UNIT) s *= alpha;
                    if constexpr (BIAS >= 0) s += n + e < p.N ? load1<BIAS>(p.bias, n + e) : 0.0f;
                    // kept from being fused with the narrowing into one mixed-precision rounding
                    v[e] = (UNIT || BIAS >= 0) ? opaque(s) : s;
                }
                if (m >= p.M) continue;
                const int64_t idx = static_cast<int64_t>(m) * p.N + n;
                if constexpr (G == 4) {
                    if (n + 3 < p.N && (p.N & 3) == 0) {
                        mx::store4<OUT>(p.out, idx, v);
                        continue;
                    }
                }
#pragma unroll
                for (int e = 0; e < G; ++e)
                    if (n + e < p.N) mx::store1<OUT>(p.out, idx + e, v[e]);
            }
        }
    }
}

}  // namespace mxsk
}  // namespace ckh

using namespace ckh;

namespace {

// Workgroups that can hold a 256 x 256 tile at once: one per CU.
constexpr int kGemmSlots = 256;

template <bool UNIT>
void launch_grid(const mx::Args& p, unsigned wgs, int out_code, int bias_code, bool has_bias, hipStream_t st) {
#define LAUNCH(O, B) hipLaunchKernelGGL((mx::gemm_kernel<O, B, UNIT>), dim3(wgs), dim3(mx::NT), 0, st, p)
#define BY_BIAS(O)                                                     \
    do {                                                               \
        if (!has_bias) LAUNCH(O, -1);                                  \
        else if (bias_code == CKH_F32) LAUNCH(O, CKH_F32);             \
        else if (bias_code == CKH_F16) LAUNCH(O, CKH_F16);             \
        else LAUNCH(O, CKH_BF16);                                      \
    } while (0)
    if (out_code == CKH_BF16) BY_BIAS(CKH_BF16);
    else if (out_code == CKH_F16) BY_BIAS(CKH_F16);
    else BY_BIAS(CKH_F32);
#undef BY_BIAS
#undef LAUNCH
}

// Activations of at most kSkinnyMaxM rows take the skinny kernel (mxsk::gemm_skinny_kernel).
constexpr int kSkinnyMaxM = 64;

template <bool UNIT>
int launch_skinny(const mx::Args& q, int out_code, int bias_code, bool has_bias, hipStream_t st) {
    mxsk::Args p{};
    p.a = q.a; p.b = q.b; p.sa = q.sa; p.sb = q.sb; p.bias = q.bias; p.out = q.out;
    p.M = q.M; p.N = q.N; p.K = q.K; p.ncb = q.ncb; p.sa_rows = q.sa_rows; p.sb_rows = q.sb_rows;
    p.tsa = q.tsa; p.tsb = q.tsb;
    // per activation size: waves per workgroup, weight tiles per workgroup, activation tiles,
    // staged activation rows (measured on N = 18432, K = 3072: M = 1 12.7 us, M = 16 15.4 us,
    // M = 32 20.5 us, M = 64 26.4 us, the last two with the activation fragments loaded
    // straight into registers).  With 16 activation rows the waves per workgroup
    // follow N: 2 waves when there are at least 256 workgroups (M = 16, N = 18432: 14.6
    // against 15.4 us with 4), 8 when there are fewer than 128 (N = 3072, K = 12288: 16.6
    // against 17.2 us; with 2 waves 25.9 us).  From 17 rows on, staging the activation
    // through LDS too (32 or 64 rows) pays where the workgroups stay small enough in LDS to
    // share CUs (same process, against the register-loaded fragments): M = 32, N = 18432
    // 17.3 against 20.5 us (4 waves, one weight tile); N = 5120, K = 5120 10.8 against 16.5
    // (8 waves); M = 64, N = 18432 21.7 against 26.3 (2 waves, two tiles); N = 5120,
    // K = 13824 29.3 against 47.4 and N = 3072, K = 12288 25.4 against 42.1 (4 waves, one
    // tile); for N from 8192 to 16383 two weight tiles with 32 staged rows (M = 24,
    // N = 13824 17.2 against 17.8) or register-loaded fragments (M = 48: 21.0, staged 64 rows
    // 21.0 with 4 waves, 24.4 with 2).  With 33-64 rows and N from 16384 on the choice
    // follows how many workgroups one round holds (same process): 4 waves and two weight
    // tiles (128 KB of LDS, one workgroup per CU) while N / 64 <= 256 (M = 64, N = 16384,
    // K = 5120 22.6 against 25.7 us; K = 3072 16.0 against 17.8); else 2 waves and one tile
    // (48 KB, three per CU) up to N = 24576 with K <= 4096 (M = 64, N = 18432, K = 3072 20.6
    // against 21.6; M = 40, N = 24576 19.9 against 22.3; at K = 5120 33.8 against 33.3);
    // else 2 waves and two tiles (N = 32768: 25.2 against 29.1 and 34.5).  17-32 rows follow the
    // same rule (same process, against 4 waves and one tile): N = 16384, K = 5120 18.7 against
    // 19.8 us; M = 32, N = 18432, K = 3072 16.4 against 17.3; M = 20, N = 32768 20.2 against 22.0;
    // at K = 12288 4 waves and one tile stay (57.4 against 57.7).  With 4-8 rows and N above
    // 16384, 2 waves rather than 8 (M = 8, N = 18432, K = 3072 13.4 against 14.5 us; N = 24576
    // 14.9 against 15.8; M = 4 13.1 against 13.6; M = 1 and 2 and N = 16384 equal).  The NVFP4
    // skinny kernel's form (128-byte chunks, two in flight per wave) measured slower here, where a
    // chunk costs only a few MFMAs: M = 1 14.5 against 12.9 us, M = 16 15.9 against 15.5, M = 64
    // 29.6 against 26.5 (same process).
#define LAUNCH(O, B, WV, NT, MT, AR)                                                              \
    hipLaunchKernelGGL((mxsk::gemm_skinny_kernel<O, B, UNIT, WV, NT, MT, AR>),                    \
                       dim3(static_cast<unsigned>(cdiv(q.N, 32 * NT))), dim3(64 * WV), 0, st, p)
#define BY_MT(O, B)                                    \
    do {                                               \
        if (p.M <= 8 && p.M >= 4 && p.N > 16384) LAUNCH(O, B, 2, 1, 1, 8); \
        else if (p.M <= 8) LAUNCH(O, B, 8, 1, 1, 8);                   \
        else if (p.M <= 16 && p.N >= 8192) LAUNCH(O, B, 2, 1, 1, 16);  \
        else if (p.M <= 16 && p.N >= 4096) LAUNCH(O, B, 4, 1, 1, 16);  \
        else if (p.M <= 16) LAUNCH(O, B, 8, 1, 1, 16);                 \
        else if (p.M <= 32 && p.N >= 16384 && p.N <= 16384) LAUNCH(O, B, 4, 2, 1, 32); \
        else if (p.M <= 32 && p.N >= 16384 && p.N <= 24576 && p.K <= 4096) LAUNCH(O, B, 2, 1, 1, 32); \
        else if (p.M <= 32 && p.N > 24576) LAUNCH(O, B, 2, 2, 1, 32);   \
        else if (p.M <= 32 && p.N >= 16384) LAUNCH(O, B, 4, 1, 1, 32); \
        else if (p.M <= 32 && p.N >= 8192) LAUNCH(O, B, 4, 2, 1, 32);  \
        else if (p.M <= 32) LAUNCH(O, B, 8, 1, 1, 32);                 \
        else if (p.N >= 16384 && p.N <= 16384) LAUNCH(O, B, 4, 2, 2, 64); \
        else if (p.N >= 16384 && p.N <= 24576 && p.K <= 4096) LAUNCH(O, B, 2, 1, 2, 64); \
        else if (p.N >= 16384) LAUNCH(O, B, 2, 2, 2, 64);              \
        else if (p.N >= 8192) LAUNCH(O, B, 4, 2, 2, 0);                \
        else LAUNCH(O, B, 4, 1, 2, 64);                                \
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
    return check_launch(UNIT ? "scaled_mm_fp8" : "scaled_mm_mxfp8");
}

// Split-K: a grid of at most half as many 256 x 256 tiles as CUs leaves most CUs idle
// while each tile walks all of K.  Such a grid with long K instead runs S K ranges of every
// tile (each of ks stages, a multiple of 4, at least kMinSplitStages) as S times as many
// workgroups, at most one per CU, which write fp32 partial tiles to the caller's workspace;
// a second launch adds them.  A partial tile (256 KB) costs about as much memory traffic
// to write and again to read back as 8 stages of operand loads, so short K (fewer than
// kMinSplitK stages) keeps whole-K half tiles instead.  With at most a quarter as many
// tiles as CUs the split runs 256 x 128 half tiles, at least two K ranges each: a half
// tile's stage costs ~53% of a full tile's (C4's last round) and its partial (128 KB) half
// as much traffic, so for the same workgroups the partials move half the bytes.  Half
// tiles split from kMinSplitKHalf stages on, and below kMinSplitK stages on at most
// kShortSplitSlots workgroups (same process, against whole-K half tiles: 512 x 4096 x 3072
// 23.0 against 28.5 us, 22.6 with 256 workgroups; 256 x 9216 x 3072 24.8 against 29.3;
// 256 x 3072 x 3072 17.9 against 21.2; with that cap on long K too, 256 x 5120 x 13824
// took 38.3 against 36.0 us).  Full tiles split only into three ranges or more: two
// ranges give as many workgroups as whole-K half tiles, which need no partials (same
// process: 256 x 32768 x 5120 57.6 against 66.6 us split, 384 x 12288 x 6144 54.0 against
// 56.2; with three, 256 x 18432 x 8192 60.7 split against 71.2).
// Measured, graph-timed: M = 256, N = 5120, K = 13824 40.5 us split in full tiles against
// 110.8 us whole-K half tiles; N = 13824, K = 5120 40.1 against 46.9 us; N = 18432,
// K = 3072 38.3 against 32.1 us (not split).  Half tiles against full tiles in the split
// (same process): 256 x 4096 x 4096 20.9 against 27.1 us, 256 x 5120 x 13824 36.3 against
// 40.4, 512 x 3072 x 13824 38.6 against 42.5, 256 x 13824 x 5120 38.7 against 40.6.
constexpr int kMinSplitStages = 12;
constexpr int kMinSplitK = 64;      // stages
constexpr int kMinSplitKHalf = 32;  // stages, half tiles
constexpr int kShortSplitSlots = 224;

struct SplitPlan {
    int S = 1;   // K ranges (1: no split)
    int ks = 0;  // stages per range
    int nw = 4;  // 4: full tiles, 2: half tiles
};

SplitPlan split_plan(int M, int N, int K) {
    SplitPlan sp;
    if (M <= kSkinnyMaxM) return sp;
    const int tiles = static_cast<int>(cdiv(M, mx::BM) * cdiv(N, mx::BN));
    const int KT = static_cast<int>(cdiv(K, mx::BK));
    const bool half = tiles <= kGemmSlots / 4;
    if (tiles > kGemmSlots / 2 || KT < (half ? kMinSplitKHalf : kMinSplitK)) return sp;
    const int units = half ? 2 * tiles : tiles;
    const int slots = half && KT < kMinSplitK ? kShortSplitSlots : kGemmSlots;
    const int S = min(slots / units, KT / kMinSplitStages);
    if (S < (half ? 2 : 3)) return sp;
    sp.ks = static_cast<int>(rup(cdiv(KT, S), 4));
    sp.S = static_cast<int>(cdiv(KT, sp.ks));
    sp.nw = half ? 2 : 4;
    return sp;
}

// one partial tile (or two partial half tiles) per tile and K range
int64_t split_workspace_bytes(int M, int N, int K) {
    const SplitPlan sp = split_plan(M, N, K);
    if (sp.S < 2) return 0;
    return cdiv(M, mx::BM) * cdiv(N, mx::BN) * sp.S * static_cast<int64_t>(mx::kPartTile) * 4;
}

template <bool UNIT, int NW>
void launch_split(mx::Args p, int out_code, int bias_code, bool has_bias, hipStream_t st) {
    const int units = p.tiles_m * p.tiles_n * (4 / NW);
    hipLaunchKernelGGL((mx::gemm_split_kernel<UNIT, NW>), dim3(static_cast<unsigned>(units * p.splits)),
                       dim3(mx::NT), 0, st, p);
    const dim3 g2(static_cast<unsigned>(units * (mx::BM * 64 * NW / 4 / 256)));
#define LAUNCH(O, B) hipLaunchKernelGGL((mx::gemm_reduce_kernel<O, B, UNIT, NW>), g2, dim3(256), 0, st, p)
#define BY_BIAS(O)                                                     \
    do {                                                               \
        if (!has_bias) LAUNCH(O, -1);                                  \
        else if (bias_code == CKH_F32) LAUNCH(O, CKH_F32);             \
        else if (bias_code == CKH_F16) LAUNCH(O, CKH_F16);             \
        else LAUNCH(O, CKH_BF16);                                      \
    } while (0)
    if (out_code == CKH_BF16) BY_BIAS(CKH_BF16);
    else if (out_code == CKH_F16) BY_BIAS(CKH_F16);
    else BY_BIAS(CKH_F32);
#undef BY_BIAS
#undef LAUNCH
}

// The 256 x 256 tiles run one per CU in rounds.  When the last round would be at most
// half full (e.g. 864 tiles = 3 rounds + 96), its tiles run as twice as many 256 x 128
// half tiles (about 55% of a full tile's time each), in the same grid.  A grid of one
// round fills the remaining CUs with weight-prefetch workgroups (prefetch_weight).
// Activations of at most kSkinnyMaxM rows take the skinny kernel, and small grids split K
// when the caller gives a workspace.
template <bool UNIT>
int launch_gemm(mx::Args p, int out_code, int bias_code, bool has_bias, void* workspace, int64_t workspace_bytes,
                hipStream_t st) {
    if (p.M <= kSkinnyMaxM) return launch_skinny<UNIT>(p, out_code, bias_code, has_bias, st);
    const SplitPlan sp = split_plan(p.M, p.N, p.K);
    if (sp.S > 1 && workspace && workspace_bytes >= split_workspace_bytes(p.M, p.N, p.K)) {
        p.splits = sp.S;
        p.ks = sp.ks;
        p.part = static_cast<float*>(workspace);
        if (sp.nw == 2) launch_split<UNIT, 2>(p, out_code, bias_code, has_bias, st);
        else launch_split<UNIT, 4>(p, out_code, bias_code, has_bias, st);
        return check_launch(UNIT ? "scaled_mm_fp8" : "scaled_mm_mxfp8");
    }
    const int tiles = p.tiles_m * p.tiles_n;
    // (a grid of at most half as many tiles as CUs with no workspace for split-K runs all
    // of its tiles as half tiles: 256 x 18432 x 3072 measured 31.9 against 41.3 us)
    const int tail = tiles > kGemmSlots ? tiles % kGemmSlots : tiles;
    p.n_half = (tail > 0 && tail <= kGemmSlots / 2) ? tail : 0;
    p.n_full = tiles - p.n_half;
    const int wgs = p.n_full + 2 * p.n_half;
    // (the CUs the device has, which a partitioned GPU reduces: prefetch workgroups that
    // found no idle CU would run after the tiles, for nothing)
    const int cus = device_cus();
    p.n_pref = wgs < cus ? cus - wgs : 0;
    launch_grid<UNIT>(p, static_cast<unsigned>(wgs + p.n_pref), out_code, bias_code, has_bias, st);
    return check_launch(UNIT ? "scaled_mm_fp8" : "scaled_mm_mxfp8");
}

mx::Args base_args(const void* a, const void* b, const void* bias, void* out, int64_t M, int64_t N, int64_t K) {
    mx::Args p{};
    p.a = static_cast<const uint8_t*>(a);
    p.b = static_cast<const uint8_t*>(b);
    p.bias = bias;
    p.out = out;
    p.M = static_cast<int>(M);
    p.N = static_cast<int>(N);
    p.K = static_cast<int>(K);
    p.tiles_m = static_cast<int>(cdiv(M, mx::BM));
    p.tiles_n = static_cast<int>(cdiv(N, mx::BN));
    return p;
}

}  // namespace

extern "C" int64_t ckh_scaled_mm_workspace_bytes(int64_t M, int64_t N, int64_t K) {
    if (M <= 0 || N <= 0 || K <= 0 || M >= (1ll << 30) || N >= (1ll << 30) || K >= (1ll << 24)) return 0;
    return split_workspace_bytes(static_cast<int>(M), static_cast<int>(N), static_cast<int>(K));
}

extern "C" int ckh_scaled_mm_mxfp8(const void* a, const void* b, const void* sa, const void* sb, const void* bias,
                                   void* out, int64_t M, int64_t N, int64_t K, int out_code, int bias_code,
                                   void* workspace, int64_t workspace_bytes, uintptr_t stream) {
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
    mx::Args p = base_args(a, b, bias, out, M, N, K);
    p.sa = static_cast<const uint8_t*>(sa);
    p.sb = static_cast<const uint8_t*>(sb);
    p.ncb = static_cast<int>(cdiv(K / 32, 4));
    p.sa_rows = static_cast<int>(rup(M, 128));
    p.sb_rows = static_cast<int>(rup(N, 128));
    CKH_REQUIRE(!workspace || aligned(workspace, 16), "scaled_mm_mxfp8: workspace misaligned");
    return launch_gemm<false>(p, out_code, bias_code, bias != nullptr, workspace, workspace_bytes,
                              reinterpret_cast<hipStream_t>(stream));
}

extern "C" int ckh_scaled_mm_fp8(const void* a, const void* b, const float* scale_a, const float* scale_b,
                                 const void* bias, void* out, int64_t M, int64_t N, int64_t K, int out_code,
                                 int bias_code, void* workspace, int64_t workspace_bytes, uintptr_t stream) {
    CKH_REQUIRE(a && b && scale_a && scale_b && out, "scaled_mm_fp8: null pointer");
    CKH_REQUIRE(M >= 0 && N >= 0 && K > 0, "scaled_mm_fp8: sizes must be M, N >= 0 and K > 0");
    CKH_REQUIRE(K % 16 == 0, "scaled_mm_fp8: K (%lld) must be a multiple of 16", (long long)K);
    CKH_REQUIRE(M * K < (1ll << 31) && N * K < (1ll << 31) && K < (1ll << 24),
                "scaled_mm_fp8: operand larger than 2 GiB");
    CKH_REQUIRE(out_code == CKH_F32 || out_code == CKH_F16 || out_code == CKH_BF16,
                "scaled_mm_fp8: unsupported output dtype code %d", out_code);
    CKH_REQUIRE(!bias || bias_code == CKH_F32 || bias_code == CKH_F16 || bias_code == CKH_BF16,
                "scaled_mm_fp8: unsupported bias dtype code %d", bias_code);
    CKH_REQUIRE(aligned(a, 16) && aligned(b, 16) && aligned(scale_a, 4) && aligned(scale_b, 4) && aligned(out, 16),
                "scaled_mm_fp8: pointers misaligned");
    if (M == 0 || N == 0) return CKH_OK;
    mx::Args p = base_args(a, b, bias, out, M, N, K);
    p.tsa = scale_a;
    p.tsb = scale_b;
    CKH_REQUIRE(!workspace || aligned(workspace, 16), "scaled_mm_fp8: workspace misaligned");
    return launch_gemm<true>(p, out_code, bias_code, bias != nullptr, workspace, workspace_bytes,
                             reinterpret_cast<hipStream_t>(stream));
}
