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
// registers; the LDS reads of stage t+1's fragments and scale words overlap stage t's
// 16 MFMAs.  Activation fragments are double-buffered (each is used by all of a stage's
// MFMA rows); each weight fragment is read into its own registers right after its last
// MFMA of the stage; with 32 fewer live VGPRs the block-scaled kernels no longer spill
// (2 VGPRs still do in some per-tensor and bf16-activation instantiations).  Global data moves in pairs of stages through registers: one load
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
#include "quant_math.h"

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
constexpr int STILE = 1024;     // bytes of one operand's scale words per stage (256 rows)
// One stage buffer: weight tile, activation tile, scales, and 64 bytes of padding.  LDS
// banks repeat every 128 bytes; a staged store writes row r of buffers s and s + 1
// from 8 neighbouring lanes (64 bytes each), which the padding puts in opposite halves
// of the bank cycle (measured conflict-free; without it every store conflicts 2-way).
constexpr int BUF = 2 * TILE + 2 * STILE + 64;
constexpr int EPI_ROW = 528;  // bytes of one staged 16-bit output row (512 + 16 pad, rows 16-byte aligned)
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
    // per-tensor mode only: the two fp32 tensor scales (device), applied in the epilogue
    const float* tsa;
    const float* tsb;
};

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

// 16-bit activation, quantized to MXFP8 in the load path (scaled_mm_mxfp8_dynamic): one
// stage at a time, 64 elements = 128 bytes of each of the tile's 256 rows.  Wave w, load j
// covers rows R = 64 w + 8 j .. +7: lane i fetches 16-byte chunk c = i % 8 (8 elements)
// of row R + i / 8, so each 8 lanes read one whole 128-byte line and lanes 4b .. 4b+3 of
// a row hold its 32-element block b.  The chunk's 8 E4M3 codes go to logical chunk c / 2,
// half c % 2, of the row in the stage's activation tile (physical chunk (c/2) ^ swz(row)).
struct Loader16 {
    __amdgpu_buffer_rsrc_t rs;
    uint32_t voff;      // lane's global byte offset for j = 0, stage 0
    uint32_t rowstep;   // 8 rows: global distance between consecutive loads j
    uint32_t lds_even;  // LDS offset of the codes within a stage tile for even j (adds 512 j);
                        // for odd j the chunk index is xor 1, i.e. the offset xor 16
    uint32_t sc_off;    // offset of the row's scale word in the stage buffer's activation
                        // scale area (j = 0), plus the block's byte within the stage
};

__device__ __forceinline__ Loader16 make_loader16(const uint8_t* tile_base, int valid_rows, int K, int wave,
                                                  int lane) {
    Loader16 L;
    L.rs = buffer_rsrc(tile_base, static_cast<uint32_t>(max(valid_rows, 0)) * 2u * K);
    const int row = 64 * wave + (lane >> 3), c = lane & 7;
    L.voff = static_cast<uint32_t>(row * 2 * K + 16 * c);
    L.rowstep = 16u * K;
    L.lds_even = static_cast<uint32_t>(row * BK + ((((c >> 1) ^ swz(row))) << 4) + (c & 1) * 8);
    // word of row R = 64 w + 8 j + i/8 in a 256-row scale chunk pair: (R/128)*512 +
    // (R%32)*16 + ((R%128)/32)*4, and block b = c/4 of the stage's two is byte b of the
    // stage's pair of bytes
    L.sc_off = static_cast<uint32_t>((wave >> 1) * 512 + (lane >> 3) * 16 + (wave & 1) * 8 + (c >> 2));
    return L;
}

// Offset added for stage s: past K the lane reads zeros from outside the descriptor.
__device__ __forceinline__ uint32_t stage_add16(int k0, int K, int lane) {
    return (k0 + 8 * (lane & 7) < K) ? static_cast<uint32_t>(2 * k0) : 0x80000000u;
}

template <int J>
__device__ __forceinline__ void load_piece16(const Loader16& L, v4u (&x)[8], uint32_t add) {
    x[J] = __builtin_amdgcn_raw_buffer_load_b128(L.rs, L.voff + J * L.rowstep + add, 0, 0);
}

// Quantize piece J (8 elements of one 32-element block) as quantize_mxfp8 does (the codes
// and exponent of mx_codes16 but for scale-0 blocks, below; block amax over the lane quad)
// and store its codes to the stage tile at
// `tile`; the quad stores the block's E8M0 byte to the stage's scale area `sc` at byte
// 2 * ODD + b of the row's word, the byte the stage's MFMAs select.
template <int AIN, int J, bool ODD>
__device__ __forceinline__ void quantize_piece16(const Loader16& L, const v4u (&x)[8], uint8_t* tile, uint8_t* sc,
                                                 int lane) {
    const uint4 w = make_uint4(x[J][0], x[J][1], x[J][2], x[J][3]);
    uint32_t m = amax16x8(w);
    m = max(m, dpp<0xB1>(m));  // quad_perm [1,0,3,2]
    m = max(m, dpp<0x4E>(m));  // quad_perm [2,3,0,1]
    const uint32_t bits = amax16_to_f32_bits<AIN>(m);
    // Branch-free (a branch here splits the stage's hand-scheduled slots and lets the
    // compiler sink the MFMAs past the stage barriers).  Exponent 0 is a zero block (+0
    // codes, as quantize_mxfp8) or a scale of 0.0 (infinite amax, or a nonzero amax of at
    // most ~1.3e-36), where quantize_mxfp8 writes 0x7E|sign / 0xFF codes whose products
    // with scale byte 0 are +-448 * 2^-127 * b: here such a block contributes 0, or NaN
    // codes when it holds a NaN (amax NaN), so the output keeps the NaN.
    const uint32_t e = mx_exponent_select(bits);
    const float scale = as_f((e ? e : 1u) << 23);
    uint2 codes = make_uint2(scaled_e4m3x4<AIN>(w.x, w.y, scale), scaled_e4m3x4<AIN>(w.z, w.w, scale));
    // materialised here: otherwise the compiler sinks the converts into a branch on e
    __asm__ volatile("" : "+v"(codes.x), "+v"(codes.y));
    const uint32_t fill = bits > 0x7f800000u ? ~0u : 0u;
    codes = e ? codes : make_uint2(fill, fill);
    *reinterpret_cast<uint2*>(tile + ((J & 1) ? (L.lds_even ^ 16u) : L.lds_even) + 512 * J) = codes;
    // all four lanes of the quad store the same byte (a guard would be a branch)
    sc[L.sc_off + (J & 3) * 128 + (J >> 2) * 4 + (ODD ? 2 : 0)] = static_cast<uint8_t>(e);
}

// Scale words of a pair of stages (one 128-wide K block): for a 256-row tile they are
// two contiguous 512-byte chunks of the swizzled tensor (rows 128*rb .. +127), chunk
// (rb * ncb + k0/128).  Wave w copies chunk rb = w & 1 of operand w >> 1 (0 = weight,
// 1 = activation), 2 words per lane.  Inside a chunk row r's word sits at
// (r % 32) * 16 + ((r % 128) / 32) * 4, so a lane's words for its four 32-row tiles are
// one contiguous 16-byte LDS read.  Both stages of the pair get a copy.
struct ScaleWords {
    uint32_t s0, s1;
};

__device__ __forceinline__ void load_scales(ScaleWords& S, __amdgpu_buffer_rsrc_t rs_b, __amdgpu_buffer_rsrc_t rs_a,
                                            int rb0_b, int rb0_a, int ncb, int k0, int K, int wave, int lane) {
    const int op = wave >> 1, rb = wave & 1;
    const __amdgpu_buffer_rsrc_t rs = op ? rs_a : rs_b;
    uint32_t chunk = static_cast<uint32_t>(((op ? rb0_a : rb0_b) + rb) * ncb + (k0 >> 7)) * 512u;
    chunk = k0 < K ? chunk : 0x80000000u;  // stages past K: zero scale words
    S.s0 = __builtin_amdgcn_raw_buffer_load_b32(rs, chunk + lane * 4, 0, 0);
    S.s1 = __builtin_amdgcn_raw_buffer_load_b32(rs, chunk + 256 + lane * 4, 0, 0);
}

__device__ __forceinline__ void store_scales(const ScaleWords& S, uint8_t* sx, uint8_t* sy, int wave, int lane) {
    const int off = (wave >> 1) * STILE + (wave & 1) * 512 + lane * 4;
    *reinterpret_cast<uint32_t*>(sx + off) = S.s0;
    *reinterpret_cast<uint32_t*>(sx + off + 256) = S.s1;
    *reinterpret_cast<uint32_t*>(sy + off) = S.s0;
    *reinterpret_cast<uint32_t*>(sy + off + 256) = S.s1;
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
// AIN: -1 when the activation is E4M3 codes with E8M0 scales; CKH_BF16 / CKH_F16 when it
// is a 16-bit tensor quantized to MXFP8 in the load path (scaled_mm_mxfp8_dynamic): each
// stage t quantizes the activation of stage t + 2 into its buffer (codes and the E8M0
// bytes its MFMAs select) and loads that of stage t + 3, so the activation moves one stage
// at a time through the same 32 staging registers; every wave moves weight scale words.
//
// Stage buffers 0, 1 and 2, 3 live in two arrays.  Every stage reads fragments from one
// array and writes staged data into the other, so the compiler knows they never alias
// and may interleave the two freely; within an array, per-lane addresses of different
// buffers differ only by immediates.
template <int OUT, int BIAS, bool UNIT, int NW, int AIN>
__device__ __forceinline__ void gemm_tile(const Args& p, int bid, uint8_t* lds01, uint8_t* lds23) {
    constexpr bool AQ = AIN >= 0;
    static_assert(!(AQ && UNIT), "the in-load quantize produces block scales");
    constexpr int TBN = 64 * NW;  // tile width along n
    constexpr int PB = TBN / 32;  // staged weight loads per lane per pair of stages
    constexpr int SLOTS = 4 * NW;  // MFMAs per wave per stage

    // Workgroups are dispatched round-robin over the 8 XCDs; full tiles are remapped so
    // each XCD walks a contiguous range of tiles (in grouped order).  Half tiles give
    // tile L's two column halves to consecutive workgroups.
    if (NW == 4 && (p.n_full & 7) == 0) bid = (bid & 7) * (p.n_full >> 3) + (bid >> 3);
    const int L = NW == 4 ? bid : p.n_full + (bid >> 1);
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
    const Loader16 LA16 = make_loader16(p.a + static_cast<int64_t>(m0) * 2 * p.K, min(BM, p.M - m0), p.K, wave, lane);
    // scale words: waves 0, 1 move the weight's, waves 2, 3 the activation's; with the
    // in-load quantize, waves 2, 3 repeat waves 0, 1 (identical bytes to the same LDS
    // words: a branch instead would let the compiler sink the MFMAs past the barriers)
    const int swave = AQ ? (wave & 1) : wave;
    const __amdgpu_buffer_rsrc_t rssb = buffer_rsrc(p.sb, static_cast<uint32_t>(p.sb_rows) * p.ncb * 4);
    const __amdgpu_buffer_rsrc_t rssa = buffer_rsrc(p.sa, static_cast<uint32_t>(p.sa_rows) * p.ncb * 4);
    const FragAddr fab = make_frag_addr(wn * 32 * NW, lane);
    const FragAddr faa = make_frag_addr(wm * 128, lane);
    const int KT = (p.K + BK - 1) / BK;

    v16f acc[NW][4];
#pragma unroll
    for (int i = 0; i < NW; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = v16f{};

    auto buf = [&](auto b_c) -> uint8_t* {
        constexpr int B = decltype(b_c)::value & 3;
        return (B < 2 ? lds01 : lds23) + (B & 1) * BUF;
    };
    // Register staging: a pair of stages of one operand (+ the pair's scale words with
    // the weight) at a time.
    v4u SB[8], SA[8];
    ScaleWords SW;
    auto load_b = [&](int s) {
        load_pair<PB>(LB, SB, s * BK, p.K);
        if constexpr (!UNIT) load_scales(SW, rssb, rssa, n0 >> 7, m0 >> 7, p.ncb, s * BK, p.K, swave, lane);
    };
    // the activation of stage s into x (16-bit path)
    auto load_a16 = [&](v4u (&x)[8], int s) {
        const uint32_t add = stage_add16(s * BK, p.K, lane);
        for_each_index([&](auto j_c) { load_piece16<decltype(j_c)::value>(LA16, x, add); },
                       std::make_integer_sequence<int, 8>{});
    };
    // quantize the staged activation x of stage s (parity ODD) into buffer b_c
    auto quantize_a16 = [&](const v4u (&x)[8], auto b_c, auto odd_c) {
        for_each_index([&](auto j_c) {
            quantize_piece16<AIN, decltype(j_c)::value, decltype(odd_c)::value>(LA16, x, buf(b_c) + TILE,
                                                                                buf(b_c) + 2 * TILE + STILE, lane);
        }, std::make_integer_sequence<int, 8>{});
    };
    auto load_a = [&](int s) { load_pair(LA, SA, s * BK, p.K); };
    auto store_a = [&](auto x_c, auto y_c) { store_pair(LA, SA, buf(x_c) + TILE, buf(y_c) + TILE); };
    // this lane's 4 scale words (tiles t = 0..3) of each operand for a stage, shifted so
    // byte 0 / byte 2 are the lane-half's scales of the even / odd 64-wide stage
    const int hs = 8 * half;
    // the weight scale chunk holding this wave's n rows, and its first 32-row tile there
    const int sbc = NW == 4 ? wn : 0, sbt = NW == 4 ? 0 : 2 * wn;
    auto read_scales = [&](auto b_c, uint32_t (&sb)[4], uint32_t (&sa)[4]) {
        if constexpr (UNIT) {
#pragma unroll
            for (int t = 0; t < 4; ++t) sb[t] = sa[t] = 0x7f7f7f7fu;
            return;
        }
        const uint8_t* st = buf(b_c) + 2 * TILE;
        const v4u wb = *reinterpret_cast<const v4u*>(st + sbc * 512 + r32 * 16);
        const v4u wa = *reinterpret_cast<const v4u*>(st + STILE + wm * 512 + r32 * 16);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            sb[t] = (NW == 4 ? wb[t] : (sbt ? wb[2 + (t & 1)] : wb[t & 1])) >> hs;
            sa[t] = wa[t] >> hs;
        }
    };

    uint32_t scb[4], sca[4];
    Frags F0, F1;
    v8i FB[NW];

    // Stage t held in buffer B = t % 4 (compile-time): activation fragments F and the
    // weight fragments FB (stage t) are in registers; read stage t+1 into G and, each
    // after its last MFMA here (slot 4i + 3), into FB[i].  A pair of stages (s, s+1), s even, moves in
    // two halves: the activation pair is loaded at stage s-4 and written to LDS at
    // s-3, the weight pair (with scales) loaded at s-3 and written at s-2.  Each write
    // targets buffers whose previous stages were read before the current barrier.
    //
    // The stage is scheduled by hand in 16 slots, one MFMA each (sched_barrier keeps
    // the order): the next stage's scale words first (their shifts 12 slots later, so
    // no LDS latency is exposed), then its fragments in the order the next stage uses
    // them, and in slots 0..7 one staged chunk written to LDS followed by the load that
    // refills its registers, which therefore has a whole stage to arrive.  (Double-
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
        const uint32_t add = EVEN ? pair_add(LA, (t + 4) * BK, p.K) : pair_add(LB, (t + 3) * BK, p.K);
        const uint32_t add16 = stage_add16((t + 3) * BK, p.K, lane);
        v4u wb, wa;
        uint32_t nb[4], na[4];
        auto slot = [&](auto k_c) {
            constexpr int k = decltype(k_c)::value;
            constexpr int i = k / 4, j = k % 4;
            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(FB[i], F.a[j], acc[i][j], 0, 0, OPSEL, scb[i],
                                                                        OPSEL, sca[j]);
            if constexpr (k == 0 && !UNIT) {
                wb = *reinterpret_cast<const v4u*>(nx + 2 * TILE + sbc * 512 + r32 * 16);
                wa = *reinterpret_cast<const v4u*>(nx + 2 * TILE + STILE + wm * 512 + r32 * 16);
            }
            if constexpr (k == 1) G.a[0] = read_frag(nx + TILE, faa);
            if constexpr (k >= 3 && k <= 5) G.a[k - 2] = read_frag(nx + TILE + (k - 2) * 32 * BK, faa);
            if constexpr (k % 4 == 3 && k / 4 < NW) FB[k / 4] = read_frag(nx + (k / 4) * 32 * BK, fab);
            if constexpr (k < 8 && AQ) {
                quantize_piece16<AIN, k, !EVEN>(LA16, SA, buf(P2{}) + TILE, buf(P2{}) + 2 * TILE + STILE, lane);
                load_piece16<k>(LA16, SA, add16);
                if constexpr (k < PB) {
                    if constexpr (EVEN) store_piece<k>(LB, SB, wx, wy);
                    else load_piece<k>(LB, SB, add);
                }
            } else if constexpr (k < 8) {
                if constexpr (EVEN) {
                    if constexpr (k < PB) store_piece<k>(LB, SB, wx, wy);
                    load_piece<k>(LA, SA, add);
                } else {
                    store_piece<k>(LA, SA, wx, wy);
                    if constexpr (k < PB) load_piece<k>(LB, SB, add);
                }
            }
            if constexpr (k == (SLOTS > 8 ? 8 : SLOTS - 1) && !UNIT) {
                if constexpr (EVEN) store_scales(SW, buf(P2{}) + 2 * TILE, buf(P3{}) + 2 * TILE, swave, lane);
                else load_scales(SW, rssb, rssa, n0 >> 7, m0 >> 7, p.ncb, (t + 3) * BK, p.K, swave, lane);
            }
            if constexpr (k == SLOTS - 4) {
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    nb[u] = UNIT ? 0x7f7f7f7fu : (NW == 4 ? wb[u] : (sbt ? wb[2 + (u & 1)] : wb[u & 1])) >> hs;
                    na[u] = UNIT ? 0x7f7f7f7fu : wa[u] >> hs;
                }
            }
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
    if constexpr (AQ) {
        // activation stages 0, 1 quantized into their buffers, stage 2 staged in SA for
        // stage 0 to quantize; weight as below
        v4u XA[8], X1[8], XB[8];
        ScaleWords XW;
        load_a16(XA, 0);
        load_a16(X1, 1);
        load_pair<PB>(LB, XB, 0, p.K);
        load_scales(XW, rssb, rssa, n0 >> 7, m0 >> 7, p.ncb, 0, p.K, swave, lane);
        load_b(2);
        load_a16(SA, 2);
        quantize_a16(XA, B0{}, std::false_type{});
        quantize_a16(X1, B1{}, std::true_type{});
        store_pair<PB>(LB, XB, buf(B0{}), buf(B1{}));
        store_scales(XW, buf(B0{}) + 2 * TILE, buf(B1{}) + 2 * TILE, swave, lane);
    } else {
        v4u XA[8], XB[8];
        ScaleWords XW;
        load_a(0);
        load_pair<PB>(LB, XB, 0, p.K);
        if constexpr (!UNIT) load_scales(XW, rssb, rssa, n0 >> 7, m0 >> 7, p.ncb, 0, p.K, wave, lane);
        load_pair(LA, XA, 2 * BK, p.K);
        load_b(2);
        store_a(B0{}, B1{});
        store_pair<PB>(LB, XB, buf(B0{}), buf(B1{}));
        if constexpr (!UNIT) store_scales(XW, buf(B0{}) + 2 * TILE, buf(B1{}) + 2 * TILE, wave, lane);
        store_pair(LA, XA, buf(B2{}) + TILE, buf(B3{}) + TILE);
    }
    stage_barrier<WAIT_LGKM0>();
    read_frags(F0, FB, lds01, fab, faa);
    read_scales(B0{}, scb, sca);

    // stages in groups of 4 (buffer index = stage % 4); stages past K are all zeros
    for (int t = 0; t < KT; t += 4) {
        stage(B0{}, t, F0, F1);
        stage(B1{}, t + 1, F1, F0);
        stage(B2{}, t + 2, F0, F1);
        stage(B3{}, t + 3, F1, F0);
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

// One grid runs both kinds of workgroup: the full tiles first, then (when the last
// round of full tiles would be at most half full) that round's tiles as half tiles.
// The dispatcher starts half-tile workgroups on CUs as their last full tile ends, so
// the tail overlaps the uneven end of the previous round instead of waiting for a
// second launch.
template <int OUT, int BIAS, bool UNIT, int AIN>
__global__ __launch_bounds__(NT) void gemm_kernel(Args p) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds01[2 * BUF];
    __shared__ __attribute__((aligned(1024))) uint8_t lds23[2 * BUF];
    const int b = blockIdx.x;
    if (b < p.n_full) gemm_tile<OUT, BIAS, UNIT, 4, AIN>(p, b, lds01, lds23);
    else gemm_tile<OUT, BIAS, UNIT, 2, AIN>(p, b - p.n_full, lds01, lds23);
}

}  // namespace mx
}  // namespace ckh

using namespace ckh;

namespace {

// Workgroups that can hold a 256 x 256 tile at once: one per CU.
constexpr int kGemmSlots = 256;

// The 16-bit-activation kernels take a bias of the output's dtype only (as the layouts
// pass it), which keeps their instantiations to three per activation dtype.
template <bool UNIT, int AIN>
void launch_grid(const mx::Args& p, unsigned wgs, int out_code, int bias_code, bool has_bias, hipStream_t st) {
#define LAUNCH(O, B) hipLaunchKernelGGL((mx::gemm_kernel<O, B, UNIT, AIN>), dim3(wgs), dim3(mx::NT), 0, st, p)
#define BY_BIAS(O)                                                     \
    do {                                                               \
        if (!has_bias) LAUNCH(O, -1);                                  \
        else if constexpr (AIN >= 0) LAUNCH(O, O);                     \
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
// half tiles (about 55% of a full tile's time each), in the same grid.
template <bool UNIT, int AIN = -1>
int launch_gemm(mx::Args p, int out_code, int bias_code, bool has_bias, hipStream_t st) {
    const int tiles = p.tiles_m * p.tiles_n;
    const int tail = tiles > kGemmSlots ? tiles % kGemmSlots : 0;
    p.n_half = (tail > 0 && tail <= kGemmSlots / 2) ? tail : 0;
    p.n_full = tiles - p.n_half;
    launch_grid<UNIT, AIN>(p, static_cast<unsigned>(p.n_full + 2 * p.n_half), out_code, bias_code, has_bias, st);
    return check_launch(UNIT ? "scaled_mm_fp8" : AIN >= 0 ? "scaled_mm_mxfp8_dynamic" : "scaled_mm_mxfp8");
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
    mx::Args p = base_args(a, b, bias, out, M, N, K);
    p.sa = static_cast<const uint8_t*>(sa);
    p.sb = static_cast<const uint8_t*>(sb);
    p.ncb = static_cast<int>(cdiv(K / 32, 4));
    p.sa_rows = static_cast<int>(rup(M, 128));
    p.sb_rows = static_cast<int>(rup(N, 128));
    return launch_gemm<false>(p, out_code, bias_code, bias != nullptr, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int ckh_scaled_mm_fp8(const void* a, const void* b, const float* scale_a, const float* scale_b,
                                 const void* bias, void* out, int64_t M, int64_t N, int64_t K, int out_code,
                                 int bias_code, uintptr_t stream) {
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
    return launch_gemm<true>(p, out_code, bias_code, bias != nullptr, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int ckh_scaled_mm_mxfp8_dynamic(const void* a, const void* b, const void* sb, const void* bias, void* out,
                                           int64_t M, int64_t N, int64_t K, int a_code, int out_code, int bias_code,
                                           uintptr_t stream) {
    CKH_REQUIRE(a && b && sb && out, "scaled_mm_mxfp8_dynamic: null pointer");
    CKH_REQUIRE(M >= 0 && N >= 0 && K > 0, "scaled_mm_mxfp8_dynamic: sizes must be M, N >= 0 and K > 0");
    CKH_REQUIRE(K % 32 == 0, "scaled_mm_mxfp8_dynamic: K (%lld) must be a multiple of 32", (long long)K);
    CKH_REQUIRE(a_code == CKH_BF16 || a_code == CKH_F16,
                "scaled_mm_mxfp8_dynamic: unsupported activation dtype code %d (bf16 or f16)", a_code);
    CKH_REQUIRE(2 * M * K < (1ll << 31) && N * K < (1ll << 31) && K < (1ll << 24),
                "scaled_mm_mxfp8_dynamic: operand larger than 2 GiB");
    CKH_REQUIRE(out_code == CKH_F32 || out_code == CKH_F16 || out_code == CKH_BF16,
                "scaled_mm_mxfp8_dynamic: unsupported output dtype code %d", out_code);
    CKH_REQUIRE(!bias || bias_code == out_code,
                "scaled_mm_mxfp8_dynamic: bias dtype code %d must be the output's (%d)", bias_code, out_code);
    CKH_REQUIRE(aligned(a, 16) && aligned(b, 16) && aligned(sb, 4) && aligned(out, 16),
                "scaled_mm_mxfp8_dynamic: pointers misaligned");
    if (M == 0 || N == 0) return CKH_OK;
    mx::Args p = base_args(a, b, bias, out, M, N, K);
    p.sa = static_cast<const uint8_t*>(sb);  // unused: the activation's scales are made in the kernel
    p.sb = static_cast<const uint8_t*>(sb);
    p.ncb = static_cast<int>(cdiv(K / 32, 4));
    p.sa_rows = 0;
    p.sb_rows = static_cast<int>(rup(N, 128));
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (a_code == CKH_BF16) return launch_gemm<false, CKH_BF16>(p, out_code, bias_code, bias != nullptr, st);
    return launch_gemm<false, CKH_F16>(p, out_code, bias_code, bias != nullptr, st);
}
