// Block-scaled quantizers (MXFP8, NVFP4) and their dequantizers for gfx950.
//
// Work unit: one row r and one group of four consecutive K-blocks (the four blocks
// whose scales form one aligned 32-bit word of the 32_4_4 swizzled layout).  Lanes of
// a unit each load 8 consecutive input elements (one 16-byte load for 16-bit inputs),
// so a wavefront reads a contiguous row segment; the block amax is reduced across the
// lanes of the block, and the four scale bytes are OR-combined across the unit so that
// one lane writes the scale word with a single 32-bit store.  Units cover the padded
// scale rows (a multiple of 128) so the kernel also writes every padding byte: outputs
// can be allocated uninitialised.
//
//   MXFP8: 32-element blocks, 4 lanes per block, 16 lanes per unit.
//   NVFP4: 16-element blocks, 2 lanes per block,  8 lanes per unit.
#include "ckh_common.h"
#include "quant_math.h"

namespace ckh {

constexpr int kThreads = 256;

template <typename T>
__device__ __forceinline__ T shfl_xor(T v, int m) {
    return __shfl_xor(v, m, 64);
}

// Load the 8 elements [k0, k0+8) of row r of x [orows, ocols]; outside x they are 0
// (the zero padding of pad_32x / pad_16x).
template <int IN>
__device__ __forceinline__ void load_row8(const void* x, int64_t r, int64_t k0, int64_t orows, int64_t ocols,
                                          bool vec_ok, float (&v)[8]) {
    constexpr int ES = ElemSize<IN>::value;
    if (vec_ok && r < orows && k0 + 8 <= ocols) {
        load8<IN>(static_cast<const char*>(x) + (r * ocols + k0) * ES, v);
    } else {
#pragma unroll
        for (int t = 0; t < 8; ++t) v[t] = (r < orows && k0 + t < ocols) ? load1<IN>(x, r * ocols + k0 + t) : 0.0f;
    }
}

__device__ __forceinline__ uint32_t absmax_bits(const float (&v)[8]) {
    // |v| as integers orders like the floats (NaN above +inf), so an integer max is
    // the float amax, NaN-propagating like torch.amax.
    uint32_t m = 0;
#pragma unroll
    for (int t = 0; t < 8; ++t) m = max(m, as_u(v[t]) & 0x7fffffffu);
    return m;
}

// ------------------------------------------------------------------- MXFP8
template <int IN>
__global__ __launch_bounds__(kThreads) void quantize_mxfp8_kernel(const void* __restrict__ x,
                                                                  uint8_t* __restrict__ qx,
                                                                  uint32_t* __restrict__ sc, int64_t rows,
                                                                  int64_t cols, int64_t orows, int64_t ocols,
                                                                  int64_t n_cb, int64_t n_units, bool vec_ok) {
    const int64_t unit = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) >> 4;
    if (unit >= n_units) return;  // whole 16-lane units leave together
    const int l = threadIdx.x & 15;
    const int64_t r = unit / n_cb;
    const int64_t j = unit - r * n_cb;
    const int64_t blk = 4 * j + (l >> 2);
    const int64_t k0 = blk * 32 + (l & 3) * 8;
    const bool live = r < rows && blk < cols / 32;

    float v[8];
    load_row8<IN>(x, r, k0, orows, ocols, vec_ok, v);
    uint32_t m = absmax_bits(v);
    m = max(m, shfl_xor(m, 1));
    m = max(m, shfl_xor(m, 2));
    const uint32_t e = live ? mx_exponent(m) : 0u;

    if (live) *reinterpret_cast<uint2*>(qx + r * cols + k0) = mx_encode8(v, m, e);

    uint32_t word = e << (8 * (l >> 2));
    word |= shfl_xor(word, 4);
    word |= shfl_xor(word, 8);
    if (l == 0) sc[swz_offset(r, 4 * j, n_cb) >> 2] = word;
}

// ------------------------------------------------------- MXFP8, 16-bit fast path
// For bf16/f16 inputs with no column padding (orig shape == padded shape up to the
// 128-row scale padding), cols % 128 == 0, 16-byte aligned, < 2^31 elements.
//
// Same units as above, with every step on packed 16-bit data:
//   * amax: |x| as 16-bit integers, two per register (v_pk_max_u16), then a DPP
//     quad_perm max over the 4 lanes of a block;
//   * codes: v_cvt_scalef32_pk_fp8_{bf16,f16} with scale 2^(e-127) computes
//     E4M3(x / 2^(e-127)) with RNE; it uses the exponent of the scale only and matches
//     the software encoder on every 16-bit input whose quotient lies in [-448, 448]
//     (checked for all 2^16 patterns and every normal power-of-two scale), which is
//     always the case here because 2^(e-127) >= amax/448;
//   * the scale word is OR-combined with two DPP row_ror steps.
// Blocks whose amax is zero, tiny (biased exponent < 10) or non-finite take the
// general encoder.

// Work mapping of the fast kernels.  The swizzled scale words of the units in one
// 128-row tile and one unit column j form a contiguous 512-byte span, but neighbouring
// words belong to rows 32 apart, so units processed in row-major order leave every
// scale line partially written by workgroups on different XCDs (each with its own L2),
// which costs about as much HBM traffic as a full line per word.  Instead a work item
// is one 128-row tile x G unit columns (G = 4 for NVFP4, whose 32-byte code runs need
// 4 units per 128-byte line; 1 for MXFP8), processed by 4 workgroups of 32 rows each
// that run on the same XCD: workgroups are dispatched round-robin over the 8 XCDs
// (XCD = blockIdx % 8), so item i gets workgroups 32*(i/8) + i%8 + 8q, q = 0..3, and
// every scale and code line of the item is written within one XCD.
struct FastItem {
    uint32_t tile, q, cg;  // 128-row tile, 32-row group in it, unit-column group
    bool valid;
};
__device__ __forceinline__ FastItem fast_item(uint32_t n_items, uint32_t n_cg, uint32_t cg_magic, uint32_t cg_shift) {
    const uint32_t b = blockIdx.x, k = b >> 3;
    const uint32_t item = (k >> 2) * 8 + (b & 7);
    FastItem f;
    f.q = k & 3;
    f.tile = static_cast<uint32_t>((static_cast<uint64_t>(item) * cg_magic) >> cg_shift);
    f.cg = item - f.tile * n_cg;
    f.valid = item < n_items;
    return f;
}

constexpr int kMxUnits = 2;  // units per thread: 2 passes of 16 units cover a workgroup's 32 rows

template <int IN>
__global__ __launch_bounds__(kThreads) void quantize_mxfp8_fast_kernel(const uint16_t* __restrict__ x,
                                                                       uint8_t* __restrict__ qx,
                                                                       uint32_t* __restrict__ sc, uint32_t rows,
                                                                       uint32_t cols, uint32_t n_cb,
                                                                       uint32_t n_items, uint32_t cg_magic,
                                                                       uint32_t cg_shift) {
    // item: 128 rows x 1 unit column; this workgroup: 32 rows, 16 per pass
    const FastItem it = fast_item(n_items, n_cb, cg_magic, cg_shift);
    if (!it.valid) return;
    const uint32_t l = threadIdx.x & 15;
    const uint32_t j = it.cg;
    uint4 w[kMxUnits];
    uint32_t r[kMxUnits], off[kMxUnits];
#pragma unroll
    for (int u = 0; u < kMxUnits; ++u) {
        r[u] = it.tile * 128 + it.q * 32 + u * (kThreads / 16) + (threadIdx.x >> 4);
        off[u] = r[u] * cols + 128 * j + 8 * l;
        w[u] = make_uint4(0u, 0u, 0u, 0u);
        if (r[u] < rows) w[u] = ld_stream16(x + off[u]);
    }
#pragma unroll
    for (int u = 0; u < kMxUnits; ++u) {
        uint32_t m = amax16x8(w[u]);
        m = max(m, dpp<0xB1>(m));  // quad_perm [1,0,3,2]
        m = max(m, dpp<0x4E>(m));  // quad_perm [2,3,0,1]
        const uint32_t bits = amax16_to_f32_bits<IN>(m);
        uint32_t e;
        const uint2 codes = mx_codes16<IN>(w[u], bits, e);
        if (r[u] < rows) *reinterpret_cast<uint2*>(qx + off[u]) = codes;
        uint32_t word = e << (8 * (l >> 2));
        word |= dpp<0x124>(word);  // row_ror:4
        word |= dpp<0x128>(word);  // row_ror:8
        if (l == 0) sc[((it.tile * n_cb + j) * 32 + (r[u] & 31)) * 4 + it.q] = word;
    }
}

// ------------------------------------------------------------------- NVFP4
// Per 16-element block (reference eager quantization.py:137-158):
//   s8 = E4M3(min(amax/6/g, 448)); T = g*s8; codes = E2M1(clamp(x/T, +-6)), T==0 -> +0.
// Divisions are IEEE fp32 divisions, as in the reference's eager path.

// NaN blocks: E2M1 has no NaN code, so the reference's codes for NaN data depend on the
// NaN's bits as its CPU arithmetic (x86 SSE) propagates them: a NaN operand is returned
// quieted (the first one if both are NaN) and an invalid operation without NaN operands
// (inf*0, inf/inf) returns the default NaN 0xFFC00000; torch converts the E4M3 NaN
// codes to 0x7FF00000 | sign.  The functions below reproduce those bits.
__device__ __forceinline__ float x86_nan(float r, float a, float b) {
    if (!is_nan(r)) return r;
    if (is_nan(a)) return as_f(as_u(a) | 0x00400000u);
    if (is_nan(b)) return as_f(as_u(b) | 0x00400000u);
    return as_f(0xffc00000u);
}

// T = g * float(s8) with the reference's NaN bits
__device__ __forceinline__ float nvfp4_total(float g, uint32_t s8) {
    const float s = (s8 & 0x7fu) == 0x7fu ? as_f(0x7ff00000u | ((s8 & 0x80u) << 24)) : hw_e4m3_to_f<0>(s8);
    return x86_nan(g * s, g, s);
}

// Codes of 8 values for a block with T != 0, by IEEE division (any T, any input).
template <bool HI_FIRST>
__device__ __forceinline__ uint32_t nvfp4_codes8_div(const float* v, float T) {
    float q[8];
    bool any_nan = false;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        q[t] = __builtin_amdgcn_fmed3f(v[t] / T, -6.0f, 6.0f);
        any_nan |= is_nan(v[t] / T);
    }
    if (!any_nan) return pack_e2m1x8<HI_FIRST>(q);
    // software codes keep the reference's NaN behaviour
    uint32_t codes[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        float qq = x86_nan(v[t] / T, v[t], T);
        qq = qq > 6.0f ? 6.0f : (qq < -6.0f ? -6.0f : qq);  // fp32 clamp returns a NaN unchanged
        codes[t] = f_to_e2m1(qq);
    }
    uint32_t w = 0;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        uint32_t b = HI_FIRST ? ((codes[2 * p] << 4) | codes[2 * p + 1]) : ((codes[2 * p + 1] << 4) | codes[2 * p]);
        w |= b << (8 * p);
    }
    return w;
}

// Out-of-line form for the fast kernel, which needs it only for rare blocks (values
// passed in registers, so the call uses no scratch memory).
template <bool HI_FIRST>
__device__ __noinline__ uint32_t nvfp4_codes8_div_rare(float v0, float v1, float v2, float v3, float v4, float v5,
                                                       float v6, float v7, float T) {
    const float v[8] = {v0, v1, v2, v3, v4, v5, v6, v7};
    return nvfp4_codes8_div<HI_FIRST>(v, T);
}

// Block scale code s8 from the block amax and the global scale (IEEE divisions).
// A NaN c keeps the sign the reference's fp32 ops give it (x86_nan): the amax (a |x|) NaN
// is positive and division returns its first NaN operand, so NaN amax -> 0x7F; else a
// NaN g passes its sign; else c is NaN from an invalid division (0/0 for an all-zero
// block with g = 0, inf/inf), the default NaN 0xFFC00000 -> 0xFF.  fp32 clamp(max=448)
// returns the NaN unchanged.
__device__ __forceinline__ uint32_t nvfp4_scale_code_of(float c, float amax, float g) {
    c = c > 448.0f ? 448.0f : c;  // NaN passes through, as torch.clamp
    if (is_nan(c)) return 0x7fu | (is_nan(amax) ? 0u : is_nan(g) ? ((as_u(g) >> 24) & 0x80u) : 0x80u);
    // 0 <= c <= 448 here (c < 0 only for g < 0, and clamp keeps it): the hardware
    // E4M3 convert is exact on [-448, 448]
    return hw_e4m3x4(c, 0.0f, 0.0f, 0.0f) & 0xffu;
}
__device__ __forceinline__ uint32_t nvfp4_scale_code(float amax, float g) {
    return nvfp4_scale_code_of((amax / 6.0f) / g, amax, g);
}
// (amax / 6) / g out of line, for the fast kernel's rare blocks (inline, the compiler
// if-converts it and executes both divisions on every block)
__device__ __noinline__ float nvfp4_c_div_rare(float amax, float g) { return (amax / 6.0f) / g; }

template <int IN, bool HI_FIRST>
__global__ __launch_bounds__(kThreads) void quantize_nvfp4_kernel(const void* __restrict__ x,
                                                                  const float* __restrict__ gptr,
                                                                  uint8_t* __restrict__ qx,
                                                                  uint32_t* __restrict__ sc, int64_t rows,
                                                                  int64_t cols, int64_t orows, int64_t ocols,
                                                                  int64_t n_cb, int64_t n_units, bool vec_ok) {
    const int64_t unit = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) >> 3;
    if (unit >= n_units) return;  // whole 8-lane units leave together
    const int l = threadIdx.x & 7;
    const int64_t r = unit / n_cb;
    const int64_t j = unit - r * n_cb;
    const int64_t blk = 4 * j + (l >> 1);
    const int64_t k0 = blk * 16 + (l & 1) * 8;
    const bool live = r < rows && blk < cols / 16;
    const float g = gptr[0];

    float v[8];
    load_row8<IN>(x, r, k0, orows, ocols, vec_ok, v);
    uint32_t m = absmax_bits(v);
    m = max(m, shfl_xor(m, 1));

    const uint32_t s8 = live ? nvfp4_scale_code(as_f(m), g) : 0u;
    const float T = nvfp4_total(g, s8);
    if (live) *reinterpret_cast<uint32_t*>(qx + r * (cols / 2) + k0 / 2) = T != 0.0f ? nvfp4_codes8_div<HI_FIRST>(v, T) : 0u;

    uint32_t word = s8 << (8 * (l >> 1));
    word |= shfl_xor(word, 2);
    word |= shfl_xor(word, 4);
    if (l == 0) sc[swz_offset(r, 4 * j, n_cb) >> 2] = word;
}

// ------------------------------------------------------- NVFP4, 16-bit fast path
// For bf16/f16 inputs with no column padding, cols % 64 == 0, 16-byte aligned, < 2^31
// elements.  One lane per 16-element block, four lanes per unit (one scale word), two
// units per thread.  A lane's block is two 16-byte chunks that another lane's loads
// share (nv_pair_exchange), so that each load instruction reads one contiguous KB
// rather than every other 16 bytes of 2 KB (which measured 6% slower).  The IEEE
// divisions of the reference are replaced by Markstein correction steps, each exact:
//   c = (amax / 6) / g:  c0 = amax*y6, c1 = fma(-fma(6, c0, -amax), y6, c0), then the
//                        same step with y_g = RN(1/g) (one IEEE division per thread);
//                        bit-identical to the two IEEE divisions for every bf16 / f16
//                        amax significand and every g significand, checked exhaustively;
//   q = v / T:           y = RN(1/T) (one IEEE division per block), q0 = v*y,
//                        e = fma(T, q0, -v), q = fma(-e, y, q0); the E2M1 code of q
//                        equals that of the IEEE quotient for every bf16 and f16 v
//                        (both signs, and +-0) and every T significand: checked
//                        exhaustively for T in [1, 2) and v in [2^-6, 2^5), which covers
//                        every code boundary, as (v*y alone gets 516 bf16 and 3904 f16
//                        codes wrong).  The negated residual keeps the sign of a zero v.
// The steps scale exactly by powers of two while every intermediate stays normal and
// finite, which the guards ensure: g and amax within [2^-60, 2^60] for the scale, and
// for the codes c <= 448 (so |v/T| < 10) and T within [2^-120, 2^120]; other blocks use
// the IEEE divisions.  The E2M1 convert saturates out-of-range inputs to +-6 exactly as
// the reference's clamp (checked on all 2^32 non-NaN floats), so no clamp is needed.
// Codes of a 16-element block by the exact division steps above (the guards hold).
// RCP: y from v_rcp_f32 and one FMA Newton step, which equals the IEEE 1.0f / T for
// every T in [2^-70, 2^71) (checked exhaustively on gfx950), covering the common-block
// range T in [2^-69, 2^69]; otherwise an IEEE division.
template <bool HI_FIRST, bool RCP = false>
__device__ __forceinline__ uint2 nvfp4_codes16_exact(const float (&v)[16], float T) {
    float y;
    if constexpr (RCP) y = rcp_newton(T);
    else y = 1.0f / T;
    float q[16];
#pragma unroll
    for (int t = 0; t < 16; ++t) q[t] = markstein_quotient(v[t], T, y);
    return make_uint2(pack_e2m1x8<HI_FIRST>(&q[0]), pack_e2m1x8<HI_FIRST>(&q[8]));
}

// Lanes t and t + 4 of a wave (bit 2 of t clear: "low", set: "high") load the two 16-byte
// halves of a pair of blocks A and B: the low lane the first halves (P = A0, Q = B0), the
// high lane the second (P = A1, Q = B1).  After the exchange the low lane holds block A
// (A0, A1) and the high lane block B (B0, B1).  DPP rows are 16 lanes; bank_mask selects
// the 4-lane banks written (0x5: banks 0, 2 = low lanes; 0xA: banks 1, 3 = high lanes).
__device__ __forceinline__ void nv_pair_exchange(uint4& P, uint4& Q) {
    auto lo_half = [](uint32_t p, uint32_t q) {  // high lanes: q of lane t - 4 (row_shr:4)
        return static_cast<uint32_t>(
            __builtin_amdgcn_update_dpp(static_cast<int>(p), static_cast<int>(q), 0x114, 0xf, 0xa, false));
    };
    auto hi_half = [](uint32_t q, uint32_t p) {  // low lanes: p of lane t + 4 (row_shl:4)
        return static_cast<uint32_t>(
            __builtin_amdgcn_update_dpp(static_cast<int>(q), static_cast<int>(p), 0x104, 0xf, 0x5, false));
    };
    const uint4 a = P, b = Q;
    P = make_uint4(lo_half(a.x, b.x), lo_half(a.y, b.y), lo_half(a.z, b.z), lo_half(a.w, b.w));
    Q = make_uint4(hi_half(b.x, a.x), hi_half(b.y, a.y), hi_half(b.z, a.z), hi_half(b.w, a.w));
}

constexpr int kNvUnits = 2;  // units per thread: 2 passes cover a workgroup's 32 rows x G units

// G = unit columns per item (4 or 16); the workgroup has 64*G threads.  A wave's 16
// units in one pass are 16/G rows x G consecutive units, so with G = 16 each load
// instruction reads 2 KB of one row.
// DYN: the global scale is not an input but the layouts' default, amax(|x|) / divisor,
// formed by every workgroup from the `nparts` partial maxima that amax_partials wrote for
// this x (scale_from_partial_words); workgroup 0 stores it to *scale_out.  The partial
// words are loaded before the x data, so that reduction runs while the data loads are in
// flight (measured: 35.4 -> 33.7 us on C5 against waiting for both).
template <int IN, bool HI_FIRST, int G, bool DYN>
__global__ __launch_bounds__(64 * G) void quantize_nvfp4_fast_kernel(const uint16_t* __restrict__ x,
                                                                     const float* __restrict__ gptr,
                                                                     uint8_t* __restrict__ qx,
                                                                     uint32_t* __restrict__ sc, uint32_t rows,
                                                                     uint32_t cols, uint32_t n_cb, uint32_t n_items,
                                                                     uint32_t n_cg, uint32_t cg_magic,
                                                                     uint32_t cg_shift,
                                                                     const uint32_t* __restrict__ partial,
                                                                     uint32_t nparts, float inv_divisor,
                                                                     float* __restrict__ scale_out) {
    // item: 128 rows x G unit columns.  This workgroup: rows 8q..8q+7 of each of the
    // tile's four 32-row groups (32 rows) x G units.  Its scale words of one unit column
    // are then 32 consecutive words (one 128-byte line): staged in LDS and stored as
    // whole lines.
    constexpr uint32_t kUnitsPerPass = 16 * G;
    const FastItem it = fast_item(n_items, n_cg, cg_magic, cg_shift);
    if (!it.valid) return;
    __shared__ uint32_t sw[G * 32];
    const uint32_t l = threadIdx.x & 3;
    uint4 w[kNvUnits][2];
    uint32_t r[kNvUnits], off[kNvUnits], j[kNvUnits], ul[kNvUnits];
    // DYN: the partial words first, then the data through a descriptor over this tile's
    // rows (no conditional loads, so the wait for the partial words before the scale
    // reduction leaves the data loads in flight)
    PartialWords<64 * G> pw;
    if constexpr (DYN) pw = load_partial_words<64 * G>(partial, nparts);
    const uint32_t row0 = it.tile * 128;
    __amdgpu_buffer_rsrc_t xrs;
    if constexpr (DYN)
        xrs = buffer_rsrc(x + static_cast<size_t>(row0) * cols, min(rows - row0, 128u) * cols * 2u);
#pragma unroll
    for (int u = 0; u < kNvUnits; ++u) {
        // The wave's 16 units (2 KB): A block k is block k of its first KB, B block k of
        // its second, and lanes t, t + 4 with k = 4 (t / 8) + t % 4 share them
        // (nv_pair_exchange).  Each load instruction then reads one contiguous KB.
        const uint32_t t = threadIdx.x & 63, hi = (t >> 2) & 1, k = 4 * (t >> 3) + (t & 3);
        const uint32_t wb = u * kUnitsPerPass + (threadIdx.x >> 6) * 16;
        ul[u] = wb + 8 * hi + (t >> 3);  // unit in the workgroup of the lane's own block
        uint32_t rr[2], jj[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t uu = wb + 8 * h + (k >> 2);  // unit of A (h = 0) / B (h = 1) block k
            const uint32_t rs = uu / G;                 // row slot: 8 rows x 4 groups
            rr[h] = it.tile * 128 + (rs & 3) * 32 + it.q * 8 + (rs >> 2);
            jj[h] = it.cg * G + uu % G;
        }
        r[u] = rr[hi];
        j[u] = jj[hi];
        off[u] = r[u] * cols + 64 * j[u] + 16 * l;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t e = 64 * jj[h] + 16 * (k & 3) + 8 * hi;  // element in the row
            if constexpr (DYN) {
                // rows past the end lie outside the descriptor, units past n_cb are sent there
                const uint32_t bo = jj[h] < n_cb ? ((rr[h] - row0) * cols + e) * 2u : 0x80000000u;
                const auto v = __builtin_amdgcn_raw_buffer_load_b128(xrs, bo, 0, 2);  // aux 2: nontemporal
                w[u][h] = make_uint4(v[0], v[1], v[2], v[3]);
            } else {
                // (plain global loads measured 3.5% faster here than the buffer form)
                w[u][h] = make_uint4(0u, 0u, 0u, 0u);
                if (rr[h] < rows && jj[h] < n_cb) w[u][h] = ld_stream16(x + rr[h] * cols + e);
            }
        }
    }
    float g;
    if constexpr (DYN) {
        __shared__ uint32_t red[G];
        g = scale_from_partial_words<IN, 64 * G>(pw, inv_divisor, red);
        if (blockIdx.x == 0 && threadIdx.x == 0) *scale_out = g;
    } else {
        g = gptr[0];
    }
    const bool g_ok = g >= 0x1p-60f && g <= 0x1p60f;  // false for NaN
    // RN(1/g) by rcp + one Newton step: equal to the IEEE division for every g in
    // [2^-70, 2^71), and yg is only used when g_ok
    const float yg = rcp_newton(g);
#pragma unroll
    for (int u = 0; u < kNvUnits; ++u) {
        nv_pair_exchange(w[u][0], w[u][1]);  // now the lane's own block
        const float amax = as_f(amax16_to_f32_bits<IN>(max(amax16x8(w[u][0]), amax16x8(w[u][1]))));
        // the scale by the exact steps (valid when g and amax are within [2^-60, 2^60])
        const float cf = nvfp4_c_steps(amax, g, yg);
        const uint32_t s8f = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(cf, 0.0f, 0, false)) & 0xffu;
        float v[16];
        unpack16x8<IN>(w[u][0], *reinterpret_cast<float(*)[8]>(&v[0]));
        unpack16x8<IN>(w[u][1], *reinterpret_cast<float(*)[8]>(&v[8]));
        uint32_t s8;
        uint2 codes = make_uint2(0u, 0u);
        // Common blocks: 0 < c <= 448 and s8 != 0, so s8 is the convert of c (no clamp,
        // no NaN), T = g * s8 lies in [2^-69, 2^69] and the exact division steps apply.
        // A row past the end has amax 0 and takes the general path.
        if (g_ok && amax >= 0x1p-60f && amax <= 0x1p60f && cf <= 448.0f && s8f != 0u) {
            s8 = s8f;
            codes = nvfp4_codes16_exact<HI_FIRST, true>(v, g * hw_e4m3_to_f<0>(s8f));
        } else {
            const float c = g_ok && amax >= 0x1p-60f && amax <= 0x1p60f ? cf : nvfp4_c_div_rare(amax, g);
            s8 = r[u] < rows ? nvfp4_scale_code_of(c, amax, g) : 0u;
            const float T = nvfp4_total(g, s8);
            if (T != 0.0f) {
                if (c <= 448.0f && T >= 0x1p-120f && T <= 0x1p120f) {
                    codes = nvfp4_codes16_exact<HI_FIRST>(v, T);
                } else {
                    codes = make_uint2(
                        nvfp4_codes8_div_rare<HI_FIRST>(v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7], T),
                        nvfp4_codes8_div_rare<HI_FIRST>(v[8], v[9], v[10], v[11], v[12], v[13], v[14], v[15], T));
                }
            }
        }
        if (r[u] < rows && j[u] < n_cb) st_stream8(qx + off[u] / 2, codes);
        uint32_t word = s8 << (8 * l);
        word |= dpp<0xB1>(word);  // quad_perm [1,0,3,2]
        word |= dpp<0x4E>(word);  // quad_perm [2,3,0,1]
        // Word (r, j) of the tensor sits at ((tile*n_cb + j)*32 + (r & 31))*4 + (r & 127)/32.
        // The workgroup stages the words of unit column j % G as one 32-word line, in which
        // row r is word ((r & 31) - 8 q) * 4 + (r & 127) / 32, i.e. its row slot ul / G.
        if (l == 0) sw[(ul[u] % G) * 32 + ul[u] / G] = word;
    }
    __syncthreads();
    if (threadIdx.x < 8 * G) {
        const uint32_t jj = threadIdx.x >> 3, part = threadIdx.x & 7, jc = it.cg * G + jj;
        if (jc < n_cb) {
            const uint4 v = *reinterpret_cast<const uint4*>(&sw[jj * 32 + part * 4]);
            st_stream16(sc + (it.tile * n_cb + jc) * 128 + it.q * 32 + part * 4, v);
        }
    }
}

// -------------------------------------------------------------- dequantize
template <int OUT>
__device__ __forceinline__ void store8(void* out, int64_t i, const float (&v)[8]) {
    if constexpr (OUT == CKH_F32) {
        float4* p = reinterpret_cast<float4*>(static_cast<float*>(out) + i);
        p[0] = make_float4(v[0], v[1], v[2], v[3]);
        p[1] = make_float4(v[4], v[5], v[6], v[7]);
    } else {
        uint32_t w[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            uint32_t lo = OUT == CKH_BF16 ? f_to_bf16(v[2 * q]) : f_to_f16(v[2 * q]);
            uint32_t hi = OUT == CKH_BF16 ? f_to_bf16(v[2 * q + 1]) : f_to_f16(v[2 * q + 1]);
            w[q] = lo | (hi << 16);
        }
        *reinterpret_cast<uint4*>(static_cast<uint16_t*>(out) + i) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

// MXFP8 dequantize (reference eager quantization.py:342-364):
//   out = (float(q) * 2^(e-127)).to(out), e == 0 -> scale 0.0.
// One thread per 8 elements of one 32-block.
template <int OUT>
__global__ __launch_bounds__(kThreads) void dequantize_mxfp8_kernel(const uint8_t* __restrict__ qx,
                                                                    const uint8_t* __restrict__ sc,
                                                                    void* __restrict__ out, int64_t rows,
                                                                    int64_t cols, int64_t n_cb) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    const int64_t per_row = cols / 8;
    if (t >= rows * per_row) return;
    const int64_t r = t / per_row;
    const int64_t k0 = (t - r * per_row) * 8;
    const float s = e8m0_to_f(sc[swz_offset(r, k0 / 32, n_cb)]);
    const uint2 c = *reinterpret_cast<const uint2*>(qx + r * cols + k0);
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = e4m3_to_f(((i < 4 ? c.x : c.y) >> (8 * (i & 3))) & 0xffu) * s;
    store8<OUT>(out, r * cols + k0, v);
}

// NVFP4 dequantize (reference eager quantization.py:178-219): every step is rounded to
// the output dtype: total = round(round(g) * s8); out = round(E2M1(c) * total).
template <int OUT>
__global__ __launch_bounds__(kThreads) void dequantize_nvfp4_kernel(const uint8_t* __restrict__ qx,
                                                                    const float* __restrict__ gptr,
                                                                    const uint8_t* __restrict__ sc,
                                                                    void* __restrict__ out, int64_t rows,
                                                                    int64_t cols, int64_t n_cb, bool hi_first) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    const int64_t per_row = cols / 8;
    if (t >= rows * per_row) return;
    const int64_t r = t / per_row;
    const int64_t k0 = (t - r * per_row) * 8;
    const float total = round_to<OUT>(round_to<OUT>(gptr[0]) * e4m3_to_f(sc[swz_offset(r, k0 / 16, n_cb)]));
    const uint32_t w = *reinterpret_cast<const uint32_t*>(qx + r * (cols / 2) + k0 / 2);
    float v[8];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        uint32_t b = (w >> (8 * p)) & 0xffu;
        uint32_t c0 = hi_first ? (b >> 4) : (b & 15u);
        uint32_t c1 = hi_first ? (b & 15u) : (b >> 4);
        v[2 * p] = round_to<OUT>(e2m1_to_f(c0) * total);
        v[2 * p + 1] = round_to<OUT>(e2m1_to_f(c1) * total);
    }
    store8<OUT>(out, r * cols + k0, v);
}

// ------------------------------------------------- block dequantize, fast paths
// 16-bit outputs, 8-byte (MXFP8) / 4-byte (NVFP4) aligned codes, cols % 8 == 0 and fewer
// than 2^31 pieces of 8 elements.  A wave handles 256 consecutive pieces, 4 per lane,
// piece p of lane l being the wave's piece 64 p + l, so every load and store instruction
// covers one contiguous run (512 or 256 bytes of codes, 1 KB of output); all of a lane's
// loads are issued before any is used.  The index math is 32-bit with a multiply-shift
// division by the pieces per row.  The arithmetic is the general kernels' (the hardware
// converts equal the software decoders on every code and on every non-NaN bf16 rounding);
// a piece whose values hold a NaN converts them to bf16 out of line in software, keeping
// its NaN bits.
// pieces of 8 elements per lane (same-process sweeps of 1, 2, 4 and 8 on C3 / C5: MXFP8
// - / 9.8 / 8.6 / 11.5 us, NVFP4 24.5 / 23.6 / 24.7 / 27.1 us)
constexpr int kDqPiecesMx = 4;
constexpr int kDqPiecesNv = 2;

// Workgroup b runs on XCD b % 8.  Give XCD x a contiguous range of the grid's pieces, so
// the rows whose swizzled scale words share a 128-byte line (32 rows of a 128-row tile)
// are read through one L2 instead of up to eight (MXFP8 dequantize, C3: 8.49 -> 8.23 us).
__device__ __forceinline__ uint32_t xcd_block() {
    const uint32_t b = blockIdx.x, n = gridDim.x, x = b & 7u, q = n >> 3, rem = n & 7u;
    return x * q + min(x, rem) + (b >> 3);
}

// row of piece t (t < 2^31) by multiply-shift
__device__ __forceinline__ uint32_t piece_row(uint32_t t, uint32_t magic, uint32_t shift) {
    return static_cast<uint32_t>((static_cast<uint64_t>(t) * magic) >> shift);
}

__device__ __noinline__ uint4 bf16x8_soft(float v0, float v1, float v2, float v3, float v4, float v5, float v6,
                                         float v7) {
    return make_uint4(f_to_bf16(v0) | (f_to_bf16(v1) << 16), f_to_bf16(v2) | (f_to_bf16(v3) << 16),
                      f_to_bf16(v4) | (f_to_bf16(v5) << 16), f_to_bf16(v6) | (f_to_bf16(v7) << 16));
}

// 8 values -> 8 packed 16-bit outputs, stored with one 16-byte nontemporal store;
// maybe_nan: some value may be a NaN (then bf16 goes through the software convert)
template <int OUT>
__device__ __forceinline__ void store8_fast(uint16_t* o, const float (&v)[8], bool maybe_nan) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if constexpr (OUT == CKH_BF16) w[i] = f_to_bf16_rne(v[2 * i]) | (f_to_bf16_rne(v[2 * i + 1]) << 16);
        else w[i] = f_to_f16(v[2 * i]) | (f_to_f16(v[2 * i + 1]) << 16);
    }
    uint4 d = make_uint4(w[0], w[1], w[2], w[3]);
    if (OUT == CKH_BF16 && maybe_nan) d = bf16x8_soft(v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7]);
    st_stream16(o, d);
}

// some byte of w is an E4M3 NaN code (0x7F or 0xFF)
__device__ __forceinline__ bool has_e4m3_nan(uint32_t w) {
    return (((w & 0x7f7f7f7fu) + 0x01010101u) & 0x80808080u) != 0u;
}

template <int OUT>
__global__ __launch_bounds__(kThreads) void dequantize_mxfp8_fast_kernel(const uint8_t* __restrict__ qx,
                                                                         const uint8_t* __restrict__ sc,
                                                                         uint16_t* __restrict__ out, uint32_t n_pieces,
                                                                         uint32_t per_row, uint32_t magic,
                                                                         uint32_t shift, uint32_t n_cb) {
    const uint32_t base = (xcd_block() * kThreads + (threadIdx.x & ~63u)) * kDqPiecesMx + (threadIdx.x & 63u);
    uint2 c[kDqPiecesMx];
    float s[kDqPiecesMx];
#pragma unroll
    for (int p = 0; p < kDqPiecesMx; ++p) {
        const uint32_t t = base + 64 * p;
        c[p] = make_uint2(0u, 0u);
        s[p] = 0.0f;
        if (t < n_pieces) {
            typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
            const u32x2 w = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(qx) + t);
            c[p] = make_uint2(w.x, w.y);
            const uint32_t r = piece_row(t, magic, shift), blk = (t - r * per_row) >> 2;  // 32-block of the row
            s[p] = e8m0_to_f(sc[(((r >> 7) * n_cb + (blk >> 2)) * 32 + (r & 31)) * 16 + ((r & 127) >> 5) * 4 + (blk & 3)]);
        }
    }
#pragma unroll
    for (int p = 0; p < kDqPiecesMx; ++p) {
        const uint32_t t = base + 64 * p;
        if (t >= n_pieces) break;
        float v[8];
        v[0] = hw_e4m3_to_f<0>(c[p].x) * s[p];
        v[1] = hw_e4m3_to_f<1>(c[p].x) * s[p];
        v[2] = hw_e4m3_to_f<2>(c[p].x) * s[p];
        v[3] = hw_e4m3_to_f<3>(c[p].x) * s[p];
        v[4] = hw_e4m3_to_f<0>(c[p].y) * s[p];
        v[5] = hw_e4m3_to_f<1>(c[p].y) * s[p];
        v[6] = hw_e4m3_to_f<2>(c[p].y) * s[p];
        v[7] = hw_e4m3_to_f<3>(c[p].y) * s[p];
        // NaN only from a NaN code, or from 0 * inf (scale byte 255)
        const bool maybe_nan = has_e4m3_nan(c[p].x) || has_e4m3_nan(c[p].y) || s[p] == __builtin_inff();
        store8_fast<OUT>(out + static_cast<size_t>(t) * 8, v, maybe_nan);
    }
}

// the two elements of byte B of w times T (in fp32; exact), low nibble first from the convert
template <bool HI_FIRST, int B>
__device__ __forceinline__ void nvfp4_pair(uint32_t w, float T, float* v) {
    const auto e = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, B);
    const float lo = e[0], hi = e[1];
    v[0] = (HI_FIRST ? hi : lo) * T;
    v[1] = (HI_FIRST ? lo : hi) * T;
}

template <int OUT, bool HI_FIRST>
__global__ __launch_bounds__(kThreads) void dequantize_nvfp4_fast_kernel(const uint8_t* __restrict__ qx,
                                                                         const float* __restrict__ gptr,
                                                                         const uint8_t* __restrict__ sc,
                                                                         uint16_t* __restrict__ out, uint32_t n_pieces,
                                                                         uint32_t per_row, uint32_t magic,
                                                                         uint32_t shift, uint32_t n_cb) {
    // blocks in grid order: the XCD-contiguous order of the MXFP8 kernel measured 9% slower
    // here (25.8 vs 23.8 us on C5), whose output writes are 4x its reads
    const uint32_t base = (blockIdx.x * kThreads + (threadIdx.x & ~63u)) * kDqPiecesNv + (threadIdx.x & 63u);
    const float gr = round_to_hw<OUT>(gptr[0]);
    uint32_t c[kDqPiecesNv], s8[kDqPiecesNv];
#pragma unroll
    for (int p = 0; p < kDqPiecesNv; ++p) {
        const uint32_t t = base + 64 * p;
        c[p] = 0u;
        s8[p] = 0u;
        if (t < n_pieces) {
            c[p] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(qx) + t);
            const uint32_t r = piece_row(t, magic, shift), blk = (t - r * per_row) >> 1;  // 16-block of the row
            s8[p] = sc[(((r >> 7) * n_cb + (blk >> 2)) * 32 + (r & 31)) * 16 + ((r & 127) >> 5) * 4 + (blk & 3)];
        }
    }
#pragma unroll
    for (int p = 0; p < kDqPiecesNv; ++p) {
        const uint32_t t = base + 64 * p;
        if (t >= n_pieces) break;
        // every step rounded to the output dtype, as the general kernel: total =
        // round(round(g) * s8), out = round(E2M1(c) * total), the last rounding being the
        // store's conversion
        // the hardware decode and rounding equal the software ones except for NaN payloads
        const float T = round_to_hw<OUT>(gr * hw_e4m3_to_f<0>(s8[p]));
        float v[8];
        nvfp4_pair<HI_FIRST, 0>(c[p], T, &v[0]);
        nvfp4_pair<HI_FIRST, 1>(c[p], T, &v[2]);
        nvfp4_pair<HI_FIRST, 2>(c[p], T, &v[4]);
        nvfp4_pair<HI_FIRST, 3>(c[p], T, &v[6]);
        // E2M1 values are finite: a NaN only from a NaN total, or from 0 * inf
        store8_fast<OUT>(out + static_cast<size_t>(t) * 8, v, !(__builtin_fabsf(T) < __builtin_inff()));
    }
}

// NVFP4 dequantize for cols % 256 == 0: a 512-thread workgroup takes the 32 rows whose
// swizzled scale words share 128-byte lines (rows 8q..8q+7 of each 32-row group of a
// 128-row tile) x 256 columns, so each scale line is read by one workgroup.  Wave
// (w, h) takes rows 32w + 8q + 4h .. +3; lane l's piece p is piece 32 (2p + l/32) + l%32
// of those 4 rows x 32 pieces, so each code load covers whole 128-byte row runs and each
// store whole 512-byte row runs.
template <int OUT, bool HI_FIRST>
__global__ __launch_bounds__(512) void dequantize_nvfp4_tile_kernel(const uint8_t* __restrict__ qx,
                                                                    const float* __restrict__ gptr,
                                                                    const uint8_t* __restrict__ sc,
                                                                    uint16_t* __restrict__ out, uint32_t rows,
                                                                    uint32_t cols, uint32_t n_ct, uint32_t n_cb) {
    const uint32_t b = blockIdx.x;
    const uint32_t ct = b % n_ct, slice = b / n_ct;  // column tile; (128-row tile, q)
    const uint32_t tile = slice >> 2, q = slice & 3;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint32_t w = wave >> 1, h = wave & 1;
    const float gr = round_to_hw<OUT>(gptr[0]);
    uint32_t c[2], s8[2], r[2], cp[2];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        r[p] = tile * 128 + 32 * w + 8 * q + 4 * h + 2 * p + (lane >> 5);
        cp[p] = ct * 32 + (lane & 31);  // 8-element piece of the row
        c[p] = 0u;
        s8[p] = 0u;
        if (r[p] < rows) {
            c[p] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(qx + static_cast<size_t>(r[p]) * (cols / 2)) + cp[p]);
            const uint32_t blk = cp[p] >> 1;
            s8[p] = sc[(((r[p] >> 7) * n_cb + (blk >> 2)) * 32 + (r[p] & 31)) * 16 + ((r[p] & 127) >> 5) * 4 + (blk & 3)];
        }
    }
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        if (r[p] >= rows) continue;
        const float T = round_to_hw<OUT>(gr * hw_e4m3_to_f<0>(s8[p]));
        float v[8];
        nvfp4_pair<HI_FIRST, 0>(c[p], T, &v[0]);
        nvfp4_pair<HI_FIRST, 1>(c[p], T, &v[2]);
        nvfp4_pair<HI_FIRST, 2>(c[p], T, &v[4]);
        nvfp4_pair<HI_FIRST, 3>(c[p], T, &v[6]);
        store8_fast<OUT>(out + static_cast<size_t>(r[p]) * cols + static_cast<size_t>(cp[p]) * 8, v,
                         !(__builtin_fabsf(T) < __builtin_inff()));
    }
}

}  // namespace ckh

using namespace ckh;

// Multiply-shift for unit / d with 0 <= unit < 2^31 (Granlund-Montgomery):
// l = ceil(log2 d), magic = ceil(2^(31+l) / d) < 2^32, unit / d = (unit * magic) >> (31+l).
static void magic_div(int64_t d, uint32_t& magic, uint32_t& shift) {
    uint32_t lg = 0;
    while ((int64_t(1) << lg) < d) ++lg;
    magic = static_cast<uint32_t>(((uint64_t(1) << (31 + lg)) + d - 1) / d);
    shift = 31 + lg;
}

extern "C" int ckh_quantize_mxfp8(const void* x, void* qx, void* scales, int64_t rows, int64_t cols,
                                  int64_t orig_rows, int64_t orig_cols, int in_code, uintptr_t stream) {
    CKH_REQUIRE(x && qx && scales, "quantize_mxfp8: null pointer");
    CKH_REQUIRE(rows >= orig_rows && cols >= orig_cols && orig_rows >= 0 && orig_cols >= 0,
                "quantize_mxfp8: padded shape [%lld, %lld] smaller than input [%lld, %lld]", (long long)rows,
                (long long)cols, (long long)orig_rows, (long long)orig_cols);
    CKH_REQUIRE(cols % 32 == 0, "quantize_mxfp8: cols (%lld) must be a multiple of 32", (long long)cols);
    CKH_REQUIRE(in_code == CKH_F32 || in_code == CKH_F16 || in_code == CKH_BF16,
                "quantize_mxfp8: unsupported input dtype code %d", in_code);
    CKH_REQUIRE(aligned(qx, 8) && aligned(scales, 4), "quantize_mxfp8: output pointers misaligned");
    if (rows == 0 || cols == 0) return CKH_OK;
    const int64_t n_cb = cdiv(cols / 32, 4);
    const int64_t n_units = rup(rows, 128) * n_cb;
    const bool vec_ok = aligned(x, 16) && orig_cols % 8 == 0;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    uint8_t* q = static_cast<uint8_t*>(qx);
    uint32_t* s = static_cast<uint32_t*>(scales);
    if ((in_code == CKH_BF16 || in_code == CKH_F16) && rows == orig_rows && cols == orig_cols && cols % 128 == 0 &&
        aligned(x, 16) && rup(rows, 128) * cols < (int64_t(1) << 31)) {
        // items: 128-row tiles x unit columns (one unit each), 4 workgroups per item
        const int64_t n_items = cdiv(rows, 128) * n_cb;
        uint32_t magic, shift;
        magic_div(n_cb, magic, shift);
        dim3 fgrid(static_cast<unsigned>(cdiv(n_items, 8) * 32));
        const uint16_t* xx = static_cast<const uint16_t*>(x);
        const auto r32 = static_cast<uint32_t>(rows), c32 = static_cast<uint32_t>(cols),
                   n32 = static_cast<uint32_t>(n_cb), i32 = static_cast<uint32_t>(n_items);
        if (in_code == CKH_BF16)
            hipLaunchKernelGGL((quantize_mxfp8_fast_kernel<CKH_BF16>), fgrid, dim3(kThreads), 0, st, xx, q, s, r32,
                               c32, n32, i32, magic, shift);
        else
            hipLaunchKernelGGL((quantize_mxfp8_fast_kernel<CKH_F16>), fgrid, dim3(kThreads), 0, st, xx, q, s, r32,
                               c32, n32, i32, magic, shift);
        return check_launch("quantize_mxfp8");
    }
    dim3 grid(static_cast<unsigned>(cdiv(n_units * 16, kThreads)));
#define LAUNCH(I)                                                                                                 \
    hipLaunchKernelGGL((quantize_mxfp8_kernel<I>), grid, dim3(kThreads), 0, st, x, q, s, rows, cols, orig_rows, \
                       orig_cols, n_cb, n_units, vec_ok)
    if (in_code == CKH_F32) LAUNCH(CKH_F32);
    else if (in_code == CKH_F16) LAUNCH(CKH_F16);
    else LAUNCH(CKH_BF16);
#undef LAUNCH
    return check_launch("quantize_mxfp8");
}

namespace {

// The 16-bit fast path applies: no padding, whole 64-column units, aligned pointers.
bool nvfp4_fast_applies(const void* x, const void* qx, const void* scales, int64_t rows, int64_t cols,
                        int64_t orig_rows, int64_t orig_cols, int in_code) {
    return (in_code == CKH_BF16 || in_code == CKH_F16) && rows == orig_rows && cols == orig_cols && cols % 64 == 0 &&
           aligned(x, 16) && aligned(qx, 8) && aligned(scales, 16) && rup(rows, 128) * cols < (int64_t(1) << 31);
}

// items: 128-row tiles x groups of G unit columns, 4 workgroups per item; G = 16 (2 KB row
// runs) unless a row has fewer than 16 units.  DYN: see quantize_nvfp4_fast_kernel.
template <bool DYN>
void launch_nvfp4_fast(const void* x, const float* g, uint8_t* q, uint32_t* s, int64_t rows, int64_t cols,
                       int in_code, bool hf, const uint32_t* partial, uint32_t nparts, float inv_divisor,
                       float* scale_out, hipStream_t st) {
    const int64_t n_cb = cdiv(cols / 16, 4);
    const int G = n_cb >= 16 ? 16 : 4;
    const int64_t n_cg = cdiv(n_cb, G), n_items = cdiv(rows, 128) * n_cg;
    uint32_t magic, shift;
    magic_div(n_cg, magic, shift);
    dim3 fgrid(static_cast<unsigned>(cdiv(n_items, 8) * 32));
    const uint16_t* xx = static_cast<const uint16_t*>(x);
    const auto r32 = static_cast<uint32_t>(rows), c32 = static_cast<uint32_t>(cols),
               n32 = static_cast<uint32_t>(n_cb), i32 = static_cast<uint32_t>(n_items),
               g32 = static_cast<uint32_t>(n_cg);
#define LAUNCH_FAST(I, H, GG)                                                                                    \
    hipLaunchKernelGGL((quantize_nvfp4_fast_kernel<I, H, GG, DYN>), fgrid, dim3(64 * GG), 0, st, xx, g, q, s, r32, \
                       c32, n32, i32, g32, magic, shift, partial, nparts, inv_divisor, scale_out)
#define BY_G(I, H)                          \
    do {                                    \
        if (G == 16) LAUNCH_FAST(I, H, 16); \
        else LAUNCH_FAST(I, H, 4);          \
    } while (0)
    if (in_code == CKH_BF16) {
        if (hf) BY_G(CKH_BF16, true);
        else BY_G(CKH_BF16, false);
    } else {
        if (hf) BY_G(CKH_F16, true);
        else BY_G(CKH_F16, false);
    }
#undef BY_G
#undef LAUNCH_FAST
}

int check_nvfp4_args(const void* qx, const void* scales, int64_t rows, int64_t cols, int64_t orig_rows,
                     int64_t orig_cols, int in_code, const char* what) {
    CKH_REQUIRE(rows >= orig_rows && cols >= orig_cols && orig_rows >= 0 && orig_cols >= 0,
                "%s: padded shape smaller than input", what);
    CKH_REQUIRE(cols % 16 == 0, "%s: cols (%lld) must be a multiple of 16", what, (long long)cols);
    CKH_REQUIRE(in_code == CKH_F32 || in_code == CKH_F16 || in_code == CKH_BF16,
                "%s: unsupported input dtype code %d", what, in_code);
    CKH_REQUIRE(aligned(qx, 4) && aligned(scales, 4), "%s: output pointers misaligned", what);
    return CKH_OK;
}

}  // namespace

extern "C" int ckh_quantize_nvfp4(const void* x, const void* global_scale, void* qx, void* scales, int64_t rows,
                                  int64_t cols, int64_t orig_rows, int64_t orig_cols, float epsilon, int in_code,
                                  int hi_first, uintptr_t stream) {
    (void)epsilon;  // accepted for ABI compatibility; the reference ignores it too
    CKH_REQUIRE(x && global_scale && qx && scales, "quantize_nvfp4: null pointer");
    if (int rc = check_nvfp4_args(qx, scales, rows, cols, orig_rows, orig_cols, in_code, "quantize_nvfp4")) return rc;
    if (rows == 0 || cols == 0) return CKH_OK;
    const int64_t n_cb = cdiv(cols / 16, 4);
    const int64_t n_units = rup(rows, 128) * n_cb;
    const bool vec_ok = aligned(x, 16) && orig_cols % 8 == 0;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const float* g = static_cast<const float*>(global_scale);
    uint8_t* q = static_cast<uint8_t*>(qx);
    uint32_t* s = static_cast<uint32_t*>(scales);
    const bool hf = hi_first != 0;
    if (nvfp4_fast_applies(x, qx, scales, rows, cols, orig_rows, orig_cols, in_code)) {
        launch_nvfp4_fast<false>(x, g, q, s, rows, cols, in_code, hf, nullptr, 0u, 0.0f, nullptr, st);
        return check_launch("quantize_nvfp4");
    }
    dim3 grid(static_cast<unsigned>(cdiv(n_units * 8, kThreads)));
#define LAUNCH(I, H)                                                                                \
    hipLaunchKernelGGL((quantize_nvfp4_kernel<I, H>), grid, dim3(kThreads), 0, st, x, g, q, s, rows, cols, \
                       orig_rows, orig_cols, n_cb, n_units, vec_ok)
#define BY_ORDER(I)          \
    do {                     \
        if (hf) LAUNCH(I, true); \
        else LAUNCH(I, false);   \
    } while (0)
    if (in_code == CKH_F32) BY_ORDER(CKH_F32);
    else if (in_code == CKH_F16) BY_ORDER(CKH_F16);
    else BY_ORDER(CKH_BF16);
#undef BY_ORDER
#undef LAUNCH
    return check_launch("quantize_nvfp4");
}

extern "C" int ckh_quantize_nvfp4_dynamic(const void* x, float divisor, void* scale_out, void* qx, void* scales,
                                          int64_t rows, int64_t cols, int64_t orig_rows, int64_t orig_cols,
                                          float epsilon, int in_code, int hi_first, void* workspace,
                                          uintptr_t stream) {
    CKH_REQUIRE(x && scale_out && qx && scales && workspace, "quantize_nvfp4_dynamic: null pointer");
    if (int rc = check_nvfp4_args(qx, scales, rows, cols, orig_rows, orig_cols, in_code, "quantize_nvfp4_dynamic"))
        return rc;
    CKH_REQUIRE(orig_rows > 0 && orig_cols > 0,
                "quantize_nvfp4_dynamic: empty tensor (torch.amax of an empty tensor is an error too)");
    CKH_REQUIRE(aligned(scale_out, 4) && aligned(workspace, 4), "quantize_nvfp4_dynamic: scale or workspace misaligned");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    uint32_t* partial = static_cast<uint32_t*>(workspace);
    const int nparts = amax_partials(x, orig_rows * orig_cols, in_code, partial, st);
    if (nvfp4_fast_applies(x, qx, scales, rows, cols, orig_rows, orig_cols, in_code)) {
        launch_nvfp4_fast<true>(x, nullptr, static_cast<uint8_t*>(qx), static_cast<uint32_t*>(scales), rows, cols,
                                in_code, hi_first != 0, partial, static_cast<uint32_t>(nparts), 1.0f / divisor,
                                static_cast<float*>(scale_out), st);
        return check_launch("quantize_nvfp4_dynamic");
    }
    // other shapes: the scale as its own launch, then the general quantize reading it
    amax_finalize(partial, nparts, in_code, divisor, static_cast<float*>(scale_out), st);
    if (int rc = check_launch("quantize_nvfp4_dynamic")) return rc;
    return ckh_quantize_nvfp4(x, scale_out, qx, scales, rows, cols, orig_rows, orig_cols, epsilon, in_code, hi_first,
                              stream);
}

extern "C" int ckh_dequantize_mxfp8(const void* qx, const void* scales, void* out, int64_t rows, int64_t cols,
                                    int out_code, uintptr_t stream) {
    CKH_REQUIRE(qx && scales && out, "dequantize_mxfp8: null pointer");
    CKH_REQUIRE(rows >= 0 && cols % 32 == 0, "dequantize_mxfp8: cols (%lld) must be a multiple of 32",
                (long long)cols);
    CKH_REQUIRE(out_code == CKH_F32 || out_code == CKH_F16 || out_code == CKH_BF16,
                "dequantize_mxfp8: unsupported output dtype code %d", out_code);
    CKH_REQUIRE(aligned(qx, 8) && aligned(out, 16), "dequantize_mxfp8: pointers misaligned");
    if (rows == 0 || cols == 0) return CKH_OK;
    const int64_t n_cb = cdiv(cols / 32, 4);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const uint8_t* q = static_cast<const uint8_t*>(qx);
    const uint8_t* s = static_cast<const uint8_t*>(scales);
    const int64_t n_pieces = rows * (cols / 8);
    if (out_code != CKH_F32 && n_pieces < (int64_t(1) << 31)) {
        uint32_t magic, shift;
        magic_div(cols / 8, magic, shift);
        const dim3 fgrid(static_cast<unsigned>(cdiv(n_pieces, kThreads * kDqPiecesMx)));
        const uint32_t np = static_cast<uint32_t>(n_pieces), pr = static_cast<uint32_t>(cols / 8),
                       ncb = static_cast<uint32_t>(n_cb);
        uint16_t* o = static_cast<uint16_t*>(out);
#define LAUNCH_FAST(O) \
    hipLaunchKernelGGL((dequantize_mxfp8_fast_kernel<O>), fgrid, dim3(kThreads), 0, st, q, s, o, np, pr, magic, shift, ncb)
        if (out_code == CKH_F16) LAUNCH_FAST(CKH_F16);
        else LAUNCH_FAST(CKH_BF16);
#undef LAUNCH_FAST
        return check_launch("dequantize_mxfp8");
    }
    dim3 grid(static_cast<unsigned>(cdiv(rows * (cols / 8), kThreads)));
#define LAUNCH(O) hipLaunchKernelGGL((dequantize_mxfp8_kernel<O>), grid, dim3(kThreads), 0, st, q, s, out, rows, cols, n_cb)
    if (out_code == CKH_F32) LAUNCH(CKH_F32);
    else if (out_code == CKH_F16) LAUNCH(CKH_F16);
    else LAUNCH(CKH_BF16);
#undef LAUNCH
    return check_launch("dequantize_mxfp8");
}

extern "C" int ckh_dequantize_nvfp4(const void* qx, const void* global_scale, const void* scales, void* out,
                                    int64_t rows, int64_t cols, int out_code, int hi_first, uintptr_t stream) {
    CKH_REQUIRE(qx && global_scale && scales && out, "dequantize_nvfp4: null pointer");
    CKH_REQUIRE(rows >= 0 && cols % 16 == 0, "dequantize_nvfp4: cols (%lld) must be a multiple of 16",
                (long long)cols);
    CKH_REQUIRE(out_code == CKH_F32 || out_code == CKH_F16 || out_code == CKH_BF16,
                "dequantize_nvfp4: unsupported output dtype code %d", out_code);
    CKH_REQUIRE(aligned(qx, 4) && aligned(out, 16), "dequantize_nvfp4: pointers misaligned");
    if (rows == 0 || cols == 0) return CKH_OK;
    const int64_t n_cb = cdiv(cols / 16, 4);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const uint8_t* q = static_cast<const uint8_t*>(qx);
    const float* g = static_cast<const float*>(global_scale);
    const uint8_t* s = static_cast<const uint8_t*>(scales);
    const bool hf = hi_first != 0;
    if (out_code != CKH_F32 && cols % 256 == 0 && rows * cols < (int64_t(1) << 31)) {
        const uint32_t n_ct = static_cast<uint32_t>(cols / 256);
        const dim3 tgrid(static_cast<unsigned>(cdiv(rows, 128) * 4 * n_ct));
        const uint32_t r32 = static_cast<uint32_t>(rows), c32 = static_cast<uint32_t>(cols),
                       ncb = static_cast<uint32_t>(n_cb);
        uint16_t* o = static_cast<uint16_t*>(out);
#define LAUNCH_TILE(O, H) \
    hipLaunchKernelGGL((dequantize_nvfp4_tile_kernel<O, H>), tgrid, dim3(512), 0, st, q, g, s, o, r32, c32, n_ct, ncb)
        if (out_code == CKH_F16) {
            if (hf) LAUNCH_TILE(CKH_F16, true);
            else LAUNCH_TILE(CKH_F16, false);
        } else {
            if (hf) LAUNCH_TILE(CKH_BF16, true);
            else LAUNCH_TILE(CKH_BF16, false);
        }
#undef LAUNCH_TILE
        return check_launch("dequantize_nvfp4");
    }
    const int64_t n_pieces = rows * (cols / 8);
    if (out_code != CKH_F32 && cols % 8 == 0 && n_pieces < (int64_t(1) << 31)) {
        uint32_t magic, shift;
        magic_div(cols / 8, magic, shift);
        const dim3 fgrid(static_cast<unsigned>(cdiv(n_pieces, kThreads * kDqPiecesNv)));
        const uint32_t np = static_cast<uint32_t>(n_pieces), pr = static_cast<uint32_t>(cols / 8),
                       ncb = static_cast<uint32_t>(n_cb);
        uint16_t* o = static_cast<uint16_t*>(out);
#define LAUNCH_FAST(O, H)                                                                                   \
    hipLaunchKernelGGL((dequantize_nvfp4_fast_kernel<O, H>), fgrid, dim3(kThreads), 0, st, q, g, s, o, np, pr, \
                       magic, shift, ncb)
        if (out_code == CKH_F16) {
            if (hf) LAUNCH_FAST(CKH_F16, true);
            else LAUNCH_FAST(CKH_F16, false);
        } else {
            if (hf) LAUNCH_FAST(CKH_BF16, true);
            else LAUNCH_FAST(CKH_BF16, false);
        }
#undef LAUNCH_FAST
        return check_launch("dequantize_nvfp4");
    }
    dim3 grid(static_cast<unsigned>(cdiv(rows * (cols / 8), kThreads)));
#define LAUNCH(O) \
    hipLaunchKernelGGL((dequantize_nvfp4_kernel<O>), grid, dim3(kThreads), 0, st, q, g, s, out, rows, cols, n_cb, hf)
    if (out_code == CKH_F32) LAUNCH(CKH_F32);
    else if (out_code == CKH_F16) LAUNCH(CKH_F16);
    else LAUNCH(CKH_BF16);
#undef LAUNCH
    return check_launch("dequantize_nvfp4");
}
