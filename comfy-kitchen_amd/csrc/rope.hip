// Fused RoPE for gfx950: apply_rope (q and k in one pass) and apply_rope1.
//
// out[2i+r] = f[i][r][0] * x[2i] + f[i][r][1] * x[2i+1], computed in the freqs dtype
// and rounded to x's dtype (reference eager rope.py:7-14).  The product f0*x0 is
// rounded to the freqs precision, then f1*x1 is added with one rounding (an FMA for
// fp32 freqs; for 16-bit freqs the fp32 FMA is exact before the final rounding).
//
// Freqs reuse: x rows (b, d1, d2) that read the same freqs row (the freqs dims of
// size 1 broadcast) are grouped, and each lane loads the rotation matrices of its pairs
// once into registers and then streams x rows of the group (both q and k), so freqs are
// read from HBM once instead of once per head.
//   rope_wave_kernel (16-byte rows, head_dim/8 lanes per row dividing 64): a wave holds
//     several consecutive freqs rows, so with the usual [B, H, S, D] layout each load
//     instruction reads a contiguous run of x; streaming loads, pipelined over rows.
//   rope_kernel (any other shape or alignment): a workgroup owns one freqs row; lanes
//     per row = head_dim / (2 * PPL), each lane holds PPL pairs.
#include "ckh_common.h"

namespace ckh {

struct RopeArgs {
    const void* xq;
    const void* xk;
    const void* freqs;
    void* oq;
    void* ok;
    int64_t D1, D2;
    int hd;
    // freqs-row grid (dims where freqs has size > 1) and broadcast grid (size 1)
    int64_t P1, P2;  // radices of the freqs-row index over (b, d1, d2)
    int64_t R1, R2;  // radices of the broadcast index over (b, d1, d2)
    int64_t R;       // x rows per freqs row
    int64_t rows_per_block;
    int64_t sxb, sx1, sx2;
    int64_t sfb, sf1, sf2;
    int lanes_per_row;
    int slots;  // rows processed concurrently by one workgroup
};

template <int C>
__device__ __forceinline__ float ld(const void* p, int64_t i) {
    return load1<C>(p, i);
}

// The output value of x's dtype as its bits (fp32 x: the value itself).
template <int XC>
__device__ __forceinline__ uint32_t to_bits(float f) {
    if constexpr (XC == CKH_F32) return as_u(f);
    else return XC == CKH_BF16 ? f_to_bf16(f) : f_to_f16(f);
}

template <int XC, int FC, int PPL>
__global__ __launch_bounds__(256) void rope_kernel(RopeArgs a) {
    const int tid = threadIdx.x;
    const int slot = tid / a.lanes_per_row;
    const int lane = tid - slot * a.lanes_per_row;
    if (slot >= a.slots) return;

    // freqs row p -> (pb, p1, p2)
    const int64_t p = blockIdx.x;
    const int64_t pb = p / (a.P1 * a.P2);
    const int64_t p1 = (p / a.P2) % a.P1;
    const int64_t p2 = p % a.P2;

    // rotation matrices of this lane's PPL pairs, in float
    float f[PPL][4];
    const int64_t fbase = pb * a.sfb + p1 * a.sf1 + p2 * a.sf2 + static_cast<int64_t>(lane) * PPL * 4;
    if constexpr (FC == CKH_F32 && PPL == 4) {
        const float4* fp = reinterpret_cast<const float4*>(static_cast<const float*>(a.freqs) + fbase);
#pragma unroll
        for (int i = 0; i < PPL; ++i) {
            float4 m = fp[i];
            f[i][0] = m.x; f[i][1] = m.y; f[i][2] = m.z; f[i][3] = m.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < PPL; ++i)
#pragma unroll
            for (int c = 0; c < 4; ++c) f[i][c] = ld<FC>(a.freqs, fbase + i * 4 + c);
    }

    const int64_t r_begin = static_cast<int64_t>(blockIdx.y) * a.rows_per_block;
    const int64_t r_end = min(a.R, r_begin + a.rows_per_block);
    for (int64_t rho = r_begin + slot; rho < r_end; rho += a.slots) {
        const int64_t rb = rho / (a.R1 * a.R2);
        const int64_t r1 = (rho / a.R2) % a.R1;
        const int64_t r2 = rho % a.R2;
        const int64_t b = pb + rb, d1 = p1 + r1, d2 = p2 + r2;  // one of each pair is 0
        const int64_t xoff = b * a.sxb + d1 * a.sx1 + d2 * a.sx2 + static_cast<int64_t>(lane) * PPL * 2;
        const int64_t ooff = ((b * a.D1 + d1) * a.D2 + d2) * a.hd + static_cast<int64_t>(lane) * PPL * 2;
#pragma unroll
        for (int which = 0; which < 2; ++which) {
            const void* src = which ? a.xk : a.xq;
            void* dst = which ? a.ok : a.oq;
            if (src == nullptr) break;
            constexpr int ES = ElemSize<XC>::value;
            float x[2 * PPL];
            if constexpr (PPL == 4) {
                load8<XC>(static_cast<const char*>(src) + xoff * ES, x);
            } else {
#pragma unroll
                for (int e = 0; e < 2 * PPL; ++e) x[e] = ld<XC>(src, xoff + e);
            }
            uint32_t o[2 * PPL];
#pragma unroll
            for (int i = 0; i < PPL; ++i) {
                const float x0 = round_to<FC>(x[2 * i]), x1 = round_to<FC>(x[2 * i + 1]);
#pragma unroll
                for (int r = 0; r < 2; ++r) {
                    const float t = round_to<FC>(__fmul_rn(f[i][2 * r], x0));
                    const float y = round_to<FC>(__fmaf_rn(f[i][2 * r + 1], x1, t));
                    o[2 * i + r] = to_bits<XC>(y);
                }
            }
            if constexpr (XC == CKH_F32) {
                uint32_t* op = static_cast<uint32_t*>(dst) + ooff;
                if constexpr (PPL == 4) {
                    *reinterpret_cast<uint4*>(op) = make_uint4(o[0], o[1], o[2], o[3]);
                    *reinterpret_cast<uint4*>(op + 4) = make_uint4(o[4], o[5], o[6], o[7]);
                } else {
#pragma unroll
                    for (int e = 0; e < 2 * PPL; ++e) op[e] = o[e];
                }
            } else {
                uint16_t* op = static_cast<uint16_t*>(dst) + ooff;
                if constexpr (PPL == 4) {
                    *reinterpret_cast<uint4*>(op) = make_uint4(o[0] | (o[1] << 16), o[2] | (o[3] << 16),
                                                               o[4] | (o[5] << 16), o[6] | (o[7] << 16));
                } else {
#pragma unroll
                    for (int e = 0; e < 2 * PPL; ++e) op[e] = static_cast<uint16_t>(o[e]);
                }
            }
        }
    }
}

// ------------------------------------------------------------ wave-position kernel
// Vectorized case (16-byte x loads, head_dim/8 = L lanes per row, L dividing 64).
// A wave holds W = 64/L consecutive freqs rows p; the workgroup's four waves share
// them and take every fourth x row rho of the rows that broadcast over them (the same
// freqs), so each lane holds its four rotation matrices (fp32 freqs: loaded once per
// workgroup and shared through LDS) and then streams up to
// kRowsPerWave rows of q and of k, loading row i+1 while row i is rotated and stored
// (apply_rope1: all rows loaded first).  With Flux's layout (freqs over the sequence,
// broadcast over heads) consecutive p are consecutive x rows, so every load
// instruction reads W * head_dim * 2 contiguous bytes.  The rho -> (b, d1, d2)
// decomposition is wave-uniform and done in scalar registers.
struct RopeWaveArgs {
    const void* xq;
    const void* xk;
    const void* freqs;
    void* oq;
    void* ok;
    int64_t D1, D2;
    int64_t sxb, sx1, sx2;
    int64_t sfb, sf1, sf2;
    int32_t hd, log2_lanes;
    int32_t P, P1, P2;  // freqs rows and their radices over (b, d1, d2)
    int32_t R, R1, R2;  // broadcast rows and their radices
    int32_t rows_per_block;
};
constexpr int kRowsPerWave = 4;  // 1, 2, 4 and 8 measured; 4 with the pipeline is fastest

template <int XC, int FC>
__device__ __forceinline__ uint4 rotate8(uint4 w, const float (&f)[4][4]) {
    float x[8];
    const uint32_t d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        x[2 * i] = XC == CKH_BF16 ? bf16_to_f(d[i] & 0xffffu) : f16_to_f(d[i] & 0xffffu);
        x[2 * i + 1] = XC == CKH_BF16 ? bf16_to_f(d[i] >> 16) : f16_to_f(d[i] >> 16);
    }
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float x0 = round_to_hw<FC>(x[2 * i]), x1 = round_to_hw<FC>(x[2 * i + 1]);
        float y[2];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const float t = round_to_hw<FC>(__fmul_rn(f[i][2 * r], x0));
            y[r] = round_to_hw<FC>(__fmaf_rn(f[i][2 * r + 1], x1, t));
        }
        if constexpr (XC == CKH_BF16) {
            // one v_cvt_pk_bf16_f32 per pair (RNE; equal to f_to_bf16 for non-NaN)
            typedef float f32x2 __attribute__((ext_vector_type(2)));
            typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
            const f32x2 yy = {y[0], y[1]};
            o[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(yy, bf16x2));
        } else {
            o[i] = f_to_f16(y[0]) | (f_to_f16(y[1]) << 16);
        }
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
}

// ONE: apply_rope1 (no k tensor)
template <int XC, int FC, bool ONE>
__global__ __launch_bounds__(256) void rope_wave_kernel(RopeWaveArgs a) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int L = 1 << a.log2_lanes;
    const int c = lane & (L - 1);                                     // column group: pairs 4c..4c+3
    // freqs row; lanes past the last row load row P - 1 and leave after the LDS exchange
    const int p_lane = blockIdx.x * (64 >> a.log2_lanes) + (lane >> a.log2_lanes);
    const bool p_ok = p_lane < a.P;
    const int p = p_ok ? p_lane : a.P - 1;
    const int p2 = p % a.P2, p1 = (p / a.P2) % a.P1, pb = p / (a.P2 * a.P1);
    const int64_t xbase = pb * a.sxb + p1 * a.sx1 + p2 * a.sx2 + 8 * c;
    const int64_t obase = ((pb * a.D1 + p1) * a.D2 + p2) * a.hd + 8 * c;

    float f[4][4];
    const int64_t fbase = pb * a.sfb + p1 * a.sf1 + p2 * a.sf2 + 16 * c;
    if constexpr (FC == CKH_F32) {
        // the four waves hold the same rows: wave w loads matrix w of every lane and the
        // others read it from LDS (a quarter of the freqs load instructions; measured ~1%
        // faster for apply_rope and apply_rope1 at C2)
        __shared__ float4 fsh[4][64];
        const float4* fp = reinterpret_cast<const float4*>(static_cast<const float*>(a.freqs) + fbase);
        fsh[wave][lane] = fp[wave];
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 m = fsh[i][lane];
            f[i][0] = m.x; f[i][1] = m.y; f[i][2] = m.z; f[i][3] = m.w;
        }
        if (!p_ok) return;
    } else {
        if (!p_ok) return;
        const uint4* fp = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.freqs) + fbase);
        const uint4 m0 = fp[0], m1 = fp[1];
        const uint32_t d[8] = {m0.x, m0.y, m0.z, m0.w, m1.x, m1.y, m1.z, m1.w};
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const uint32_t h = (d[e >> 1] >> (16 * (e & 1))) & 0xffffu;
            f[e >> 2][e & 3] = FC == CKH_BF16 ? bf16_to_f(h) : f16_to_f(h);
        }
    }

    const int r0 = blockIdx.y * a.rows_per_block + wave;
    const int r_end = min(a.R, static_cast<int>(blockIdx.y + 1) * a.rows_per_block);
    if constexpr (ONE) {
        // apply_rope1: all of the wave's rows are loaded before any is rotated (up to
        // kRowsPerWave 16-byte loads in flight per lane); measured 3.5% faster than the
        // pipelined loop below for q alone, 2% slower for q and k
        int64_t oo[kRowsPerWave];
        uint4 cq[kRowsPerWave];
#pragma unroll
        for (int i = 0; i < kRowsPerWave; ++i) {
            const int rho = r0 + 4 * i;
            if (rho < r_end) {
                const int r2 = rho % a.R2, r1 = (rho / a.R2) % a.R1, rb = rho / (a.R2 * a.R1);
                const int64_t xo = xbase + rb * a.sxb + r1 * a.sx1 + r2 * a.sx2;
                oo[i] = obase + ((rb * a.D1 + r1) * a.D2 + r2) * a.hd;
                cq[i] = ld_stream16(static_cast<const uint16_t*>(a.xq) + xo);
            }
        }
#pragma unroll
        for (int i = 0; i < kRowsPerWave; ++i) {
            if (r0 + 4 * i >= r_end) break;
            st_stream16(static_cast<uint16_t*>(a.oq) + oo[i], rotate8<XC, FC>(cq[i], f));
        }
    } else {
        // apply_rope: software pipeline, row i+1's loads in flight while row i is rotated
        // and stored
        auto offs = [&](int rho, int64_t& xo, int64_t& oo) {
            const int r2 = rho % a.R2, r1 = (rho / a.R2) % a.R1, rb = rho / (a.R2 * a.R1);
            xo = xbase + rb * a.sxb + r1 * a.sx1 + r2 * a.sx2;
            oo = obase + ((rb * a.D1 + r1) * a.D2 + r2) * a.hd;
        };
        int64_t xo, oo;
        uint4 cq = make_uint4(0, 0, 0, 0), ck = cq;
        if (r0 < r_end) {
            offs(r0, xo, oo);
            cq = ld_stream16(static_cast<const uint16_t*>(a.xq) + xo);
            if (a.xk) ck = ld_stream16(static_cast<const uint16_t*>(a.xk) + xo);
        }
#pragma unroll
        for (int i = 0; i < kRowsPerWave; ++i) {
            if (r0 + 4 * i >= r_end) break;
            const int64_t o_cur = oo;
            uint4 nq = cq, nk = ck;
            if (i + 1 < kRowsPerWave && r0 + 4 * (i + 1) < r_end) {
                offs(r0 + 4 * (i + 1), xo, oo);
                nq = ld_stream16(static_cast<const uint16_t*>(a.xq) + xo);
                if (a.xk) nk = ld_stream16(static_cast<const uint16_t*>(a.xk) + xo);
            }
            st_stream16(static_cast<uint16_t*>(a.oq) + o_cur, rotate8<XC, FC>(cq, f));
            if (a.xk) st_stream16(static_cast<uint16_t*>(a.ok) + o_cur, rotate8<XC, FC>(ck, f));
            cq = nq;
            ck = nk;
        }
    }
}

}  // namespace ckh

using namespace ckh;

extern "C" int ckh_apply_rope(const void* xq, const void* xk, const void* freqs, void* xq_out, void* xk_out,
                              int64_t batch, int64_t dim1, int64_t dim2, int64_t head_dim, int64_t freqs_batch,
                              int64_t freqs_dim1, int64_t freqs_dim2, int64_t sx_batch, int64_t sx_dim1,
                              int64_t sx_dim2, int64_t sf_batch, int64_t sf_dim1, int64_t sf_dim2, int in_code,
                              int freqs_code, uintptr_t stream) {
    CKH_REQUIRE(xq && freqs && xq_out, "apply_rope: null pointer");
    CKH_REQUIRE((xk == nullptr) == (xk_out == nullptr), "apply_rope: xk and xk_out must both be given or both NULL");
    CKH_REQUIRE(batch >= 0 && dim1 >= 0 && dim2 >= 0, "apply_rope: negative shape");
    CKH_REQUIRE(head_dim > 0 && head_dim % 2 == 0 && head_dim <= 4096, "apply_rope: head_dim (%lld) must be even",
                (long long)head_dim);
    CKH_REQUIRE(in_code == CKH_F32 || in_code == CKH_F16 || in_code == CKH_BF16,
                "apply_rope: unsupported x dtype code %d", in_code);
    CKH_REQUIRE(freqs_code == CKH_F32 || freqs_code == CKH_F16 || freqs_code == CKH_BF16,
                "apply_rope: unsupported freqs dtype code %d", freqs_code);
    CKH_REQUIRE(freqs_batch == 1 || freqs_batch == batch, "apply_rope: freqs dim 0 (%lld) does not broadcast to %lld",
                (long long)freqs_batch, (long long)batch);
    CKH_REQUIRE(freqs_dim1 == 1 || freqs_dim1 == dim1, "apply_rope: freqs dim 1 (%lld) does not broadcast to %lld",
                (long long)freqs_dim1, (long long)dim1);
    CKH_REQUIRE(freqs_dim2 == 1 || freqs_dim2 >= dim2, "apply_rope: freqs dim 2 (%lld) shorter than x dim 2 (%lld)",
                (long long)freqs_dim2, (long long)dim2);
    if (batch == 0 || dim1 == 0 || dim2 == 0) return CKH_OK;

    RopeArgs a{};
    a.xq = xq; a.xk = xk; a.freqs = freqs; a.oq = xq_out; a.ok = xk_out;
    a.D1 = dim1; a.D2 = dim2; a.hd = static_cast<int>(head_dim);
    // freqs dims of size 1 broadcast; dim 2 longer than x's is truncated (rope.py:9-10)
    const int64_t Pb = freqs_batch == 1 ? 1 : batch, P1 = freqs_dim1 == 1 ? 1 : dim1, P2 = freqs_dim2 == 1 ? 1 : dim2;
    const int64_t Rb = freqs_batch == 1 ? batch : 1, R1 = freqs_dim1 == 1 ? dim1 : 1, R2 = freqs_dim2 == 1 ? dim2 : 1;
    a.P1 = P1; a.P2 = P2; a.R1 = R1; a.R2 = R2; a.R = Rb * R1 * R2;
    a.sxb = sx_batch; a.sx1 = sx_dim1; a.sx2 = sx_dim2;
    a.sfb = sf_batch; a.sf1 = sf_dim1; a.sf2 = sf_dim2;

    const bool vec = head_dim % 8 == 0 && aligned(xq, 16) && aligned(xq_out, 16) && (!xk || (aligned(xk, 16) && aligned(xk_out, 16))) &&
                     sx_batch % 8 == 0 && sx_dim1 % 8 == 0 && sx_dim2 % 8 == 0 &&
                     (freqs_code != CKH_F32 || (aligned(freqs, 16) && sf_batch % 4 == 0 && sf_dim1 % 4 == 0 && sf_dim2 % 4 == 0));
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int64_t P = Pb * P1 * P2;
    const int64_t lanes = head_dim / 8;
    // 16-byte freqs loads: f32 rows are covered by vec; 16-bit rows need it here
    const bool fvec = freqs_code == CKH_F32 ||
                      (aligned(freqs, 16) && sf_batch % 8 == 0 && sf_dim1 % 8 == 0 && sf_dim2 % 8 == 0);
    if (in_code != CKH_F32 && vec && fvec && lanes <= 64 && (64 % lanes) == 0 && P < (int64_t(1) << 30) &&
        a.R < (int64_t(1) << 30)) {
        RopeWaveArgs w{};
        w.xq = xq; w.xk = xk; w.freqs = freqs; w.oq = xq_out; w.ok = xk_out;
        w.D1 = dim1; w.D2 = dim2;
        w.sxb = sx_batch; w.sx1 = sx_dim1; w.sx2 = sx_dim2;
        w.sfb = sf_batch; w.sf1 = sf_dim1; w.sf2 = sf_dim2;
        w.hd = static_cast<int32_t>(head_dim);
        int lg = 0;
        while ((int64_t(1) << lg) < lanes) ++lg;
        w.log2_lanes = lg;
        w.P = static_cast<int32_t>(P); w.P1 = static_cast<int32_t>(P1); w.P2 = static_cast<int32_t>(P2);
        w.R = static_cast<int32_t>(a.R); w.R1 = static_cast<int32_t>(R1); w.R2 = static_cast<int32_t>(R2);
        const int64_t chunks = cdiv(a.R, 4 * kRowsPerWave);
        w.rows_per_block = static_cast<int32_t>(rup(cdiv(a.R, chunks), 4));  // <= 4 * kRowsPerWave
        CKH_REQUIRE(chunks < 65536, "apply_rope: grid too large");
        dim3 grid(static_cast<unsigned>(cdiv(P, 64 / lanes)), static_cast<unsigned>(chunks));
#define LAUNCH_W(XC, FC)                                                                        \
    do {                                                                                        \
        if (xk) hipLaunchKernelGGL((rope_wave_kernel<XC, FC, false>), grid, dim3(256), 0, st, w); \
        else hipLaunchKernelGGL((rope_wave_kernel<XC, FC, true>), grid, dim3(256), 0, st, w);    \
    } while (0)
#define BY_FC_W(XC)                                         \
    do {                                                    \
        if (freqs_code == CKH_F32) LAUNCH_W(XC, CKH_F32);       \
        else if (freqs_code == CKH_F16) LAUNCH_W(XC, CKH_F16);  \
        else LAUNCH_W(XC, CKH_BF16);                            \
    } while (0)
        if (in_code == CKH_BF16) BY_FC_W(CKH_BF16);
        else BY_FC_W(CKH_F16);
#undef BY_FC_W
#undef LAUNCH_W
        return check_launch("apply_rope");
    }

    const int ppl = vec ? 4 : 1;
    a.lanes_per_row = static_cast<int>(head_dim / (2 * ppl));
    CKH_REQUIRE(a.lanes_per_row <= 256, "apply_rope: head_dim too large for this kernel");
    const int max_slots = 256 / a.lanes_per_row;
    const int64_t n_chunks = cdiv(a.R, max_slots);
    a.rows_per_block = cdiv(a.R, n_chunks);
    a.slots = static_cast<int>(a.rows_per_block);  // rows_per_block <= max_slots
    int threads = a.slots * a.lanes_per_row;
    threads = static_cast<int>(rup(threads, 64));
    CKH_REQUIRE(P < (int64_t(1) << 31) && n_chunks < 65536, "apply_rope: grid too large");
    dim3 grid(static_cast<unsigned>(P), static_cast<unsigned>(n_chunks));

#define LAUNCH(XC, FC, PPL) hipLaunchKernelGGL((rope_kernel<XC, FC, PPL>), grid, dim3(threads), 0, st, a)
#define BY_PPL(XC, FC)              \
    do {                            \
        if (vec) LAUNCH(XC, FC, 4); \
        else LAUNCH(XC, FC, 1);     \
    } while (0)
#define BY_FC(XC)                                      \
    do {                                               \
        if (freqs_code == CKH_F32) BY_PPL(XC, CKH_F32); \
        else if (freqs_code == CKH_F16) BY_PPL(XC, CKH_F16); \
        else BY_PPL(XC, CKH_BF16);                      \
    } while (0)
    if (in_code == CKH_BF16) BY_FC(CKH_BF16);
    else if (in_code == CKH_F16) BY_FC(CKH_F16);
    else BY_FC(CKH_F32);
#undef BY_FC
#undef BY_PPL
#undef LAUNCH
    return check_launch("apply_rope");
}
