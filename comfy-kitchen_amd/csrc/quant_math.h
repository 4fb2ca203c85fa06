// Exact arithmetic steps of the block quantizers' fast paths (quant_block.hip), in a
// header so that the exhaustive hardware checks (tests/hw/identities.hip) test these very
// functions.  Each is exact, or equal to the reference's IEEE operation, on the domain
// stated with it; the callers keep to those domains and take IEEE paths elsewhere.
#pragma once

#include "ckh_common.h"

namespace ckh {

typedef unsigned short ckh_u16x2 __attribute__((ext_vector_type(2)));
typedef short ckh_i16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 ckh_bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 ckh_f16x2 __attribute__((ext_vector_type(2)));

// ------------------------------------------------------------------- MXFP8
// E8M0 exponent of a block from its amax bits (reference eager quantization.py:292-302):
//   s = max(amax/448, 2^-127); e = clamp(ceil(log2 s) + 127, 0, 254).
// ceil(log2 s) is taken exactly from the bit fields of s: for normal s it is the
// unbiased exponent plus one if any mantissa bit is set; s = 2^-127 (the clamp) gives
// e = 0 and the only other subnormals, 2^-127 < s < 2^-126, give e = 1.  Non-finite
// amax gives e = 0, as the reference's float->int32 conversion of ceil(log2(inf/NaN))
// does on x86.
//
// For amax with a biased exponent >= 10 the division folds away: amax/448 =
// (1.f / 1.75) * 2^(E-8) with 1.f the significand, so s is a power of two only when
// 1.f == 1.75 exactly, and e = E - 8 + (f > 0.75).  (Checked against the division form
// on all 2^31 non-negative floats.)
__device__ __forceinline__ uint32_t mx_exponent(uint32_t amax_bits) {
    if (amax_bits >= (10u << 23) && amax_bits < 0x7f800000u)
        return (amax_bits >> 23) - 8u + ((amax_bits & 0x7fffffu) > 0x600000u);
    if (amax_bits == 0 || amax_bits >= 0x7f800000u) return 0;
    uint32_t s = as_u(as_f(amax_bits) / 448.0f);
    if (s <= 0x00400000u) return 0;
    if (s < 0x00800000u) return 1;
    uint32_t e = (s >> 23) + ((s & 0x7fffffu) != 0);
    return e > 254u ? 254u : e;
}

// Codes of the two packed pairs a, b: E4M3(x / 2^(e-127)), scale = 2^(e-127).
template <int IN>
__device__ __forceinline__ uint32_t scaled_e4m3x4(uint32_t a, uint32_t b, float scale) {
    ckh_i16x2 o = {0, 0};
    if constexpr (IN == CKH_BF16) {
        o = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(o, __builtin_bit_cast(ckh_bf16x2, a), scale, false);
        o = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(o, __builtin_bit_cast(ckh_bf16x2, b), scale, true);
    } else {
        o = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(o, __builtin_bit_cast(ckh_f16x2, a), scale, false);
        o = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(o, __builtin_bit_cast(ckh_f16x2, b), scale, true);
    }
    return __builtin_bit_cast(uint32_t, o);
}

// Codes for one lane's 8 values given the block's amax bits and exponent.
__device__ __forceinline__ uint2 mx_encode8(const float (&v)[8], uint32_t amax_bits, uint32_t e) {
    uint32_t w[2] = {0u, 0u};
    if (amax_bits == 0) return make_uint2(0u, 0u);  // zero block: +0 codes
    if (e == 0) {
        // Scale 0.0 (eager's fp32 division on x86): x/0 is +-inf, clamped to +-448, for
        // non-NaN x != 0 (inf included); 0/0 is x86's default NaN, which is negative
        // (0xFF); a NaN x stays x's NaN, sign kept (0x7F | sign).
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const uint32_t u = as_u(v[t]), a = u & 0x7fffffffu, sign = (u >> 24) & 0x80u;
            const uint32_t c = a == 0 ? 0xffu : (a > 0x7f800000u ? (0x7fu | sign) : (0x7eu | sign));
            w[t >> 2] |= c << (8 * (t & 3));
        }
        return make_uint2(w[0], w[1]);
    }
    // x / 2^(e-127) == x * 2^(127-e) exactly (both correctly rounded); 1 <= e <= 254
    // keeps 2^(127-e) a normal float.  Here amax is finite and 2^(e-127) >= amax/448, so
    // every |q| <= 448: the reference's clamp is a no-op and the hardware convert
    // (RNE, identical to f_to_e4m3 on this range) encodes directly.
    const float mul = as_f((254u - e) << 23);
    float q[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) q[t] = v[t] * mul;
    return make_uint2(hw_e4m3x4(q[0], q[1], q[2], q[3]), hw_e4m3x4(q[4], q[5], q[6], q[7]));
}

// |x| maxima of 8 packed 16-bit values as a 16-bit integer (orders like the values).
__device__ __forceinline__ uint32_t amax16x8(uint4 w) {
    auto h = [](uint32_t v) { return __builtin_bit_cast(ckh_u16x2, v & 0x7fff7fffu); };
    ckh_u16x2 m = __builtin_elementwise_max(__builtin_elementwise_max(h(w.x), h(w.y)),
                                            __builtin_elementwise_max(h(w.z), h(w.w)));
    return max(static_cast<uint32_t>(m.x), static_cast<uint32_t>(m.y));
}


// 16-bit amax bits -> fp32 bits of the same value
template <int IN>
__device__ __forceinline__ uint32_t amax16_to_f32_bits(uint32_t m) {
    if constexpr (IN == CKH_BF16) return m << 16;
    else return as_u(static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(m))));
}

template <int IN>
__device__ __forceinline__ void unpack16x8(uint4 w, float (&v)[8]) {
    const uint32_t p[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if constexpr (IN == CKH_BF16) {
            v[2 * i] = as_f(p[i] << 16);
            v[2 * i + 1] = as_f(p[i] & 0xffff0000u);
        } else {
            ckh_f16x2 h = __builtin_bit_cast(ckh_f16x2, p[i]);
            v[2 * i] = static_cast<float>(h.x);
            v[2 * i + 1] = static_cast<float>(h.y);
        }
    }
}

// Codes of one lane's 8 packed 16-bit values w (E4M3) and the E8M0 exponent e of their
// 32-element block, whose amax has fp32 bits `bits`: the packed scaled convert on the
// common range, the general encoder for zero, tiny and non-finite blocks.
template <int IN>
__device__ __forceinline__ uint2 mx_codes16(uint4 w, uint32_t bits, uint32_t& e) {
    if (bits >= (10u << 23) && bits < 0x7f800000u) {
        e = (bits >> 23) - 8u + ((bits & 0x7fffffu) > 0x600000u);
        const float scale = as_f(e << 23);
        return make_uint2(scaled_e4m3x4<IN>(w.x, w.y, scale), scaled_e4m3x4<IN>(w.z, w.w, scale));
    }
    e = mx_exponent(bits);
    float v[8];
    unpack16x8<IN>(w, v);
    return mx_encode8(v, bits, e);
}

// Pack 8 non-NaN values into E2M1 nibbles with the hardware convert: RNE, identical to
// f_to_e2m1 of the value clamped to [-6, 6] (the convert saturates), and the first
// operand lands in the low nibble.
template <bool HI_FIRST>
__device__ __forceinline__ uint32_t pack_e2m1x8(const float* q) {
    const int f = HI_FIRST ? 1 : 0, o = 1 - f;  // element of each pair that goes to the low nibble
    uint32_t w = 0;
    w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, q[0 + f], q[0 + o], 1.0f, 0);
    w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, q[2 + f], q[2 + o], 1.0f, 1);
    w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, q[4 + f], q[4 + o], 1.0f, 2);
    w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, q[6 + f], q[6 + o], 1.0f, 3);
    return w;
}

// RN(1/T) from v_rcp_f32 and one FMA Newton step: equal to the IEEE 1.0f / T for every
// float T in [2^-70, 2^71).
__device__ __forceinline__ float rcp_newton(float T) {
    const float y0 = __builtin_amdgcn_rcpf(T);
    return __builtin_fmaf(__builtin_fmaf(-T, y0, 1.0f), y0, y0);
}

// v / T by one Markstein correction of v * y, y = RN(1/T): q0 = v*y, e = fma(T, q0, -v),
// q = fma(-e, y, q0).  Its E2M1 code equals that of the IEEE quotient for every bf16 and
// f16 v (both signs, and +-0) and every T whose products stay normal (the negated
// residual keeps the sign of a zero v).
__device__ __forceinline__ float markstein_quotient(float v, float T, float y) {
    const float q0 = v * y;
    const float e = __builtin_fmaf(T, q0, -v);
    return __builtin_fmaf(-e, y, q0);
}

// (amax / 6) / g by two Markstein steps with the constant RN(1/6) and yg = RN(1/g):
// bit-identical to the two IEEE divisions for every bf16 / f16 amax significand and every
// g significand while g and amax lie within [2^-60, 2^60].
__device__ __forceinline__ float nvfp4_c_steps(float amax, float g, float yg) {
    constexpr float y6 = 1.0f / 6.0f;
    const float c0 = amax * y6;
    const float c1 = __builtin_fmaf(-__builtin_fmaf(6.0f, c0, -amax), y6, c0);
    const float d0 = c1 * yg;
    return __builtin_fmaf(-__builtin_fmaf(g, d0, -c1), yg, d0);
}

// ----------------------------------------------------- NVFP4 GEMM operand decode
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

// Byte SEL of w (two E2M1 codes) -> 2 fp16 (low nibble first), times the scale pair s.
// Exact: E2M1 x E4M3 products have at most 6 significant bits and lie in [2^-10, 2688]
// (or are zero), all fp16 normals.  (The convert's own scale operand cannot carry the
// E4M3 scale: the hardware uses only its exponent.)
template <int SEL>
__device__ __forceinline__ v2h decode2(uint32_t w, v2h s) {
    return __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, SEL) * s;
}

// 4 bytes of E2M1 codes -> 8 fp16 (low nibble first), times the block scale pair s.
__device__ __forceinline__ v8h decode8(uint32_t w, v2h s) {
    const v2h e0 = decode2<0>(w, s), e1 = decode2<1>(w, s), e2 = decode2<2>(w, s), e3 = decode2<3>(w, s);
    return v8h{e0[0], e0[1], e1[0], e1[1], e2[0], e2[1], e3[0], e3[1]};
}

// Two E4M3 block scales (bytes sh/8 and sh/8 + 1 of the word) as fp16; exact for every
// finite code.
__device__ __forceinline__ v2h scale_pair(uint32_t word, int sh) {
    return __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(word >> sh, 1.0f, false);
}

}  // namespace ckh
