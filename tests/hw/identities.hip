// Exhaustive checks of the gfx950 hardware identities that the quantizers' and GEMMs'
// bit-exactness rests on.  TEST CODE ONLY: built into tests/hw/libckh_hwcheck.so, loaded
// by tests/test_gpu_hw_identities.py, never by the product library.
//
// Each sweep compares a product helper (ckh_common.h, quant_math.h: the very functions
// the kernels call) with its software or IEEE definition over the whole domain on which
// the kernels rely on it, counts the mismatches (one global atomic per thread) and
// records the smallest mismatching input index.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ckh_common.h"
#include "quant_math.h"

using namespace ckh;

namespace {

constexpr int kThreads = 256;
constexpr int kBlocks = 2048;

struct Tally {
    unsigned long long* count;  // [0] mismatches, [1] smallest mismatching index
};

__device__ __forceinline__ void report(Tally t, unsigned long long bad, unsigned long long first) {
    if (bad) {
        atomicAdd(t.count, bad);
        atomicMin(t.count + 1, first);
    }
}

__device__ __forceinline__ float clampf(float v, float lo, float hi) { return __builtin_amdgcn_fmed3f(v, lo, hi); }

// ---------------------------------------------------------------- sweeps
// Each returns true when index i checks out.  Indices outside a sweep's domain pass.

// 0: v_cvt_pk_fp8_f32 == f_to_e4m3 on every non-NaN fp32 after the kernels' +-448 clamp.
__device__ bool sweep_e4m3(uint64_t i) {
    const float f = as_f(static_cast<uint32_t>(i));
    if (is_nan(f)) return true;
    const float c = clampf(f, -448.0f, 448.0f);
    return (hw_e4m3x4(c, c, 0.0f, 0.0f) & 0xffffu) == (f_to_e4m3(c) * 0x101u);
}

// 1: v_cvt_pk_bf8_f32 == f_to_e5m2 after the +-57344 clamp.
__device__ bool sweep_e5m2(uint64_t i) {
    const float f = as_f(static_cast<uint32_t>(i));
    if (is_nan(f)) return true;
    const float c = clampf(f, -57344.0f, 57344.0f);
    return (hw_e5m2x4(c, c, 0.0f, 0.0f) & 0xffffu) == (f_to_e5m2(c) * 0x101u);
}

// 2: v_cvt_pk_bf16_f32 (f_to_bf16_rne) == the software RNE f_to_bf16 on every non-NaN fp32.
__device__ bool sweep_bf16(uint64_t i) {
    const float f = as_f(static_cast<uint32_t>(i));
    if (is_nan(f)) return true;
    return f_to_bf16_rne(f) == f_to_bf16(f);
}

// 3: v_cvt_scalef32_pk_fp4_f32 (pack_e2m1x8) == f_to_e2m1 of the value clamped to +-6, on
// every non-NaN fp32, in both nibble orders (element 0 -> high nibble when HI_FIRST).
__device__ bool sweep_e2m1(uint64_t i) {
    const float f = as_f(static_cast<uint32_t>(i));
    if (is_nan(f)) return true;
    const float q[8] = {f, -f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    const uint32_t want_f = f_to_e2m1(clampf(f, -6.0f, 6.0f)), want_n = f_to_e2m1(clampf(-f, -6.0f, 6.0f));
    const uint32_t hi = pack_e2m1x8<true>(q) & 0xffu, lo = pack_e2m1x8<false>(q) & 0xffu;
    return hi == ((want_f << 4) | want_n) && lo == ((want_n << 4) | want_f);
}

// 4: v_cvt_f32_fp8 (hw_e4m3_to_f) == e4m3_to_f for every code byte (NaN codes: both NaN).
__device__ bool sweep_e4m3_decode(uint64_t i) {
    if (i >= 256) return true;
    const uint32_t c = static_cast<uint32_t>(i);
    const float h = hw_e4m3_to_f<0>(c), s = e4m3_to_f(c);
    return is_nan(s) ? is_nan(h) : as_u(h) == as_u(s);
}

// 5/6: v_cvt_scalef32_pk_fp8_bf16 / _f16 (scaled_e4m3x4) == f_to_e4m3(x / 2^(e-127)) for
// every 16-bit x (non-NaN) and every normal E8M0 scale e in [1, 254], wherever the exact
// quotient lies in [-448, 448] (the MXFP8 fast path's scale is >= amax/448).  The exact
// quotient of a power-of-two division is x scaled by 2^(127-e); below the fp32 normal
// range it is far under half of E4M3's smallest subnormal (2^-10), so its code is a zero.
template <int IN>
__device__ bool sweep_scaled_e4m3(uint64_t i) {
    if (i >= (uint64_t(1) << 16) * 254) return true;
    const uint32_t xb = static_cast<uint32_t>(i & 0xffffu), e = static_cast<uint32_t>(i >> 16) + 1;
    const float x = IN == CKH_BF16 ? bf16_to_f(xb) : f16_to_f(xb);
    if (is_nan(x) || !(fabsf(x) <= 3.0e38f)) return true;
    const double q = ldexp(static_cast<double>(x), 127 - static_cast<int>(e));
    if (!(fabs(q) <= 448.0)) return true;
    const uint32_t sign = (xb >> 8) & 0x80u;  // bit 15 of either format
    const uint32_t want = fabs(q) < 0x1p-126 ? sign : f_to_e4m3(static_cast<float>(q));
    const uint32_t got = scaled_e4m3x4<IN>(xb | (xb << 16), 0u, e8m0_to_f(e));
    return (got & 0xffffu) == want * 0x101u;
}

// 7: rcp_newton(T) == IEEE 1.0f / T for every T in [2^-70, 2^71).
__device__ bool sweep_rcp(uint64_t i) {
    const uint64_t lo = 57u << 23, hi = 198u << 23;  // biased exponents of 2^-70 and 2^71
    if (i >= hi - lo) return true;
    const float T = as_f(static_cast<uint32_t>(lo + i));
    return as_u(rcp_newton(T)) == as_u(1.0f / T);
}

// 8/9: the E2M1 code of markstein_quotient(v, T, RN(1/T)) == that of the IEEE quotient v/T,
// for every T in [1, 2) and every bf16 (8) / f16 (9) v of either sign with |v| in
// [2^-6, 2^5), plus +-0.  That covers every E2M1 rounding boundary (|v/T| in 1/4 .. 5);
// both steps scale exactly by powers of two while the intermediates stay normal, which
// the kernels' guards ensure, so this range stands for all of them.
template <int IN>
__device__ bool sweep_markstein(uint64_t i) {
    constexpr uint32_t kSig = IN == CKH_BF16 ? 128u : 1024u;           // significands per binade
    constexpr uint32_t kE0 = IN == CKH_BF16 ? 121u : 9u;               // biased exponent of 2^-6
    constexpr uint32_t kV = 2u * 11u * kSig + 2u;                       // v values per T
    if (i >= uint64_t(kV) << 23) return true;
    const uint32_t ti = static_cast<uint32_t>(i % (uint64_t(1) << 23)), vi = static_cast<uint32_t>(i >> 23);
    const float T = as_f(0x3f800000u | ti);
    float v;
    if (vi >= 2u * 11u * kSig) {
        v = vi & 1u ? -0.0f : 0.0f;
    } else {
        const uint32_t sign = vi & 1u, k = vi >> 1, e = kE0 + k / kSig, m = k % kSig;
        v = IN == CKH_BF16 ? bf16_to_f((sign << 15) | (e << 7) | m) : f16_to_f((sign << 15) | (e << 10) | m);
    }
    const float y = 1.0f / T;
    const float qm = markstein_quotient(v, T, y), qi = v / T;
    return f_to_e2m1(clampf(qm, -6.0f, 6.0f)) == f_to_e2m1(clampf(qi, -6.0f, 6.0f));
}

// 10: nvfp4_c_steps(amax, g, RN(1/g)) == (amax / 6) / g (two IEEE divisions) for every f16
// amax significand (which include every bf16 one) and every g significand, both in [1, 2);
// the steps scale exactly by powers of two within the kernels' guards.
__device__ bool sweep_c_steps(uint64_t i) {
    if (i >= uint64_t(1024) << 23) return true;
    const float g = as_f(0x3f800000u | static_cast<uint32_t>(i % (uint64_t(1) << 23)));
    const float amax = as_f(0x3f800000u | (static_cast<uint32_t>(i >> 23) << 13));
    return as_u(nvfp4_c_steps(amax, g, 1.0f / g)) == as_u((amax / 6.0f) / g);
}

// 11: mx_exponent's closed form for amax with biased exponent >= 10 == its division form
// (s = amax/448 by IEEE division, e = ceil(log2 s) + 127 from s's bit fields, clamped to
// [0, 254]) for every finite non-negative amax in that range.
__device__ bool sweep_mx_exponent(uint64_t i) {
    const uint32_t a = static_cast<uint32_t>(i);
    if (a < (10u << 23) || a >= 0x7f800000u) return true;
    const uint32_t s = as_u(as_f(a) / 448.0f);
    uint32_t want;
    if (s <= 0x00400000u) want = 0;
    else if (s < 0x00800000u) want = 1;
    else {
        want = (s >> 23) + ((s & 0x7fffffu) != 0);
        want = want > 254u ? 254u : want;
    }
    return mx_exponent(a) == want;
}

// 12: the NVFP4 GEMM's operand decode (scale_pair, decode8) == E2M1(code) * E4M3(scale)
// exactly, for every code byte and every pair of finite scale bytes; the low nibble of
// each byte is the earlier element.
__device__ bool sweep_nvfp4_decode(uint64_t i) {
    if (i >= (uint64_t(1) << 24)) return true;
    const uint32_t code = static_cast<uint32_t>(i & 0xffu), s0 = static_cast<uint32_t>((i >> 8) & 0xffu),
                   s1 = static_cast<uint32_t>(i >> 16);
    if ((s0 & 0x7fu) == 0x7fu || (s1 & 0x7fu) == 0x7fu) return true;
    const v2h s = scale_pair(s0 | (s1 << 8) | 0x7f7f0000u, 0);
    const uint32_t w = code | ((code ^ 0x88u) << 8) | (0x10u << 16) | (0xf7u << 24);
    const v8h d = decode8(w, s);
    bool ok = true;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint32_t nib = (w >> (4 * k)) & 0xfu;
        const float want = e2m1_to_f(nib) * e4m3_to_f(k & 1 ? s1 : s0);
        ok &= as_u(static_cast<float>(d[k])) == as_u(want);
    }
    return ok;
}

template <int S>
__device__ bool check(uint64_t i) {
    if constexpr (S == 0) return sweep_e4m3(i);
    else if constexpr (S == 1) return sweep_e5m2(i);
    else if constexpr (S == 2) return sweep_bf16(i);
    else if constexpr (S == 3) return sweep_e2m1(i);
    else if constexpr (S == 4) return sweep_e4m3_decode(i);
    else if constexpr (S == 5) return sweep_scaled_e4m3<CKH_BF16>(i);
    else if constexpr (S == 6) return sweep_scaled_e4m3<CKH_F16>(i);
    else if constexpr (S == 7) return sweep_rcp(i);
    else if constexpr (S == 8) return sweep_markstein<CKH_BF16>(i);
    else if constexpr (S == 9) return sweep_markstein<CKH_F16>(i);
    else if constexpr (S == 10) return sweep_c_steps(i);
    else if constexpr (S == 11) return sweep_mx_exponent(i);
    else return sweep_nvfp4_decode(i);
}

template <int S>
__global__ __launch_bounds__(kThreads) void sweep_kernel(uint64_t begin, uint64_t end, Tally t) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kThreads;
    unsigned long long bad = 0, first = ~0ull;
    for (uint64_t i = begin + static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < end; i += stride) {
        if (!check<S>(i)) {
            ++bad;
            first = i < first ? i : first;
        }
    }
    report(t, bad, first);
}

}  // namespace

// Domain size (number of indices) of sweep `which`, or 0 for an unknown sweep.
extern "C" uint64_t ckh_hw_sweep_size(int which) {
    switch (which) {
        case 0: case 1: case 2: case 3: case 11: return uint64_t(1) << 32;
        case 4: return 256;
        case 5: case 6: return (uint64_t(1) << 16) * 254;
        case 7: return uint64_t(198u - 57u) << 23;
        case 8: return uint64_t(2u * 11u * 128u + 2u) << 23;
        case 9: return uint64_t(2u * 11u * 1024u + 2u) << 23;
        case 10: return uint64_t(1024) << 23;
        case 12: return uint64_t(1) << 24;
        default: return 0;
    }
}

// Check indices [begin, end) of sweep `which`, adding to counts[0] (mismatches) and
// lowering counts[1] (smallest mismatching index); counts is 2 x u64 on the device,
// initialised by the caller to {0, UINT64_MAX}.  Returns 0, or 1 for a bad argument or a
// rejected launch.
extern "C" int ckh_hw_sweep(int which, uint64_t begin, uint64_t end, void* counts, uintptr_t stream) {
    if (!counts || end < begin || end > ckh_hw_sweep_size(which)) return 1;
    const Tally t{static_cast<unsigned long long*>(counts)};
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
#define L(S) hipLaunchKernelGGL(sweep_kernel<S>, dim3(kBlocks), dim3(kThreads), 0, st, begin, end, t)
    switch (which) {
        case 0: L(0); break;
        case 1: L(1); break;
        case 2: L(2); break;
        case 3: L(3); break;
        case 4: L(4); break;
        case 5: L(5); break;
        case 6: L(6); break;
        case 7: L(7); break;
        case 8: L(8); break;
        case 9: L(9); break;
        case 10: L(10); break;
        case 11: L(11); break;
        case 12: L(12); break;
        default: return 1;
    }
#undef L
    return hipGetLastError() == hipSuccess ? 0 : 1;
}
