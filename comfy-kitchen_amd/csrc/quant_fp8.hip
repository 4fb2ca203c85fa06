// Per-tensor FP8 quantize / dequantize: HBM-streaming kernels for gfx950.
//
// Arithmetic is the reference eager backend's, step for step, so codes are bit-exact:
//   quantize   (backends/eager/quantization.py:53-55):
//       r = (1/scale) rounded to x's dtype; t = x*r rounded to x's dtype;
//       t = clamp(t, +-max); code = round-to-nearest-even FP8(t)
//   dequantize (quantization.py:60): out = x.to(out) * scale.to(out), rounded to out.
// For bf16/f16 inputs the product of two 16-bit floats is exact in fp32, so rounding
// the fp32 product to the 16-bit type equals the 16-bit multiply of the reference.
//
// Launch shape: aligned 16-bit inputs of at least 1024 elements take a persistent kernel
// whose waves walk 1024-element tiles with the next tile's loads in flight
// (quantize_fp8_pipe_kernel); other quantize calls and every dequantize use 128-thread
// workgroups with 16 elements per thread, one tile per thread.
#include "ckh_common.h"

namespace ckh {

// 128-thread workgroups: same-process A/B on C1 (quantize / dequantize, us): 128 threads
// 8.74 / 9.05, 256 threads 8.74 / 9.21, 512 threads 8.92 / 9.38
constexpr int kThreads = 128;
constexpr int kPerThread = 16;

template <int OUT>
__device__ __forceinline__ uint32_t encode_fp8(float t) {
    if constexpr (OUT == CKH_E4M3) {
        t = t > 448.0f ? 448.0f : (t < -448.0f ? -448.0f : t);  // NaN passes through
        return f_to_e4m3(t);
    } else {
        t = t > 57344.0f ? 57344.0f : (t < -57344.0f ? -57344.0f : t);
        return f_to_e5m2(t);
    }
}

// The code of a NaN product t = x * r, as the reference's eager arithmetic writes it
// (torch's vectorised CPU kernels on x86; the c10 E4M3/E5M2 cast is 0x7F | sign for NaN):
//  - bf16: the bf16 narrowing of the product (vec512_bfloat16.h cvtfp32_bf16) turns every
//    NaN into 0xFFFF, so every NaN code is 0xFF.  (Eager's scalar remainder, the < 64
//    elements of each thread's chunk past its last whole vector pair, narrows through
//    c10::BFloat16 instead, whose NaN is 0x7FC0: 0x7F there.)
//  - f16 / f32: the NaN keeps its sign through the multiply, clamp and narrowing.  The
//    product's NaN is r's when r = 1/scale is NaN (scale NaN, r keeps its sign), else x's,
//    else x86's default NaN, which is negative (0 * inf).
template <int IN>
__device__ __forceinline__ uint32_t fp8_nan_code(float x, float scale) {
    if constexpr (IN == CKH_BF16) {
        return 0xffu;
    } else {
        const uint32_t s = is_nan(scale) ? as_u(scale) : (is_nan(x) ? as_u(x) : 0x80000000u);
        return 0x7fu | ((s >> 24) & 0x80u);
    }
}

// One element through the reference's steps (software converts), NaN bytes included.
template <int IN, int OUT>
__device__ __forceinline__ uint32_t quantize_one(float x, float r, float scale) {
    const float t = round_to<IN>(x * r);
    return is_nan(t) ? fp8_nan_code<IN>(x, scale) : encode_fp8<OUT>(t);
}

template <int IN, int OUT, bool VEC>
__global__ __launch_bounds__(kThreads) void quantize_fp8_kernel(const void* __restrict__ x,
                                                                const float* __restrict__ scale,
                                                                uint8_t* __restrict__ out, int64_t n) {
    // a wave's 1024 elements: lane l takes the 8-element pieces l and 64 + l, so every load
    // and store instruction covers one contiguous run
    const int64_t wbase = (static_cast<int64_t>(blockIdx.x) * kThreads + (threadIdx.x & ~63u)) * kPerThread;
    const int64_t ia = wbase + 8 * (threadIdx.x & 63u), ib = ia + 512;
    constexpr int ES = ElemSize<IN>::value;
    if (VEC && ib + 8 <= n) {
        // the data loads go out before the scale is read and inverted, so the two
        // latencies overlap instead of adding up
        const Raw8<IN> ra = load8_raw<IN>(static_cast<const char*>(x) + ia * ES);
        const Raw8<IN> rb = load8_raw<IN>(static_cast<const char*>(x) + ib * ES);
        const float sc = scale[0];
        const float r = round_to<IN>(1.0f / sc);
        float v[16];
        unpack8<IN>(ra, *reinterpret_cast<float(*)[8]>(&v[0]));
        unpack8<IN>(rb, *reinterpret_cast<float(*)[8]>(&v[8]));
        // hardware path: product rounded to x's dtype, clamped, converted in pairs
        float t[16];
        bool any_nan = false;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            t[e] = round_to_hw<IN>(v[e] * r);
            any_nan |= is_nan(t[e]);
        }
        constexpr float MX = OUT == CKH_E4M3 ? 448.0f : 57344.0f;
        uint32_t w[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float c[4];
#pragma unroll
            for (int b = 0; b < 4; ++b) c[b] = __builtin_amdgcn_fmed3f(t[4 * q + b], -MX, MX);
            w[q] = OUT == CKH_E4M3 ? hw_e4m3x4(c[0], c[1], c[2], c[3]) : hw_e5m2x4(c[0], c[1], c[2], c[3]);
        }
        if (any_nan) {  // the reference's NaN bytes (fp8_nan_code)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                uint32_t acc = 0;
#pragma unroll
                for (int b = 0; b < 4; ++b) acc |= quantize_one<IN, OUT>(v[4 * q + b], r, sc) << (8 * b);
                w[q] = acc;
            }
        }
        st_stream8(out + ia, make_uint2(w[0], w[1]));
        st_stream8(out + ib, make_uint2(w[2], w[3]));
    } else {
        const float sc = scale[0];
        const float r = round_to<IN>(1.0f / sc);
        for (int64_t i = ia; i < n && i < ia + 8; ++i)
            out[i] = static_cast<uint8_t>(quantize_one<IN, OUT>(load1<IN>(x, i), r, sc));
        for (int64_t i = ib; i < n && i < ib + 8; ++i)
            out[i] = static_cast<uint8_t>(quantize_one<IN, OUT>(load1<IN>(x, i), r, sc));
    }
}

// One wave-tile (1024 elements; lane l: pieces l and 64 + l) of the quantizer from its
// raw loads: codes stored, a NaN-containing lane re-encoded by the software path.
template <int IN, int OUT>
__device__ __forceinline__ void quantize_tile(const Raw8<IN>& ra, const Raw8<IN>& rb, float r, float sc,
                                              uint8_t* out, int64_t ia, int64_t ib) {
    float v[16];
    unpack8<IN>(ra, *reinterpret_cast<float(*)[8]>(&v[0]));
    unpack8<IN>(rb, *reinterpret_cast<float(*)[8]>(&v[8]));
    float t[16];
    bool any_nan = false;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        t[e] = round_to_hw<IN>(v[e] * r);
        any_nan |= is_nan(t[e]);
    }
    constexpr float MX = OUT == CKH_E4M3 ? 448.0f : 57344.0f;
    uint32_t w[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        float c[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) c[b] = __builtin_amdgcn_fmed3f(t[4 * q + b], -MX, MX);
        w[q] = OUT == CKH_E4M3 ? hw_e4m3x4(c[0], c[1], c[2], c[3]) : hw_e5m2x4(c[0], c[1], c[2], c[3]);
    }
    if (any_nan) {  // the reference's NaN bytes (fp8_nan_code)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            uint32_t acc = 0;
#pragma unroll
            for (int b = 0; b < 4; ++b) acc |= quantize_one<IN, OUT>(v[4 * q + b], r, sc) << (8 * b);
            w[q] = acc;
        }
    }
    st_stream8(out + ia, make_uint2(w[0], w[1]));
    st_stream8(out + ib, make_uint2(w[2], w[3]));
}

// Persistent form for aligned 16-bit inputs: the grid's W waves (about kQWavesPerCU per CU,
// with the whole wave-tiles spread evenly over them) each walk tiles t = w, w + W, ...,
// issuing the loads of tile t + W before converting and storing tile t, so every wave
// keeps a tile in flight while it computes.  Elements past the last whole tile are done
// by wave 0 with the scalar path.  Same-process A/B on C1 against the one-tile-per-lane
// kernel below: 93.2% vs 90.8% and 91.7% vs 89.6% of the copy floor (16 waves per CU;
// 8, 12, 24 and 32 measured 87-90%).
constexpr int kQWavesPerCU = 16;

template <int IN, int OUT>
__global__ __launch_bounds__(256) void quantize_fp8_pipe_kernel(const void* __restrict__ x,
                                                                const float* __restrict__ scale,
                                                                uint8_t* __restrict__ out, int64_t n) {
    constexpr int ES = ElemSize<IN>::value;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t W = gridDim.x * 4u;
    const uint32_t w0 = blockIdx.x * 4u + (threadIdx.x >> 6);
    const uint32_t tiles = static_cast<uint32_t>(n >> 10);
    const char* xb = static_cast<const char*>(x);
    uint32_t t = w0;
    Raw8<IN> ra{}, rb{};
    if (t < tiles) {
        ra = load8_raw<IN>(xb + (static_cast<int64_t>(t) * 1024 + 8 * lane) * ES);
        rb = load8_raw<IN>(xb + (static_cast<int64_t>(t) * 1024 + 512 + 8 * lane) * ES);
    }
    const float sc = scale[0];
    const float r = round_to<IN>(1.0f / sc);
    while (t < tiles) {
        const uint32_t tn = t + W;
        Raw8<IN> na = ra, nb = rb;
        if (tn < tiles) {
            na = load8_raw<IN>(xb + (static_cast<int64_t>(tn) * 1024 + 8 * lane) * ES);
            nb = load8_raw<IN>(xb + (static_cast<int64_t>(tn) * 1024 + 512 + 8 * lane) * ES);
        }
        const int64_t ia = static_cast<int64_t>(t) * 1024 + 8 * lane;
        quantize_tile<IN, OUT>(ra, rb, r, sc, out, ia, ia + 512);
        t = tn;
        ra = na;
        rb = nb;
    }
    if (w0 == 0) {
        for (int64_t i = static_cast<int64_t>(tiles) * 1024 + lane; i < n; i += 64)
            out[i] = static_cast<uint8_t>(quantize_one<IN, OUT>(load1<IN>(x, i), r, sc));
    }
}

template <int IN>
__device__ __forceinline__ float decode_fp8(uint32_t c) {
    return IN == CKH_E4M3 ? e4m3_to_f(c) : e5m2_to_f(c);
}

template <int OUT>
__device__ __forceinline__ void store_out(void* out, int64_t i, float v) {
    if constexpr (OUT == CKH_F32) reinterpret_cast<float*>(out)[i] = v;
    else if constexpr (OUT == CKH_BF16) reinterpret_cast<uint16_t*>(out)[i] = static_cast<uint16_t>(f_to_bf16(v));
    else reinterpret_cast<uint16_t*>(out)[i] = static_cast<uint16_t>(f_to_f16(v));
}

// Store 16 rounded outputs: v[0..7] at element i, v[8..15] at element j (each 16-byte
// aligned); 16-bit outputs rounded by the hardware converts (callers route NaN-containing
// data elsewhere).
template <int OUT>
__device__ __forceinline__ void store16_hw(void* out, int64_t i, int64_t j, const float (&v)[16]) {
    if constexpr (OUT == CKH_F32) {
        float* p = static_cast<float*>(out) + i;
        float* q = static_cast<float*>(out) + j;
        st_stream16(p, make_uint4(as_u(v[0]), as_u(v[1]), as_u(v[2]), as_u(v[3])));
        st_stream16(p + 4, make_uint4(as_u(v[4]), as_u(v[5]), as_u(v[6]), as_u(v[7])));
        st_stream16(q, make_uint4(as_u(v[8]), as_u(v[9]), as_u(v[10]), as_u(v[11])));
        st_stream16(q + 4, make_uint4(as_u(v[12]), as_u(v[13]), as_u(v[14]), as_u(v[15])));
    } else {
        uint32_t w[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            uint32_t lo = OUT == CKH_BF16 ? f_to_bf16_rne(v[2 * k]) : f_to_f16(v[2 * k]);
            uint32_t hi = OUT == CKH_BF16 ? f_to_bf16_rne(v[2 * k + 1]) : f_to_f16(v[2 * k + 1]);
            w[k] = lo | (hi << 16);
        }
        st_stream16(static_cast<uint16_t*>(out) + i, make_uint4(w[0], w[1], w[2], w[3]));
        st_stream16(static_cast<uint16_t*>(out) + j, make_uint4(w[4], w[5], w[6], w[7]));
    }
}

// The same with the software converts (keeps the software's NaN bits).
template <int OUT>
__device__ __forceinline__ void store16(void* out, int64_t i, int64_t j, const float (&v)[16]) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        store_out<OUT>(out, i + k, v[k]);
        store_out<OUT>(out, j + k, v[8 + k]);
    }
}

// The scale as eager reads it, scale.to(out dtype): widened to fp32 from its own dtype
// (exact), then rounded to the output dtype.
__device__ __forceinline__ float load_scale(const void* p, int code) {
    if (code == CKH_F32) return *static_cast<const float*>(p);
    const uint32_t h = *static_cast<const uint16_t*>(p);
    return code == CKH_BF16 ? bf16_to_f(h) : f16_to_f(h);
}

template <int IN, int OUT, bool VEC>
__global__ __launch_bounds__(kThreads) void dequantize_fp8_kernel(const uint8_t* __restrict__ x,
                                                                  const void* __restrict__ scale, int scale_code,
                                                                  void* __restrict__ out, int64_t n) {
    // a wave's 1024 codes: lane l takes the 8-code pieces l and 64 + l, so every load and
    // store instruction covers one contiguous run
    const int64_t wbase = (static_cast<int64_t>(blockIdx.x) * kThreads + (threadIdx.x & ~63u)) * kPerThread;
    const int64_t ia = wbase + 8 * (threadIdx.x & 63u), ib = ia + 512;
    if (VEC && ib + 8 <= n) {
        typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
        // the code loads go out before the scale is read and rounded
        const u32x2 ca = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(x + ia));
        const u32x2 cb = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(x + ib));
        const float s = round_to<OUT>(load_scale(scale, scale_code));
        uint32_t cw[4] = {ca.x, ca.y, cb.x, cb.y};
        // a NaN code (0x7f / 0xff in E4M3) takes the software path, which fixes its bytes
        bool nan_code = false;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t m = cw[q] & 0x7f7f7f7fu;
            if constexpr (IN == CKH_E4M3) nan_code |= ((m + 0x01010101u) & 0x80808080u) != 0;  // some byte == 0x7f
            else nan_code = true;
        }
        float v[16];
        if (!nan_code) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                v[4 * q] = hw_e4m3_to_f<0>(cw[q]) * s;
                v[4 * q + 1] = hw_e4m3_to_f<1>(cw[q]) * s;
                v[4 * q + 2] = hw_e4m3_to_f<2>(cw[q]) * s;
                v[4 * q + 3] = hw_e4m3_to_f<3>(cw[q]) * s;
            }
            store16_hw<OUT>(out, ia, ib, v);
        } else {
#pragma unroll
            for (int j = 0; j < 16; ++j) v[j] = decode_fp8<IN>((cw[j >> 2] >> (8 * (j & 3))) & 0xffu) * s;
            store16<OUT>(out, ia, ib, v);
        }
    } else {
        const float s = round_to<OUT>(load_scale(scale, scale_code));
        for (int64_t i = ia; i < n && i < ia + 8; ++i) store_out<OUT>(out, i, decode_fp8<IN>(x[i]) * s);
        for (int64_t i = ib; i < n && i < ib + 8; ++i) store_out<OUT>(out, i, decode_fp8<IN>(x[i]) * s);
    }
}

}  // namespace ckh

using namespace ckh;

#define CKH_DISPATCH_VEC(vec, ...) \
    do {                            \
        if (vec) {                  \
            constexpr bool V = true; \
            __VA_ARGS__;            \
        } else {                    \
            constexpr bool V = false; \
            __VA_ARGS__;            \
        }                           \
    } while (0)

extern "C" int ckh_quantize_fp8(const void* x, void* out, const void* scale, int64_t numel, int in_code,
                                int out_code, uintptr_t stream) {
    CKH_REQUIRE(numel >= 0, "quantize_fp8: numel < 0");
    if (numel == 0) return CKH_OK;
    CKH_REQUIRE(x && scale && out, "quantize_fp8: null pointer");
    CKH_REQUIRE(in_code == CKH_F32 || in_code == CKH_F16 || in_code == CKH_BF16,
                "quantize_fp8: unsupported input dtype code %d", in_code);
    CKH_REQUIRE(out_code == CKH_E4M3 || out_code == CKH_E5M2, "quantize_fp8: unsupported output dtype code %d",
                out_code);
    const bool vec = aligned(x, 16) && aligned(out, 16);
    if (vec && in_code != CKH_F32 && numel >= 1024) {
        // waves: at most kQWavesPerCU per CU, as many tiles per wave as that forces, and the
        // tiles spread evenly over the waves
        const int64_t tiles = numel >> 10;
        const int64_t per_wave = cdiv(tiles, static_cast<int64_t>(device_cus()) * kQWavesPerCU);
        const dim3 pgrid(static_cast<unsigned>(cdiv(cdiv(tiles, per_wave), 4)));
        hipStream_t pst = reinterpret_cast<hipStream_t>(stream);
        const float* psp = static_cast<const float*>(scale);
        uint8_t* po = static_cast<uint8_t*>(out);
#define LAUNCH_P(I, O) hipLaunchKernelGGL((quantize_fp8_pipe_kernel<I, O>), pgrid, dim3(256), 0, pst, x, psp, po, numel)
        if (out_code == CKH_E4M3) {
            if (in_code == CKH_F16) LAUNCH_P(CKH_F16, CKH_E4M3);
            else LAUNCH_P(CKH_BF16, CKH_E4M3);
        } else {
            if (in_code == CKH_F16) LAUNCH_P(CKH_F16, CKH_E5M2);
            else LAUNCH_P(CKH_BF16, CKH_E5M2);
        }
#undef LAUNCH_P
        return check_launch("quantize_fp8");
    }
    dim3 grid(static_cast<unsigned>(cdiv(numel, kThreads * kPerThread)));
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const float* sp = static_cast<const float*>(scale);
    uint8_t* o = static_cast<uint8_t*>(out);
#define LAUNCH_Q(I, O)                                                                              \
    CKH_DISPATCH_VEC(vec, hipLaunchKernelGGL((quantize_fp8_kernel<I, O, V>), grid, dim3(kThreads), 0, st, \
                                             x, sp, o, numel))
    if (out_code == CKH_E4M3) {
        if (in_code == CKH_F32) LAUNCH_Q(CKH_F32, CKH_E4M3);
        else if (in_code == CKH_F16) LAUNCH_Q(CKH_F16, CKH_E4M3);
        else LAUNCH_Q(CKH_BF16, CKH_E4M3);
    } else {
        if (in_code == CKH_F32) LAUNCH_Q(CKH_F32, CKH_E5M2);
        else if (in_code == CKH_F16) LAUNCH_Q(CKH_F16, CKH_E5M2);
        else LAUNCH_Q(CKH_BF16, CKH_E5M2);
    }
#undef LAUNCH_Q
    return check_launch("quantize_fp8");
}

extern "C" int ckh_dequantize_fp8(const void* x, void* out, const void* scale, int64_t numel, int in_code,
                                  int out_code, int scale_code, uintptr_t stream) {
    CKH_REQUIRE(numel >= 0, "dequantize_fp8: numel < 0");
    if (numel == 0) return CKH_OK;
    CKH_REQUIRE(x && scale && out, "dequantize_fp8: null pointer");
    CKH_REQUIRE(in_code == CKH_E4M3 || in_code == CKH_E5M2, "dequantize_fp8: unsupported input dtype code %d",
                in_code);
    CKH_REQUIRE(out_code == CKH_F32 || out_code == CKH_F16 || out_code == CKH_BF16,
                "dequantize_fp8: unsupported output dtype code %d", out_code);
    CKH_REQUIRE(scale_code == CKH_F32 || scale_code == CKH_F16 || scale_code == CKH_BF16,
                "dequantize_fp8: unsupported scale dtype code %d", scale_code);
    CKH_REQUIRE(aligned(scale, scale_code == CKH_F32 ? 4 : 2), "dequantize_fp8: scale misaligned");
    const bool vec = aligned(x, 16) && aligned(out, 16);
    dim3 grid(static_cast<unsigned>(cdiv(numel, kThreads * kPerThread)));
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const uint8_t* xi = static_cast<const uint8_t*>(x);
#define LAUNCH_DQ(I, O)                                                                               \
    CKH_DISPATCH_VEC(vec, hipLaunchKernelGGL((dequantize_fp8_kernel<I, O, V>), grid, dim3(kThreads), 0, st, \
                                             xi, scale, scale_code, out, numel))
    if (in_code == CKH_E4M3) {
        if (out_code == CKH_F32) LAUNCH_DQ(CKH_E4M3, CKH_F32);
        else if (out_code == CKH_F16) LAUNCH_DQ(CKH_E4M3, CKH_F16);
        else LAUNCH_DQ(CKH_E4M3, CKH_BF16);
    } else {
        if (out_code == CKH_F32) LAUNCH_DQ(CKH_E5M2, CKH_F32);
        else if (out_code == CKH_F16) LAUNCH_DQ(CKH_E5M2, CKH_F16);
        else LAUNCH_DQ(CKH_E5M2, CKH_BF16);
    }
#undef LAUNCH_DQ
    return check_launch("dequantize_fp8");
}
