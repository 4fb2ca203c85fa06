// Shared device helpers for the gfx950 kernels: dtype codes, exact float format
// conversions, the 32_4_4 scale swizzle, and the thread-local error channel.
//
// Every conversion here is written from the format definitions (IEEE-754 binary16 /
// bfloat16, OCP FP8 E4M3FN / E5M2, OCP MX E8M0, OCP FP4 E2M1) with round-to-nearest-
// even, so results do not depend on the FP mode register or on hardware convert
// instructions.  Callers clamp to the finite range before FP8 encoding, as the
// reference's eager backend does (backends/eager/quantization.py:54,154,314).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ckh.h"

namespace ckh {

// ------------------------------------------------------------------ errors
void set_error(const char* fmt, ...);
void clear_error();
int check_launch(const char* what);

#define CKH_REQUIRE(cond, ...)            \
    do {                                  \
        if (!(cond)) {                    \
            ::ckh::set_error(__VA_ARGS__); \
            return CKH_ERR_INVALID;       \
        }                                 \
    } while (0)

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }
inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline int64_t rup(int64_t a, int64_t b) { return cdiv(a, b) * b; }

// --------------------------------------------------------- bit reinterpret
__device__ __forceinline__ float as_f(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t as_u(float f) { return __float_as_uint(f); }

// ------------------------------------------------------ 16-bit float formats
// bfloat16 <-> float.  Widening is exact.  Narrowing is round-to-nearest-even; a NaN
// becomes a quiet NaN with its sign kept.
__device__ __forceinline__ float bf16_to_f(uint32_t h) { return as_f(h << 16); }
__device__ __forceinline__ uint32_t f_to_bf16(float f) {
    uint32_t u = as_u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f(f_to_bf16(f)); }

// bfloat16 round-to-nearest-even through the hardware convert (v_cvt_pk_bf16_f32).
// Checked against f_to_bf16 on all 2^32 inputs on gfx950: identical for every
// non-NaN input, NaN stays NaN.
__device__ __forceinline__ uint32_t f_to_bf16_rne(float f);

// Hide a value from instruction selection.  Without it the backend folds
// "fp32 multiply (or FMA), then narrow to f16" into one v_fma_mix*_f16 with a +0
// addend: that rounds once instead of twice and turns a -0 product into +0, both of
// which break bit-exactness with the reference's fp32-then-f16 arithmetic.
__device__ __forceinline__ float opaque(float f) {
    __asm__("" : "+v"(f));
    return f;
}

// binary16 <-> float through the IEEE conversion instructions (round-to-nearest-even,
// subnormals kept, which is the default FP mode of HIP kernels).
__device__ __forceinline__ float f16_to_f(uint32_t h) {
    _Float16 v;
    uint16_t hb = static_cast<uint16_t>(h);
    __builtin_memcpy(&v, &hb, 2);
    return static_cast<float>(v);
}
__device__ __forceinline__ uint32_t f_to_f16(float f) {
    _Float16 v = static_cast<_Float16>(opaque(f));
    uint16_t hb;
    __builtin_memcpy(&hb, &v, 2);
    return hb;
}
__device__ __forceinline__ float round_f16(float f) { return f16_to_f(f_to_f16(f)); }

__device__ __forceinline__ uint32_t f_to_bf16_rne(float f) {
    __bf16 b = static_cast<__bf16>(opaque(f));
    uint16_t hb;
    __builtin_memcpy(&hb, &b, 2);
    return hb;
}

// ------------------------------------------------- hardware convert helpers
// gfx950's convert instructions, each checked against the software encoders above on
// all 2^32 fp32 inputs (after the callers' clamps): v_cvt_pk_fp8_f32 == f_to_e4m3,
// v_cvt_pk_bf8_f32 == f_to_e5m2 and v_cvt_scalef32_pk_fp4_f32 (scale 1) == f_to_e2m1
// for every non-NaN input in range, v_cvt_pk_bf16_f32 == f_to_bf16 for every non-NaN
// input, and v_cvt_f32_fp8 == e4m3_to_f for every code.  A NaN input gives some NaN
// code whose sign / payload may differ from the software's, so callers that must keep
// the software's NaN bytes take a software path when a NaN is present.

// four E4M3 / E5M2 codes (byte i = code of x_i), inputs already clamped to the range
__device__ __forceinline__ uint32_t hw_e4m3x4(float a, float b, float c, float d) {
    int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true));
}
__device__ __forceinline__ uint32_t hw_e5m2x4(float a, float b, float c, float d) {
    int w = __builtin_amdgcn_cvt_pk_bf8_f32(a, b, 0, false);
    return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_bf8_f32(c, d, w, true));
}

// E4M3 code in byte B of w -> float (exact)
template <int B>
__device__ __forceinline__ float hw_e4m3_to_f(uint32_t w) {
    return __builtin_amdgcn_cvt_f32_fp8(static_cast<int>(w), B);
}

__device__ __forceinline__ bool is_nan(float f) { return (as_u(f) & 0x7fffffffu) > 0x7f800000u; }

// Round to the precision of dtype code C through the hardware converts (NaN -> some NaN).
template <int C>
__device__ __forceinline__ float round_to_hw(float f) {
    if constexpr (C == CKH_BF16) return bf16_to_f(f_to_bf16_rne(f));
    else if constexpr (C == CKH_F16) return round_f16(f);
    else return f;
}

// Round a float to the precision of dtype code `c` (f32 is the identity).
template <int C>
__device__ __forceinline__ float round_to(float f) {
    if constexpr (C == CKH_BF16) return round_bf16(f);
    else if constexpr (C == CKH_F16) return round_f16(f);
    else return f;
}

// -------------------------------------------------------------- OCP FP8
// E4M3FN: bias 7, 3 mantissa bits, no infinities, 0x7F/0xFF NaN, max 448.
// Input must be in [-448, 448] or NaN.  NaN encodes as 0xFF (the all-ones NaN that
// PyTorch's vectorised CPU clamp produces).
__device__ __forceinline__ uint32_t f_to_e4m3(float f) {
    uint32_t u = as_u(f);
    uint32_t s = (u >> 24) & 0x80u;
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return 0xffu;
    uint32_t m;
    if (a < 0x3c800000u) {  // |f| < 2^-6: subnormal codes, quantum 2^-9
        // Adding 2^14 (whose ulp is 2^-9) rounds |f| to a multiple of 2^-9 (RNE).
        m = as_u(as_f(a) + 16384.0f) - 0x46800000u;
    } else {  // rebias exponent 127 -> 7, round mantissa at bit 20 to nearest even
        m = (a - (120u << 23) + 0x7ffffu + ((a >> 20) & 1u)) >> 20;
    }
    return s | m;
}

// E5M2: bias 15, 2 mantissa bits, max 57344.  Input in [-57344, 57344] or NaN.
__device__ __forceinline__ uint32_t f_to_e5m2(float f) {
    uint32_t u = as_u(f);
    uint32_t s = (u >> 24) & 0x80u;
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return 0xffu;
    uint32_t m;
    if (a < 0x38800000u) {  // |f| < 2^-14: subnormal codes, quantum 2^-16
        m = as_u(as_f(a) + 128.0f) - 0x43000000u;
    } else {
        m = (a - (112u << 23) + 0xfffffu + ((a >> 21) & 1u)) >> 21;
    }
    return s | m;
}

__device__ __forceinline__ float e4m3_to_f(uint32_t c) {
    uint32_t s = (c & 0x80u) << 24;
    uint32_t e = (c >> 3) & 0xfu, m = c & 7u;
    if ((c & 0x7fu) == 0x7fu) return as_f(s | 0x7fc00000u);
    if (e == 0) return as_f(s | as_u(static_cast<float>(m) * 0.001953125f));  // m * 2^-9
    return as_f(s | ((e + 120u) << 23) | (m << 20));
}

__device__ __forceinline__ float e5m2_to_f(uint32_t c) {
    uint32_t s = (c & 0x80u) << 24;
    uint32_t e = (c >> 2) & 0x1fu, m = c & 3u;
    if (e == 0x1f) return as_f(s | (m ? 0x7fc00000u : 0x7f800000u));
    if (e == 0) return as_f(s | as_u(static_cast<float>(m) * 1.52587890625e-05f));  // m * 2^-16
    return as_f(s | ((e + 112u) << 23) | (m << 21));
}

// --------------------------------------------------------------- OCP E8M0
// Scale byte e -> 2^(e-127); e == 0 decodes to 0.0 (reference float_utils.py:376-382).
__device__ __forceinline__ float e8m0_to_f(uint32_t e) { return as_f(e == 0 ? 0u : (e << 23)); }

// --------------------------------------------------------------- OCP E2M1
// Round-to-nearest-even of |v| (already clamped to [0, 6]) onto the magnitudes
// {0, 0.5, 1, 1.5, 2, 3, 4, 6} = codes 0..7.  Each threshold is the midpoint between
// neighbouring magnitudes; at a midpoint the even code wins, hence > or >=.
__device__ __forceinline__ uint32_t e2m1_mag(float a) {
    return (a > 0.25f) + (a >= 0.75f) + (a > 1.25f) + (a >= 1.75f) + (a > 2.5f) + (a >= 3.5f) +
           (a > 5.0f);
}
// A NaN takes the reference's normal-range branch (float_utils.py:96-147 has no NaN
// case): the magnitude bits are rebiased, rounded to one mantissa bit and truncated to
// 8 bits, which gives code 2, 3 or 4 for the NaN magnitudes.
__device__ __forceinline__ uint32_t f_to_e2m1(float v) {
    const uint32_t sign = (as_u(v) >> 28) & 8u;
    if (is_nan(v)) {
        const uint32_t m = as_u(v) & 0x7fffffffu;
        return sign | (((m + (static_cast<uint32_t>(1 - 127) << 23) + (1u << 21) - 1u + ((m >> 22) & 1u)) >> 22) & 0xffu);
    }
    return sign | e2m1_mag(fabsf(v));
}
// Code -> value (sign in bit 3).
__device__ __forceinline__ float e2m1_to_f(uint32_t c) {
    // Codes 2..7 are normal: exponent (mag >> 1) - 1, one mantissa bit (mag & 1).
    const uint32_t mag = c & 7u;
    uint32_t bits = mag >= 2u ? (((126u + (mag >> 1)) << 23) | ((mag & 1u) << 22))
                              : (mag ? 0x3f000000u : 0u);
    return as_f(bits | ((c & 8u) << 28));
}

// -------------------------------------------------------- 32_4_4 swizzle
// Byte offset of logical scale (r, c) in a swizzled tensor whose logical width is
// C (n_cb = ceil(C/4) column blocks).  4 consecutive c (4j..4j+3) of one row are one
// aligned 32-bit word.
__host__ __device__ __forceinline__ int64_t swz_offset(int64_t r, int64_t c, int64_t n_cb) {
    return (((r >> 7) * n_cb + (c >> 2)) * 32 + (r & 31)) * 16 + ((r & 127) >> 5) * 4 + (c & 3);
}

// ---------------------------------------------------------- element loads
// Streaming (nontemporal) 16-byte loads: input read once by a kernel is not kept in the
// caches.  On gfx950 this lifts the quantizers' bandwidth by 10-15% over plain loads at
// the benchmark sizes.
typedef unsigned ckh_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_stream16(const void* p) {
    ckh_u32x4 a = __builtin_nontemporal_load(static_cast<const ckh_u32x4*>(p));
    return make_uint4(a.x, a.y, a.z, a.w);
}

// Streaming (nontemporal) stores of outputs written once.  Measured against plain stores
// on gfx950 in the benchmark runs: dequantize_per_tensor_fp8 -9%, apply_rope1 -9%,
// apply_rope -2.5%, quantize_nvfp4 -3%, quantize_per_tensor_fp8 -1%; the MXFP8
// quantizer's 8-byte code stores were 9% slower, so that kernel keeps plain stores.
typedef unsigned ckh_u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void st_stream16(void* p, uint4 v) {
    __builtin_nontemporal_store(ckh_u32x4{v.x, v.y, v.z, v.w}, static_cast<ckh_u32x4*>(p));
}
__device__ __forceinline__ void st_stream8(void* p, uint2 v) {
    __builtin_nontemporal_store(ckh_u32x2{v.x, v.y}, static_cast<ckh_u32x2*>(p));
}

// Load 8 consecutive elements of dtype code C as floats from an address aligned to
// 8 * sizeof(element), as a streaming read.
// v from another lane of the row of 16 selected by the DPP control CTRL (e.g. 0xB1 =
// quad_perm [1,0,3,2], the neighbouring lane).  Every lane the control reads must be active.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xf, 0xf, false));
}

// load8 in two steps, so a kernel can issue its data loads before anything that must
// wait (e.g. a device scalar it reads): the raw 16-byte chunks of 8 elements (two for f32),
// then their values.
template <int C>
struct Raw8 {
    uint4 a, b;
};
template <int C>
__device__ __forceinline__ Raw8<C> load8_raw(const void* p) {
    Raw8<C> r;
    r.a = ld_stream16(p);
    r.b = C == CKH_F32 ? ld_stream16(static_cast<const char*>(p) + 16) : make_uint4(0u, 0u, 0u, 0u);
    return r;
}
template <int C>
__device__ __forceinline__ void unpack8(const Raw8<C>& r, float (&v)[8]) {
    if constexpr (C == CKH_F32) {
        v[0] = as_f(r.a.x); v[1] = as_f(r.a.y); v[2] = as_f(r.a.z); v[3] = as_f(r.a.w);
        v[4] = as_f(r.b.x); v[5] = as_f(r.b.y); v[6] = as_f(r.b.z); v[7] = as_f(r.b.w);
    } else {
        const uint32_t d[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if constexpr (C == CKH_BF16) {
                v[2 * i] = bf16_to_f(d[i] & 0xffffu);
                v[2 * i + 1] = bf16_to_f(d[i] >> 16);
            } else {
                v[2 * i] = f16_to_f(d[i] & 0xffffu);
                v[2 * i + 1] = f16_to_f(d[i] >> 16);
            }
        }
    }
}

template <int C>
__device__ __forceinline__ void load8(const void* p, float (&v)[8]) {
    if constexpr (C == CKH_F32) {
        uint4 a = ld_stream16(p), b = ld_stream16(static_cast<const char*>(p) + 16);
        v[0] = as_f(a.x); v[1] = as_f(a.y); v[2] = as_f(a.z); v[3] = as_f(a.w);
        v[4] = as_f(b.x); v[5] = as_f(b.y); v[6] = as_f(b.z); v[7] = as_f(b.w);
    } else {
        uint4 w = ld_stream16(p);
        uint32_t d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if constexpr (C == CKH_BF16) {
                v[2 * i] = bf16_to_f(d[i] & 0xffffu);
                v[2 * i + 1] = bf16_to_f(d[i] >> 16);
            } else {
                v[2 * i] = f16_to_f(d[i] & 0xffffu);
                v[2 * i + 1] = f16_to_f(d[i] >> 16);
            }
        }
    }
}

// Load one element of dtype code C as float.
template <int C>
__device__ __forceinline__ float load1(const void* p, int64_t i) {
    if constexpr (C == CKH_F32) return reinterpret_cast<const float*>(p)[i];
    else if constexpr (C == CKH_BF16) return bf16_to_f(reinterpret_cast<const uint16_t*>(p)[i]);
    else return f16_to_f(reinterpret_cast<const uint16_t*>(p)[i]);
}

template <int C>
struct ElemSize { static constexpr int value = (C == CKH_F32) ? 4 : 2; };

// ------------------------------------------------------------ GEMM tile order
// Tile L of a tiles_m x tiles_n output-tile grid in grouped order: groups of
// kTileGroup tile rows (m), each group walked column by column.  The GEMMs hand each
// XCD a contiguous run of L per round (32 tiles on 32 CUs); in grouped order such a run
// is a compact ~6 x 5 block of tiles, which touches ~12 operand panels instead of the
// ~20 of a column-major run (18 m-tiles x 2 columns at the 4608-row configs), so fewer
// operand lines miss in that XCD's L2.
#ifndef CKH_TILE_GROUP
#define CKH_TILE_GROUP 6
#endif
constexpr int kTileGroup = CKH_TILE_GROUP;

__device__ __forceinline__ void grouped_tile(int L, int tiles_m, int tiles_n, int& tm, int& tn) {
    if (kTileGroup <= 0 || kTileGroup >= tiles_m) {
        tm = L % tiles_m;
        tn = L / tiles_m;
        return;
    }
    const int g = L / (kTileGroup * tiles_n);
    const int i = L - g * kTileGroup * tiles_n;
    const int gs = min(kTileGroup, tiles_m - g * kTileGroup);  // the last group may be shorter
    tm = g * kTileGroup + i % gs;
    tn = i / gs;
}


// ------------------------------------------------ dynamic per-tensor scale (amax.hip)
// Pass 1 of the layouts' default scale amax(|x|) / divisor: each workgroup of the launch
// writes the largest |x| of its share, as ordered fp32 bits (NaN above inf), to its word
// of `partial` (at most CKH_AMAX_WORKSPACE_BYTES / 4 words).  Returns the number of words.
int amax_partials(const void* x, int64_t numel, int in_code, uint32_t* partial, hipStream_t st);
// Pass 2 as its own launch: *scale_out = the scale from `nparts` partial words.
void amax_finalize(const uint32_t* partial, int nparts, int in_code, float divisor, float* scale_out,
                   hipStream_t st);

// The scale from the partial words: round_IN(amax * inv_divisor), inv_divisor = the fp32
// reciprocal torch multiplies by when it divides a GPU tensor by a Python scalar.
template <int IN>
__device__ __forceinline__ float scale_of_amax_bits(uint32_t amax_bits, float inv_divisor) {
    const float q = as_f(amax_bits) * inv_divisor;
    if constexpr (IN == CKH_BF16) return bf16_to_f(f_to_bf16(q));
    else if constexpr (IN == CKH_F16) return round_f16(q);
    else return q;
}

// Compute units of the current device (cached per device; 256 if the query fails).
inline int device_cus() {
    static int cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cus[dev]) {
        int c = 0;
        if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
        cus[dev] = c;
    }
    return cus[dev];
}

// Raw buffer descriptor over [p, p + bytes): loads at offsets past `bytes` return 0.  The
// inputs are wave-uniform by construction; reading them through readfirstlane keeps the
// descriptor in SGPRs (a descriptor the compiler believes divergent turns every load into
// a per-lane loop).  The address halves are taken as unsigned 32-bit values, so the low
// half is zero-extended when the 64-bit base is rebuilt.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* p, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a)));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a >> 32)));
    const uint32_t n = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(bytes));
    void* base = reinterpret_cast<void*>((static_cast<uint64_t>(hi) << 32) | static_cast<uint64_t>(lo));
    return __builtin_amdgcn_make_buffer_rsrc(base, 0, static_cast<int>(n), 0x00020000);
}

// Pass 2 fused into a kernel's prologue, in two steps.  load_partial_words issues the
// thread's share of the (at most CKH_AMAX_WORKSPACE_BYTES / 4) partial words as
// unconditional buffer loads (words past nparts read as 0): a caller that issues them
// before its own data loads can later wait for them without waiting for its data, since
// loads complete in order.  scale_from_partial_words then reduces them over the NT threads
// of the workgroup (every thread must call it; `red` is NT / 64 words of LDS) to the
// scale; its barrier waits for LDS traffic only.
template <int NT>
struct PartialWords {
    static constexpr int N = (CKH_AMAX_WORKSPACE_BYTES / 4 + NT - 1) / NT;
    uint32_t v[N];
};

template <int NT>
__device__ __forceinline__ PartialWords<NT> load_partial_words(const uint32_t* __restrict__ partial,
                                                               uint32_t nparts) {
    const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(partial, nparts * 4u);
    PartialWords<NT> w;
#pragma unroll
    for (int i = 0; i < PartialWords<NT>::N; ++i)
        w.v[i] = __builtin_amdgcn_raw_buffer_load_b32(rs, (threadIdx.x + i * NT) * 4u, 0, 0);
    return w;
}

template <int IN, int NT>
__device__ __forceinline__ float scale_from_partial_words(const PartialWords<NT>& w, float inv_divisor,
                                                          uint32_t* red) {
    uint32_t m = w.v[0];
#pragma unroll
    for (int i = 1; i < PartialWords<NT>::N; ++i) m = max(m, w.v[i]);
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) m = max(m, static_cast<uint32_t>(__shfl_xor(static_cast<int>(m), s, 64)));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0); vmcnt and expcnt unconstrained
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
    uint32_t b = red[0];
#pragma unroll
    for (int i = 1; i < NT / 64; ++i) b = max(b, red[i]);
    return scale_of_amax_bits<IN>(b, inv_divisor);
}

}  // namespace ckh
