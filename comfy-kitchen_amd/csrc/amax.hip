// Dynamic per-tensor scale on the device: scale = amax(|x|) / divisor, computed in x's
// dtype and widened to fp32.  This is the default scale of the layouts' quantize
// (reference tensor/fp8.py:56-61: torch.amax(tensor.abs()) / finfo(e4m3).max, and
// tensor/nvfp4.py:64-69: ... / (448 * 6)): a 0-dim tensor of x's dtype, i.e. the fp32
// quotient of the (exact) amax and the divisor rounded once to x's dtype.
//
// Three launches on the caller's stream, no allocation and no host synchronisation, so
// the scale feeds the quantize kernels (which read it from device memory) directly:
//   1. clear the 4-byte result word (a kernel, so the sequence can be graph-captured);
//   2. the maximum of |x| as ordered integer bits (NaN orders above inf, so a NaN
//      propagates as in torch.amax) with one atomic max per workgroup into that word;
//   3. divide by `divisor`, round to x's dtype and store the fp32 value in place.
// Pass 2 reads x with ordinary (cached) loads: the quantize kernel that follows finds
// the tensor in the 256 MB infinity cache when it fits there.
#include "ckh_common.h"

namespace ckh {
namespace am {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;  // 16-byte loads in flight per thread per iteration

__global__ void clear_kernel(uint32_t* word) { *word = 0u; }

// |x| bits of 8 packed 16-bit values -> the largest, as fp32 bits
template <int IN>
__device__ __forceinline__ uint32_t max16(uint4 w) {
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    auto h = [](uint32_t v) { return __builtin_bit_cast(u16x2, v & 0x7fff7fffu); };
    u16x2 m = __builtin_elementwise_max(__builtin_elementwise_max(h(w.x), h(w.y)),
                                        __builtin_elementwise_max(h(w.z), h(w.w)));
    return max(static_cast<uint32_t>(m.x), static_cast<uint32_t>(m.y));
}

template <int IN>
__device__ __forceinline__ uint32_t to_f32_bits(uint32_t m16) {
    if constexpr (IN == CKH_BF16) return m16 << 16;
    else return as_u(static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(m16))));
}

template <int IN>
__device__ __forceinline__ uint32_t abs_bits1(const void* x, int64_t i) {
    if constexpr (IN == CKH_F32) return as_u(static_cast<const float*>(x)[i]) & 0x7fffffffu;
    else return to_f32_bits<IN>(static_cast<const uint16_t*>(x)[i] & 0x7fffu);
}

// VEC: x is 16-byte aligned; chunks of 16 bytes, then a scalar tail.
template <int IN, bool VEC>
__global__ __launch_bounds__(kThreads) void amax_kernel(const void* __restrict__ x, int64_t n, uint32_t* word) {
    constexpr int PER = 16 / ElemSize<IN>::value;  // elements per 16-byte chunk
    const int64_t tid = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
    uint32_t m = 0;
    int64_t tail_begin = 0;
    if constexpr (VEC) {
        const int64_t chunks = n / PER;
        const uint4* p = static_cast<const uint4*>(x);
        int64_t c = tid;
        for (; c + (kUnroll - 1) * stride < chunks; c += kUnroll * stride) {
            uint4 w[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) w[u] = p[c + u * stride];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                if constexpr (IN == CKH_F32)
                    m = max(m, max(max(w[u].x & 0x7fffffffu, w[u].y & 0x7fffffffu),
                                   max(w[u].z & 0x7fffffffu, w[u].w & 0x7fffffffu)));
                else
                    m = max(m, to_f32_bits<IN>(max16<IN>(w[u])));
            }
        }
        for (; c < chunks; c += stride) {
            const uint4 w = p[c];
            if constexpr (IN == CKH_F32)
                m = max(m, max(max(w.x & 0x7fffffffu, w.y & 0x7fffffffu), max(w.z & 0x7fffffffu, w.w & 0x7fffffffu)));
            else
                m = max(m, to_f32_bits<IN>(max16<IN>(w)));
        }
        tail_begin = chunks * PER;
    }
    for (int64_t i = tail_begin + tid; i < n; i += stride) m = max(m, abs_bits1<IN>(x, i));
    // wave maximum, then the workgroup's through LDS, then one atomic per workgroup (a
    // vector-memory atomic; same-address atomics serialise, so there are few of them)
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) m = max(m, static_cast<uint32_t>(__shfl_xor(static_cast<int>(m), s, 64)));
    __shared__ uint32_t wmax[kThreads / 64];
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t b = wmax[0];
#pragma unroll
        for (int w = 1; w < kThreads / 64; ++w) b = max(b, wmax[w]);
        atomicMax(word, b);
    }
}

// word holds the amax as fp32 bits; replace it with float(round_IN(amax / divisor))
template <int IN>
__global__ void finalize_kernel(uint32_t* word, float divisor) {
    const float q = as_f(*word) / divisor;
    float r;
    if constexpr (IN == CKH_BF16) r = bf16_to_f(f_to_bf16(q));
    else if constexpr (IN == CKH_F16) r = round_f16(q);
    else r = q;
    *reinterpret_cast<float*>(word) = r;
}

}  // namespace am
}  // namespace ckh

using namespace ckh;

extern "C" int ckh_amax_scale(const void* x, int64_t numel, int in_code, float divisor, void* scale_out,
                              uintptr_t stream) {
    CKH_REQUIRE(x && scale_out, "amax_scale: null pointer");
    CKH_REQUIRE(numel > 0, "amax_scale: empty tensor (torch.amax of an empty tensor is an error too)");
    CKH_REQUIRE(in_code == CKH_F32 || in_code == CKH_F16 || in_code == CKH_BF16,
                "amax_scale: unsupported input dtype code %d", in_code);
    CKH_REQUIRE(aligned(scale_out, 4), "amax_scale: output misaligned");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    uint32_t* word = static_cast<uint32_t*>(scale_out);
    const int es = in_code == CKH_F32 ? 4 : 2;
    const bool vec = aligned(x, 16);
    // four workgroups per CU at most (1024 atomics); each thread strides through x with
    // kUnroll 16-byte loads in flight
    const int64_t chunks = cdiv(numel * es, 16);
    const unsigned blocks =
        static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>(1024, cdiv(chunks, am::kThreads * am::kUnroll))));
    hipLaunchKernelGGL(am::clear_kernel, dim3(1), dim3(1), 0, st, word);
#define LAUNCH(I)                                                                                      \
    do {                                                                                               \
        if (vec) hipLaunchKernelGGL((am::amax_kernel<I, true>), dim3(blocks), dim3(am::kThreads), 0, st, x, numel, word); \
        else hipLaunchKernelGGL((am::amax_kernel<I, false>), dim3(blocks), dim3(am::kThreads), 0, st, x, numel, word); \
        hipLaunchKernelGGL((am::finalize_kernel<I>), dim3(1), dim3(1), 0, st, word, divisor);           \
    } while (0)
    if (in_code == CKH_F32) LAUNCH(CKH_F32);
    else if (in_code == CKH_F16) LAUNCH(CKH_F16);
    else LAUNCH(CKH_BF16);
#undef LAUNCH
    return check_launch("amax_scale");
}
