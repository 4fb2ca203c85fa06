// Dynamic per-tensor scale on the device: scale = amax(|x|) / divisor, computed in x's
// dtype and widened to fp32.  This is the default scale of the layouts' quantize
// (reference tensor/fp8.py:56-61: torch.amax(tensor.abs()) / finfo(e4m3).max, and
// tensor/nvfp4.py:64-69: ... / (448 * 6)): a 0-dim tensor of x's dtype.  torch evaluates
// that division on a GPU tensor by a Python-scalar divisor as a multiply by the fp32
// reciprocal: RN32(amax * RN32(1/divisor)), rounded once to x's dtype.  The kernel does the
// same (the reciprocal is formed on the host in fp32), so it matches the reference on the
// device bit for bit; a true division differs from it in the last fp32 bit for about half
// of all fp32 amaxes and for some tiny f16 ones.
//
// Two launches on the caller's stream, no allocation and no host synchronisation, so
// the scale feeds the quantize kernels (which read it from device memory) directly:
//   1. each workgroup writes the maximum of |x| over its share, as ordered integer bits
//      (NaN orders above inf, so a NaN propagates as in torch.amax), to its word of the
//      caller's workspace;
//   2. one workgroup reduces those words, divides by `divisor`, rounds to x's dtype and
//      stores the fp32 value.
// No atomics and no cleared words: every workspace word that pass 2 reads was written by
// pass 1 of the same call.  Pass 1 reads x with ordinary (cached) loads, kUnroll 16-byte
// loads in flight per thread: the quantize kernel that follows finds the tensor in the
// 256 MB infinity cache when it fits there.
#include <atomic>
#include <mutex>

#include "ckh_common.h"

namespace ckh {
namespace am {

constexpr int kThreads = 256;
constexpr int kUnroll = 16;                // 16-byte loads in flight per thread
constexpr int kMaxBlocks = CKH_AMAX_WORKSPACE_BYTES / 4;  // one partial word per workgroup

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

template <int IN>
__device__ __forceinline__ uint32_t chunk_max(uint4 w) {
    if constexpr (IN == CKH_F32)
        return max(max(w.x & 0x7fffffffu, w.y & 0x7fffffffu), max(w.z & 0x7fffffffu, w.w & 0x7fffffffu));
    else return to_f32_bits<IN>(max16<IN>(w));
}

// the workgroup's maximum of m (every thread must call it); valid in thread 0
__device__ __forceinline__ uint32_t block_max(uint32_t m) {
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) m = max(m, static_cast<uint32_t>(__shfl_xor(static_cast<int>(m), s, 64)));
    __shared__ uint32_t wmax[kThreads / 64];
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = m;
    __syncthreads();
    uint32_t b = wmax[0];
#pragma unroll
    for (int w = 1; w < kThreads / 64; ++w) b = max(b, wmax[w]);
    return b;
}

// VEC: x is 16-byte aligned; chunks of 16 bytes, then a scalar tail.  Thread t reads
// chunks t, t + stride, ... in batches of kUnroll, all of a batch's loads issued before
// any is used.
template <int IN, bool VEC>
__global__ __launch_bounds__(kThreads) void amax_kernel(const void* __restrict__ x, int64_t n,
                                                        uint32_t* __restrict__ partial) {
    constexpr int PER = 16 / ElemSize<IN>::value;  // elements per 16-byte chunk
    const int64_t tid = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
    uint32_t m = 0;
    int64_t tail_begin = 0;
    if constexpr (VEC) {
        const int64_t chunks = n / PER;
        const uint4* p = static_cast<const uint4*>(x);
        for (int64_t c0 = tid; c0 < chunks; c0 += kUnroll * stride) {
            uint4 w[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                const int64_t c = c0 + u * stride;
                w[u] = c < chunks ? p[c] : make_uint4(0u, 0u, 0u, 0u);
            }
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) m = max(m, chunk_max<IN>(w[u]));
        }
        tail_begin = chunks * PER;
    }
    for (int64_t i = tail_begin + tid; i < n; i += stride) m = max(m, abs_bits1<IN>(x, i));
    const uint32_t b = block_max(m);
    if (threadIdx.x == 0) partial[blockIdx.x] = b;
}

// *out = float(round_IN(amax * inv_divisor)), amax = the largest of the nblocks partial words
template <int IN>
__global__ __launch_bounds__(kThreads) void finalize_kernel(const uint32_t* __restrict__ partial, int nblocks,
                                                            float inv_divisor, float* __restrict__ out) {
    uint32_t m = 0;
    for (int i = threadIdx.x; i < nblocks; i += kThreads) m = max(m, partial[i]);
    const uint32_t b = block_max(m);
    if (threadIdx.x == 0) *out = scale_of_amax_bits<IN>(b, inv_divisor);
}

}  // namespace am

int amax_partials(const void* x, int64_t numel, int in_code, uint32_t* partial, hipStream_t st) {
    const int es = in_code == CKH_F32 ? 4 : 2;
    const bool vec = aligned(x, 16);
    // up to 8 workgroups per CU, each thread with kUnroll 16-byte loads in flight; never
    // more workgroups than the workspace has partial words
    const int64_t chunks = cdiv(numel * es, 16);
    const int blocks = static_cast<int>(
        std::max<int64_t>(1, std::min<int64_t>(am::kMaxBlocks, cdiv(chunks, am::kThreads * am::kUnroll))));
#define LAUNCH(I)                                                                                                \
    do {                                                                                                         \
        if (vec) hipLaunchKernelGGL((am::amax_kernel<I, true>), dim3(blocks), dim3(am::kThreads), 0, st, x, numel, partial); \
        else hipLaunchKernelGGL((am::amax_kernel<I, false>), dim3(blocks), dim3(am::kThreads), 0, st, x, numel, partial); \
    } while (0)
    if (in_code == CKH_F32) LAUNCH(CKH_F32);
    else if (in_code == CKH_F16) LAUNCH(CKH_F16);
    else LAUNCH(CKH_BF16);
#undef LAUNCH
    return blocks;
}

void amax_finalize(const uint32_t* partial, int nparts, int in_code, float divisor, float* scale_out,
                   hipStream_t st) {
    // torch's op-math reciprocal of the scalar divisor: fp32 division on the host
    const float inv_divisor = 1.0f / divisor;
#define LAUNCH(I) \
    hipLaunchKernelGGL((am::finalize_kernel<I>), dim3(1), dim3(am::kThreads), 0, st, partial, nparts, inv_divisor, scale_out)
    if (in_code == CKH_F32) LAUNCH(CKH_F32);
    else if (in_code == CKH_F16) LAUNCH(CKH_F16);
    else LAUNCH(CKH_BF16);
#undef LAUNCH
}

}  // namespace ckh

using namespace ckh;

namespace {

// Both entry points: pass 1 (per-workgroup maxima into `partial`) and pass 2 (the scale).
int launch_amax(const void* x, int64_t numel, int in_code, float divisor, void* scale_out, uint32_t* partial,
                hipStream_t st) {
    const int blocks = amax_partials(x, numel, in_code, partial, st);
    amax_finalize(partial, blocks, in_code, divisor, static_cast<float*>(scale_out), st);
    return CKH_OK;
}

int check_amax_args(const void* x, int64_t numel, int in_code, void* scale_out, const char* what) {
    CKH_REQUIRE(x && scale_out, "%s: null pointer", what);
    CKH_REQUIRE(numel > 0, "%s: empty tensor (torch.amax of an empty tensor is an error too)", what);
    CKH_REQUIRE(in_code == CKH_F32 || in_code == CKH_F16 || in_code == CKH_BF16,
                "%s: unsupported input dtype code %d", what, in_code);
    CKH_REQUIRE(aligned(scale_out, 4), "%s: scale_out misaligned", what);
    return CKH_OK;
}

}  // namespace

extern "C" int ckh_amax_scale(const void* x, int64_t numel, int in_code, float divisor, void* scale_out,
                              void* workspace, uintptr_t stream) {
    if (int rc = check_amax_args(x, numel, in_code, scale_out, "amax_scale")) return rc;
    CKH_REQUIRE(workspace, "amax_scale: null pointer (workspace)");
    CKH_REQUIRE(aligned(workspace, 4), "amax_scale: output or workspace misaligned");
    launch_amax(x, numel, in_code, divisor, scale_out, static_cast<uint32_t*>(workspace),
                reinterpret_cast<hipStream_t>(stream));
    return check_launch("amax_scale");
}

// ------------------------------------------------------------- no-allocation variant
// The partial maxima of ckh_amax_scale_noalloc live in this file-scope device array
// instead of a caller's workspace: CKH_AMAX_WORKSPACE_BYTES (8 KB) on each GPU the
// library runs on, held until the process ends.  In host code `scratch` names a host-side
// stand-in, not device memory: the kernels get the device address that
// hipGetSymbolAddress returns for the current device, resolved once per device on the
// first call there and cached.  Every call on a GPU shares that GPU's array, so calls
// that overlap on one GPU (different streams, or threads) race on it.  Pass 2 reads only
// the words pass 1 of the same call wrote, so nothing needs clearing between calls.
static __device__ __align__(256) uint32_t scratch[am::kMaxBlocks];

namespace {

constexpr int kMaxDevices = 64;
std::atomic<uint32_t*> g_scratch[kMaxDevices];  // device address of `scratch`, per device
std::mutex g_scratch_init;

// The device address of `scratch` on `dev`, which must be the current device.
int scratch_on(int dev, uint32_t** out) {
    uint32_t* p = g_scratch[dev].load(std::memory_order_acquire);
    if (p == nullptr) {
        std::lock_guard<std::mutex> lock(g_scratch_init);
        p = g_scratch[dev].load(std::memory_order_relaxed);
        if (p == nullptr) {
            void* addr = nullptr;
            const hipError_t e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
            if (e != hipSuccess || addr == nullptr) {
                set_error("amax_scale_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                          hipGetErrorString(e));
                return CKH_ERR_LAUNCH;
            }
            p = static_cast<uint32_t*>(addr);
            g_scratch[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return CKH_OK;
}

}  // namespace

extern "C" int ckh_amax_scale_noalloc(const void* x, int64_t numel, int in_code, float divisor, void* scale_out,
                                      uintptr_t stream) {
    if (int rc = check_amax_args(x, numel, in_code, scale_out, "amax_scale_noalloc")) return rc;
    // The launch never uses more workgroups, i.e. partial words, than the scratch array
    // holds (launch_amax caps the grid at kMaxBlocks), so no input size needs more of it.
    static_assert(sizeof(scratch) == CKH_AMAX_WORKSPACE_BYTES, "scratch holds one word per workgroup");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    int dev = -1, cur = -1;
    hipError_t e = hipStreamGetDevice(st, &dev);
    if (e == hipSuccess) e = hipGetDevice(&cur);
    if (e != hipSuccess) {
        set_error("amax_scale_noalloc: device query failed: %s", hipGetErrorString(e));
        return CKH_ERR_LAUNCH;
    }
    CKH_REQUIRE(dev == cur, "amax_scale_noalloc: the stream belongs to device %d but device %d is current", dev, cur);
    CKH_REQUIRE(dev >= 0 && dev < kMaxDevices, "amax_scale_noalloc: device %d beyond the %d supported", dev,
                kMaxDevices);
    uint32_t* partial = nullptr;
    if (int rc = scratch_on(dev, &partial)) return rc;
    launch_amax(x, numel, in_code, divisor, scale_out, partial, st);
    return check_launch("amax_scale_noalloc");
}
