// MFMA-busy calibration for bench.py's counter pass (not part of libckh.so): every wave
// issues `iters` rounds of 16 independent v_mfma_scale_f32_32x32x64_f8f6f4 on operands
// that differ per lane, with nothing else in the loop, so the SIMDs' matrix cores are
// busy for the whole dispatch.  The ratio SQ_VALU_MFMA_BUSY_CYCLES / SQ_BUSY_CYCLES this
// kernel reads is what 100% MFMA busy reads as; the GEMMs' ratios are divided by it.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

__global__ __launch_bounds__(256) void mfma_loop_kernel(int iters, float* __restrict__ out) {
    v8i a, b;
    for (int i = 0; i < 8; ++i) {
        a[i] = static_cast<int>((threadIdx.x * 0x9E3779B1u) ^ (i * 0x85EBCA77u) ^ (blockIdx.x * 0xC2B2AE3Du));
        b[i] = static_cast<int>((threadIdx.x * 0x27D4EB2Fu) ^ (i * 0x165667B1u) ^ (blockIdx.x * 0x61C88647u));
    }
    v16f acc[16];
    for (int i = 0; i < 16; ++i) acc[i] = v16f{};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int i = 0; i < 16; ++i)
            acc[i] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, acc[i], 0, 0, 0, 120, 0, 120);
    }
    float s = 0.0f;
    for (int i = 0; i < 16; ++i)
        for (int j = 0; j < 16; ++j) s += acc[i][j];
    out[blockIdx.x * 256 + threadIdx.x] = s;
}

}  // namespace

// out: workgroups * 256 floats of device memory.  One workgroup of 4 waves per CU (the
// GEMMs' occupancy) when workgroups equals the CU count.
extern "C" int ckh_bench_mfma_loop(float* out, int workgroups, int iters, uint64_t stream) {
    if (!out || workgroups <= 0 || iters <= 0) return 1;
    hipLaunchKernelGGL(mfma_loop_kernel, dim3(workgroups), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                       iters, out);
    return hipGetLastError() == hipSuccess ? 0 : 2;
}
