/*
 * ckh.h -- C ABI of the MI355X (gfx950) kernels behind comfy_kitchen's "hip" backend.
 *
 * Conventions (all entry points):
 *   - Plain device pointers, int64 sizes, int dtype codes, and the HIP stream as an
 *     integer handle (hipStream_t cast to uintptr_t; 0 = the null stream).
 *   - Nothing allocates, nothing synchronises, no device scalar is read on the host:
 *     scales (`scale`, `global_scale`, `alpha`) stay in device memory and are read by
 *     the kernels.  Launches are asynchronous on `stream` and safe to capture in a
 *     hipGraph.
 *   - Return value: CKH_OK, or an error code with a message retrievable through
 *     ckh_last_error() (thread-local; valid until the next failing call on the thread).
 *   - Outputs are written in full, including the zero padding of swizzled scale
 *     tensors, so callers may allocate them uninitialised.
 *
 * Dtype codes are the reference's (backends/cuda/dlpack_bindings.cpp:27-41,
 * backends/eager/quantization.py:31-39): 0=f32 1=f16 2=bf16 3=u8 4=i8 5=e4m3fn 6=e5m2.
 *
 * Byte layouts: E4M3 / E5M2 codes are OCP FP8 bytes; NVFP4 codes are E2M1 nibbles,
 * two per byte, the even element in the high nibble when hi_first != 0; block scales
 * (E8M0 for MXFP8, E4M3 for NVFP4) use the 32_4_4 swizzle: logical scale (r, c) of a
 * [R, C] matrix padded to [ceil(R/128)*128, ceil(C/4)*4] lives at byte offset
 *   ((r/128 * ceil(C/4) + c/4) * 32 + r%32) * 16 + ((r%128)/32) * 4 + c%4.
 */
#ifndef CKH_H
#define CKH_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CKH_ABI_VERSION 8

enum ckh_dtype {
    CKH_F32 = 0,
    CKH_F16 = 1,
    CKH_BF16 = 2,
    CKH_U8 = 3,
    CKH_I8 = 4,
    CKH_E4M3 = 5,
    CKH_E5M2 = 6,
};

enum ckh_status {
    CKH_OK = 0,
    CKH_ERR_INVALID = 1, /* bad argument: shape, dtype, alignment, null pointer */
    CKH_ERR_LAUNCH = 2,  /* the HIP runtime rejected the launch */
};

/* Version of this ABI (CKH_ABI_VERSION of the built library). */
int ckh_abi_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char* ckh_last_error(void);

/*
 * Per-tensor FP8 quantize: out = fp8(clamp(x * r, +-max)), r = (1/scale) rounded to
 * x's dtype, the product rounded to x's dtype, then round-to-nearest-even to FP8.
 * x: numel elements of in_code (f32/f16/bf16); scale: one f32 on device;
 * out: numel bytes of out_code (e4m3 / e5m2).  A NaN product gives the byte eager's
 * vectorised CPU loop writes: 0xFF for bf16 x; 0x7F | sign for f16 / f32 x (the sign of
 * r's NaN, else of x's NaN, else negative for 0 * inf).
 * Replaces launch_quantize_fp8_kernel (reference backends/cuda/dlpack_bindings.cpp:45-48,
 * ops/per_tensor_quantize.cu:170-209), with the same argument order; arithmetic follows
 * backends/eager/quantization.py:41-55.
 */
int ckh_quantize_fp8(const void* x, void* out, const void* scale, int64_t numel,
                     int in_code, int out_code, uintptr_t stream);

/*
 * Per-tensor FP8 dequantize: out = x.to(out) * scale.to(out), rounded to out_code.
 * scale: one element of scale_code (f32 / f16 / bf16) on device, as eager accepts it.
 * Replaces launch_dequantize_fp8_kernel (dlpack_bindings.cpp:50-53,
 * ops/per_tensor_quantize.cu:211-249): the same arguments in the same order, plus
 * scale_code before the stream (that launcher reads an f32 scale only); arithmetic
 * follows eager quantization.py:57-61.
 */
int ckh_dequantize_fp8(const void* x, void* out, const void* scale, int64_t numel,
                       int in_code, int out_code, int scale_code, uintptr_t stream);

/*
 * MXFP8 quantize of x [orig_rows, orig_cols] (row-major, in_code f32/f16/bf16) into
 * codes [rows, cols] e4m3 (rows/cols >= orig, zero padded) and E8M0 block-32 scales in
 * the swizzled layout [roundup(rows,128), roundup(cols/32,4)].  cols % 32 == 0.
 * Replaces launch_quantize_mxfp8_kernel (dlpack_bindings.cpp:130-139,
 * ops/quantize_mxfp8.cu:148-208); arithmetic follows eager quantization.py:257-324.
 */
int ckh_quantize_mxfp8(const void* x, void* qx, void* scales, int64_t rows, int64_t cols,
                       int64_t orig_rows, int64_t orig_cols, int in_code, uintptr_t stream);

/*
 * MXFP8 dequantize: out[r,k] = (float(q[r,k]) * 2^(s[r,k/32]-127), s==0 -> 0).to(out).
 * qx [rows, cols] e4m3, scales swizzled, out [rows, cols] of out_code.
 * No native counterpart in the reference; arithmetic follows eager quantization.py:327-364.
 */
int ckh_dequantize_mxfp8(const void* qx, const void* scales, void* out, int64_t rows,
                         int64_t cols, int out_code, uintptr_t stream);

/*
 * NVFP4 quantize of x [orig_rows, orig_cols] with device f32 global scale g into packed
 * E2M1 codes [rows, cols/2] u8 and E4M3 block-16 scales, swizzled
 * [roundup(rows,128), roundup(cols/16,4)].  cols % 16 == 0 (rows need not be a
 * multiple of anything; the layouts pad them to 16 as the reference's pad_16x does).
 * epsilon is accepted and ignored, as in the reference.
 * Replaces launch_quantize_nvfp4_kernel (dlpack_bindings.cpp:104-116,
 * ops/quantize_nvfp4.cu:323-384); arithmetic follows eager quantization.py:115-160.
 */
int ckh_quantize_nvfp4(const void* x, const void* global_scale, void* qx, void* scales,
                       int64_t rows, int64_t cols, int64_t orig_rows, int64_t orig_cols,
                       float epsilon, int in_code, int hi_first, uintptr_t stream);

/*
 * NVFP4 dequantize: out = E2M1(q) * (g.to(out) * s8.to(out)) in out_code arithmetic.
 * qx [rows, cols/2] u8, scales swizzled, out [rows, cols].
 * Replaces launch_dequantize_nvfp4_kernel (dlpack_bindings.cpp:118-127,
 * ops/quantize_nvfp4.cu:386-434); arithmetic follows eager quantization.py:171-219.
 */
int ckh_dequantize_nvfp4(const void* qx, const void* global_scale, const void* scales,
                         void* out, int64_t rows, int64_t cols, int out_code, int hi_first,
                         uintptr_t stream);

/*
 * RoPE on x [batch, dim1, dim2, head_dim] (element strides sx_*; innermost stride 1)
 * with freqs [fb, fd1, fd2, head_dim/2, 2, 2] (element strides sf_* for the first
 * three dims; the inner [head_dim/2, 2, 2] must be contiguous).  A freqs dim of size 1
 * broadcasts; otherwise it must equal x's (dim 2 may be longer and is then truncated).
 * out_i = f[i,0]*x0 + f[i,1]*x1 per pair, computed in the freqs dtype, rounded to x's.
 * x: in_code f32 / f16 / bf16; freqs: freqs_code f32 / f16 / bf16.
 * xk / xk_out may be NULL (apply_rope1).  Outputs are contiguous [batch,dim1,dim2,hd].
 * Replaces launch_apply_rope_kernel (dlpack_bindings.cpp:76-102,
 * ops/apply_rope.cu:317-362); arithmetic follows eager rope.py:7-18.
 */
int ckh_apply_rope(const void* xq, const void* xk, const void* freqs, void* xq_out,
                   void* xk_out, int64_t batch, int64_t dim1, int64_t dim2,
                   int64_t head_dim, int64_t freqs_batch, int64_t freqs_dim1,
                   int64_t freqs_dim2, int64_t sx_batch, int64_t sx_dim1, int64_t sx_dim2,
                   int64_t sf_batch, int64_t sf_dim1, int64_t sf_dim2, int in_code,
                   int freqs_code, uintptr_t stream);

/*
 * Bytes of device workspace ckh_scaled_mm_mxfp8 / ckh_scaled_mm_fp8 use at this shape to
 * split K (0: the shape does not split).  A small grid of 256 x 256 output tiles with long
 * K (e.g. M = 256, N = 13824, K = 5120) splits K over up to 256 workgroups, which write fp32
 * partial tiles to the workspace: grids of at most 64 tiles as 256 x 128 half tiles
 * (128 KB partials) from 32 stages of 64 along K, grids of 65-128 tiles as whole tiles
 * (256 KB) from 64 stages when three ranges or more fit.  A second launch adds the
 * partials in a fixed order and applies scale, bias and output rounding.  No counterpart
 * in the reference (torch's scaled_mm takes no workspace).
 */
int64_t ckh_scaled_mm_workspace_bytes(int64_t M, int64_t N, int64_t K);

/*
 * MXFP8 GEMM: out[M,N] = sum_k A[m,k]*2^(sa-127) * B[n,k]*2^(sb-127) (+ bias[n]).
 * a [M,K] e4m3, b [N,K] e4m3 (both K-major), sa/sb E8M0 swizzled with logical shapes
 * [M, K/32] / [N, K/32]; bias NULL or [N] of bias_code (f32/f16/bf16);
 * out [M,N] row-major of out_code (f32/f16/bf16).  K % 32 == 0.
 * workspace: NULL, or ckh_scaled_mm_workspace_bytes(M, N, K) bytes of device memory
 * (16-byte aligned) that the call may overwrite; with less than that the call does not
 * split K (same result within fp32 summation order, slower on small grids).  Calls running
 * at the same time need workspaces of their own.
 * No native counterpart in the reference (eager quantization.py:367-402 routes to
 * torch F.scaled_mm via scaled_mm_v2.py:27-53); replaces that call.
 */
int ckh_scaled_mm_mxfp8(const void* a, const void* b, const void* sa, const void* sb,
                        const void* bias, void* out, int64_t M, int64_t N, int64_t K,
                        int out_code, int bias_code, void* workspace, int64_t workspace_bytes,
                        uintptr_t stream);

/*
 * Per-tensor FP8 GEMM: out[M,N] = scale_a * scale_b * sum_k A[m,k] * B[n,k] (+ bias[n]).
 * a [M,K] e4m3, b [N,K] e4m3 (both K-major), scale_a / scale_b one f32 each on device;
 * bias NULL or [N] of bias_code; out [M,N] row-major of out_code.  K % 16 == 0.
 * workspace: as for ckh_scaled_mm_mxfp8.
 * Replaces the TensorWise torch F.scaled_mm call behind TensorCoreFP8Layout's
 * linear / mm / addmm (tensor/fp8.py:86-101 -> scaled_mm_v2.py:27-53).
 */
int ckh_scaled_mm_fp8(const void* a, const void* b, const float* scale_a, const float* scale_b,
                      const void* bias, void* out, int64_t M, int64_t N, int64_t K,
                      int out_code, int bias_code, void* workspace, int64_t workspace_bytes,
                      uintptr_t stream);

/*
 * NVFP4 GEMM: out[M,N] = alpha * sum_k E2M1(a)*sa[m,k/16] * E2M1(b)*sb[n,k/16] (+bias[n]).
 * a [M,K/2] u8, b [N,K/2] u8 (hi_first packing), sa/sb E4M3 swizzled with logical
 * shapes [M, K/16] / [N, K/16]; alpha one f32 on device; bias NULL or [N].
 * K % 32 == 0.
 * Replaces launch_cublas_gemm_blockwise_fp4_kernel (dlpack_bindings.cpp:59-74,
 * ops/cublas_gemm_nvfp4.cu:297-342); semantics follow eager quantization.py:222-246.
 * workspace: NULL, or ckh_scaled_mm_nvfp4_workspace_bytes(M, N, K) bytes of device memory
 * (16-byte aligned) in which small tile grids split K (as ckh_scaled_mm_mxfp8); with less
 * the call does not split.  Calls running at the same time need workspaces of their own.
 * Argument differences from that launcher: the activation comes first (the launcher takes
 * B before A because cuBLASLt is column-major; the product is the same A B^T); the
 * workspace is sized by ckh_scaled_mm_nvfp4_workspace_bytes rather than by the caller's
 * choice, and there is no `accumulate` flag (its only caller,
 * backends/cuda/__init__.py:353, always passes false, i.e. out is overwritten); bias_code
 * names the bias dtype, which that launcher takes from the DLPack tensor.
 */
int ckh_scaled_mm_nvfp4(const void* a, const void* b, const void* sa, const void* sb,
                        const void* alpha, const void* bias, void* out, int64_t M,
                        int64_t N, int64_t K, int out_code, int bias_code, void* workspace,
                        int64_t workspace_bytes, uintptr_t stream);

/*
 * Bytes of device workspace ckh_scaled_mm_nvfp4 uses at this shape to split K (0: no
 * split): grids of at most 64 output tiles of 256 x 256 with K of at least 2048 (split as
 * 256 x 128 half tiles), and grids of 65-128 tiles with K of at least 4096 when three K
 * ranges or more fit.  No
 * counterpart in the reference (its launcher takes a cuBLASLt workspace of the caller's
 * size).
 */
int64_t ckh_scaled_mm_nvfp4_workspace_bytes(int64_t M, int64_t N, int64_t K);

/*
 * Dynamic per-tensor scale: *scale_out = float(round_x(amax(|x|) * RN32(1/divisor))),
 * the amax and the product rounded to x's dtype (in_code), as the layouts' default scale
 * torch.amax(tensor.abs()) / max computes it on a GPU tensor (torch multiplies by the
 * fp32 reciprocal of a scalar divisor there).  x: numel contiguous elements; scale_out:
 * one f32 on device; workspace: CKH_AMAX_WORKSPACE_BYTES of device memory (4-byte
 * aligned, contents ignored and overwritten) that holds the per-workgroup partial maxima,
 * so the call allocates nothing.  Calls running at the same time need workspaces of their
 * own.  A NaN in x gives a NaN scale.  Replaces that torch expression in
 * TensorCoreFP8Layout.quantize (tensor/fp8.py:56-61, divisor 448) and
 * TensorCoreNVFP4Layout.quantize (tensor/nvfp4.py:64-69, divisor 2688); the result feeds
 * ckh_quantize_fp8 / ckh_quantize_nvfp4 on the same stream without a host round trip.
 */
#define CKH_AMAX_WORKSPACE_BYTES 8192
int ckh_amax_scale(const void* x, int64_t numel, int in_code, float divisor, void* scale_out,
                   void* workspace, uintptr_t stream);

/*
 * ckh_amax_scale without the workspace argument: the same kernels and result, with the
 * per-workgroup partial maxima in an 8 KB (CKH_AMAX_WORKSPACE_BYTES) device array that
 * the library holds on each GPU until the process ends.  The call allocates nothing
 * (no hipMalloc, no torch allocator): for callers that cannot allocate, such as code
 * under hipGraph capture with no allocator of its own or serving loops that forbid
 * allocation.  Every input size fits (the grid never has more workgroups than the array
 * has words).  `stream` must belong to the current device.  The first call on a device
 * resolves the array's address there (hipGetSymbolAddress) and must run outside stream
 * capture; later calls may be captured into a hipGraph.  All calls on one GPU share
 * its array: calls that overlap on that GPU (other streams, other threads) race and must
 * be serialised by the caller.  No counterpart in the reference.
 */
int ckh_amax_scale_noalloc(const void* x, int64_t numel, int in_code, float divisor,
                           void* scale_out, uintptr_t stream);

/*
 * NVFP4 quantize with the layouts' dynamic global scale: ckh_amax_scale (divisor 2688 for
 * TensorCoreNVFP4Layout) followed by ckh_quantize_nvfp4 with that scale, in two launches
 * instead of three.  Launch 1 writes the per-workgroup partial maxima of |x| to
 * `workspace` (CKH_AMAX_WORKSPACE_BYTES, 4-byte aligned; its loads are cached, so the
 * quantize that follows finds x in the 256 MB infinity cache when it fits there); launch 2
 * quantizes, every workgroup forming the scale from those words itself, and stores the
 * scale to *scale_out (one f32 on device).  Codes, block scales and *scale_out equal those
 * of the two separate calls bit for bit.  Shapes and arguments as ckh_quantize_nvfp4,
 * plus x non-empty; shapes outside the 16-bit fast path (padding, f32 input, cols % 64,
 * alignment) run the separate scale launch and the general quantize.  Calls running at
 * the same time need workspaces of their own.  Replaces the scale=None branch of
 * TensorCoreNVFP4Layout.quantize (tensor/nvfp4.py:64-69: torch.amax(x.abs()) / 2688, then
 * ck.quantize_nvfp4), the dynamic input quantization of samples/nvfp4_linear.py:55-59.
 */
int ckh_quantize_nvfp4_dynamic(const void* x, float divisor, void* scale_out, void* qx, void* scales,
                               int64_t rows, int64_t cols, int64_t orig_rows, int64_t orig_cols,
                               float epsilon, int in_code, int hi_first, void* workspace,
                               uintptr_t stream);

#ifdef __cplusplus
}
#endif

#endif /* CKH_H */
