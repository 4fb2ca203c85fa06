// Weight staging shared by the skinny-activation GEMMs (gemm_mxfp8.hip, gemm_nvfp4.hip).
//
// A skinny GEMM (few activation rows) streams every weight byte once; each wave copies a
// chunk of kSkRow bytes of each of its weight rows into its own LDS area with direct-to-LDS
// loads in which every instruction reads 8 whole 128-byte lines, then reads its MFMA
// fragments from there.
#pragma once

#include "ckh_common.h"

namespace ckh {
namespace sk {

typedef __attribute__((address_space(3))) void lds_void;

constexpr int kSkRow = 256;              // staged bytes per row and chunk
constexpr int kSkCpr = kSkRow / 16;      // 16-byte chunks per staged row
constexpr int kSkRpl = 1024 / kSkRow;    // staged rows per direct-to-LDS load (1 KB)
constexpr int kAuxNontemporal = 2;       // buffer-load cache policy bit: the weight is read once

// Staging layout: row r of a chunk is 256 bytes; logical 16-byte chunk c sits at physical
// chunk c ^ (r % 16).  LDS banks repeat every 256 bytes, so a fragment read (16 lanes = 16
// consecutive rows, one logical chunk) hits 16 distinct 16-byte bank groups.
__device__ __forceinline__ uint32_t sk_swz(int r) { return static_cast<uint32_t>(r & (kSkCpr - 1)); }

// Direct-to-LDS whole-line loads of rows [0, NQ * kSkRpl) of a chunk of rows `pitch` bytes
// long, starting at byte kbase of each row: load q writes 1 KB, rows kSkRpl q .. , lane i to
// row kSkRpl q + i / kSkCpr, physical chunk i % kSkCpr, so each load reads 8 whole 128-byte
// lines.  Bytes past the row's end, and rows outside the descriptor, arrive as zeros.
template <int NQ, int AUX>
__device__ __forceinline__ void stage_rows(__amdgpu_buffer_rsrc_t rs, uint8_t* dst, int pitch, int kbase, int lane) {
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        const int row = kSkRpl * q + lane / kSkCpr;
        const int k = kbase + static_cast<int>(((lane % kSkCpr) ^ sk_swz(row)) << 4);
        const uint32_t off = k < pitch ? static_cast<uint32_t>(row * pitch + k) : 0x80000000u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(dst + q * 1024), 16, off, 0, 0, AUX);
    }
}

// Logical 16-byte chunk c of staged row r.
typedef unsigned v4u __attribute__((ext_vector_type(4)));
__device__ __forceinline__ v4u staged_chunk(const uint8_t* st, int r, int c) {
    return *reinterpret_cast<const v4u*>(st + r * kSkRow + ((static_cast<uint32_t>(c) ^ sk_swz(r)) << 4));
}

// XCD-contiguous order of a skinny grid's row groups: workgroups are dispatched round-robin
// over the 8 XCDs (blockIdx % 8), so dealing the groups in 8 contiguous ranges puts the
// 32-row groups that share a 128-row block of swizzled scale lines on one XCD (its L2
// fetches those lines once).
__device__ __forceinline__ int xcd_group(int b, int n) { return (n & 7) == 0 ? (b & 7) * (n >> 3) + (b >> 3) : b; }

}  // namespace sk
}  // namespace ckh
