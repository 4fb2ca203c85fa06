// Pieces shared by the skinny-activation GEMMs (gemm_mxfp8.hip, gemm_nvfp4.hip).
//
// A skinny GEMM (few activation rows) streams every weight byte once.  A workgroup owns a
// few 32-row weight tiles and all of K; its waves split K in chunks of kCb bytes per row,
// and each wave keeps D chunks in flight: the chunk's weight rows go to one of D LDS buffers
// by direct-to-LDS loads in which every instruction reads 8 whole 128-byte lines, its scale
// words (and activation codes) to registers.  The loads of chunk i + D are issued as soon as
// chunk i's LDS reads are done.
#pragma once

#include "ckh_common.h"

namespace ckh {
namespace sk {

typedef __attribute__((address_space(3))) void lds_void;
typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef unsigned v2u __attribute__((ext_vector_type(2)));

constexpr int kCb = 128;              // staged bytes per row and chunk
constexpr int kAuxNontemporal = 2;    // buffer-load cache policy bit: the weight is read once

// s_waitcnt immediate: vmcnt in [3:0] and [15:14], expcnt [6:4] (left at 7), lgkmcnt 0
constexpr int waitcnt_vm_lgkm0(int vm) { return (vm & 15) | (7 << 4) | ((vm >> 4) << 14); }

template <int WAITCNT>
__device__ __forceinline__ void wait() {
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(WAITCNT);
    __asm__ volatile("" ::: "memory");
}

// Staged rows are 128 bytes; logical 16-byte chunk c of row r sits at physical chunk
// c ^ (r % 8) ^ ((r / 8) % 2), so the 16 rows of a fragment read (one logical chunk each)
// hit 16 distinct 16-byte groups of the 256-byte bank cycle.
__device__ __forceinline__ uint32_t swz8(int r) { return static_cast<uint32_t>((r & 7) ^ ((r >> 3) & 1)); }

// Direct-to-LDS loads of rows [0, 8 NQ) of a chunk (bytes [b0, b0 + 128) of rows `pitch`
// bytes long): load q writes 1 KB (rows 8 q .. 8 q + 7), lane i to row 8 q + i / 8, physical
// chunk i % 8, i.e. 8 whole 128-byte lines per load.  Bytes past the row's end, and rows
// outside the descriptor, arrive as zeros.
template <int NQ, int AUX>
__device__ __forceinline__ void stage_rows(__amdgpu_buffer_rsrc_t rs, uint8_t* dst, int pitch, int b0, int lane) {
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        const int row = 8 * q + (lane >> 3);
        const int k = b0 + static_cast<int>(((lane & 7) ^ swz8(row)) << 4);
        const uint32_t off = k < pitch ? static_cast<uint32_t>(row * pitch + k) : 0x80000000u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(dst + q * 1024), 16, off, 0, 0, AUX);
    }
}

// Logical 16-byte chunk c of staged row r.
__device__ __forceinline__ v4u staged_chunk(const uint8_t* st, int r, int c) {
    return *reinterpret_cast<const v4u*>(st + r * kCb + ((static_cast<uint32_t>(c) ^ swz8(r)) << 4));
}

// n consecutive scale words (n = 1 or 2) from offset off of a swizzled scale tensor
template <int N>
__device__ __forceinline__ void load_words(__amdgpu_buffer_rsrc_t rs, uint32_t off, uint32_t (&w)[N]) {
    if constexpr (N == 2) {
        const v2u x = __builtin_bit_cast(v2u, __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, 0));
        w[0] = x[0];
        w[1] = x[1];
    } else {
        w[0] = __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0);
    }
}

// Scale word of row r (< 32) of the first of a workgroup's weight tiles starting at row n0 in
// word column 0 of a swizzled scale tensor with ncb word columns:
// ((row/128 * ncb + c) * 32 + row%32) * 16 + ((row%128)/32) * 4 plus c * 512 for column c.
// With two tiles (n0 a multiple of 64) the second tile's word follows.
__device__ __forceinline__ uint32_t weight_word_offset(int n0, int r, int ncb) {
    return static_cast<uint32_t>((n0 >> 7) * ncb * 512 + r * 16 + ((n0 & 127) >> 5) * 4);
}

// XCD-contiguous order of a skinny grid's row groups: workgroups are dispatched round-robin
// over the 8 XCDs (blockIdx % 8), so dealing the groups in 8 contiguous ranges puts the
// 32-row groups that share a 128-row block of swizzled scale lines on one XCD (its L2
// fetches those lines once).
__device__ __forceinline__ int xcd_group(int b, int n) { return (n & 7) == 0 ? (b & 7) * (n >> 3) + (b >> 3) : b; }

}  // namespace sk
}  // namespace ckh
