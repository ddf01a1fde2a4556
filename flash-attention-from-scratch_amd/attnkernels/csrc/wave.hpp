// Wave64 helpers for the gfx950 (CDNA4) attention kernels.
//
// Replaces the reference's warp32 helpers (attnkernels/csrc/common.cuh:15-59):
// cross-lane reductions use DPP row permutes inside 16-lane rows and
// ds_swizzle/bpermute across rows; exp2 is the hardware v_exp_f32; 16-byte
// vector types map onto global_load_dwordx4 / ds_read_b128.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ak {

using f16 = _Float16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// log2(e): softmax runs in base 2, exp(x) = 2^(x * log2 e), with the softmax
// scale folded into the same multiply (the reference's convention, README.md:80-82).
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kWave = 64;
constexpr int kNumXcd = 8;  // MI355X: 8 XCDs, workgroups dispatched round-robin

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ int lane_id() { return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }

// Wave-uniform copy of a value (forces it into an SGPR).
__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

// DPP lane permute inside each 16-lane row.
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i <- lane 7-i within each 8
constexpr int kDppMirror = 0x140;      // lane i <- lane 15-i within each 16

// Sum over aligned groups of N lanes (N = 8 or 16); every lane gets its group's sum.
template <int N>
__device__ __forceinline__ float group_sum(float x) {
    static_assert(N == 8 || N == 16, "group of 8 or 16 lanes");
    x += dpp<kDppXor1>(x);
    x += dpp<kDppXor2>(x);
    x += dpp<kDppHalfMirror>(x);
    if constexpr (N == 16) x += dpp<kDppMirror>(x);
    return x;
}

// Value held by lane (l ^ MASK) for MASK in {8, 16, 32}: ds_swizzle / bpermute.
template <int MASK>
__device__ __forceinline__ float shfl_xor(float x) {
    return __shfl_xor(x, MASK, kWave);
}

// 32x32x16 f16 MFMA with fp32 accumulators (CDNA4).
//   A (32 x 16): lane l holds row l%32, k = 8*(l/32) .. +7
//   B (16 x 32): lane l holds col l%32, k = 8*(l/32) .. +7
//   C (32 x 32): lane l holds col l%32, rows 8*(r/4) + 4*(l/32) + r%4, r = 0..15
__device__ __forceinline__ f32x16 mfma32x32x16(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// 16x16x32 f16 MFMA with fp32 accumulators (CDNA4).
//   A (16 x 32): lane l holds row l%16 and 8 k values selected by l/16
//   B (32 x 16): lane l holds col l%16 and the same 8 k values
//   C (16 x 16): lane l holds col l%16, rows 4*(l/16) + r, r = 0..3
// A and B select k by (lane / 16, element) in the same way, so any operand
// pair loaded with one (group, element) -> k map multiplies correctly.
__device__ __forceinline__ f32x4 mfma16x16x32(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Swap bits 2 and 3 of a lane/row index (an involution).  Used to line up the
// MFMA accumulator row order with 8-element contiguous runs.
__host__ __device__ constexpr int swap23(int x) { return (x & ~0xC) | ((x & 4) << 1) | ((x & 8) >> 1); }

// Remap a linear workgroup id so that consecutive logical tiles land on the
// same XCD (each XCD has its own L2): the hardware hands workgroup i to XCD
// i % 8, so XCD x receives the logical range [x*per + min(x, rem), ...).
__device__ __forceinline__ int xcd_remap(int bid, int total) {
    const int per = total / kNumXcd, rem = total % kNumXcd;
    const int x = bid % kNumXcd, slot = bid / kNumXcd;
    return x * per + (x < rem ? x : rem) + slot;
}

// Remap a linear workgroup id so that logical chunks of `chunk` consecutive
// tiles go to the XCDs round-robin (chunk j to XCD j % 8), each chunk whole on
// one XCD: its tiles share that XCD's L2, and every XCD receives a
// representative mix of chunks even when their costs differ.  A bijection on
// [0, total): ids past the last full group of 8 chunks map to themselves.
__device__ __forceinline__ int xcd_chunk_remap(int bid, int total, int chunk) {
    const int group = kNumXcd * chunk;
    if (bid >= total / group * group) return bid;
    const int x = bid % kNumXcd, slot = bid / kNumXcd;
    return slot / chunk * group + x * chunk + slot % chunk;
}

}  // namespace ak
