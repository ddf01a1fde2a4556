// Internal launch interface between the C-ABI layer (capi.cpp) and the HIP
// kernels (prefill.hip, decode.hip).  Arguments are validated by the caller.
#pragma once

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

namespace ak {

struct PrefillArgs {
    const void* q;
    const void* k;
    const void* v;
    void* o;
    int64_t bh;      // batch * query heads
    int64_t n;       // sequence length (packed layout: the longest sequence)
    int64_t hq;      // query heads
    int64_t hkv;     // kv heads, dividing hq
    const int32_t* cu;  // packed layout: [batch + 1] sequence starts; nullptr: dense [B, H, N, D]
    int64_t total_rows; // packed layout: rows of q/k/v; every sequence is clamped into [0, total_rows)
    int d;           // head dim, 64 or 128
    bool causal;
    float sl2;       // |scale| * log2(e)
    uint32_t qflip;  // 0x80008000 when scale < 0 (sign folded into Q), else 0
    void* stream;
};

// Launches of the grouped-query decode kernel with at least this many waves
// (at 4 per workgroup) keep 4-wave workgroups; smaller grids use 8 waves per
// workgroup.
constexpr int64_t kGqaManyWaves = 2048;

struct DecodeArgs {
    const void* q;         // [B, hq, D] fp16
    const void* k_cache;   // [num_blocks, hkv, bs, D] fp16
    const void* v_cache;
    const int32_t* block_tables;  // [B, max_blocks]
    const int32_t* context_lens;  // [B]
    void* out;             // [B, hq, D] fp16
    float* o_part;         // [B, hq, S, D]  (S > 1 only)
    float* m_part;         // [B, hq, S]
    float* l_part;         // [B, hq, S]
    // One int per (sequence, kv head), zero on entry and left zero: when set
    // (and 1 < S <= kFusedMaxSplits), the last split of each (sequence, kv
    // head) to finish merges the partials in the decode kernel, with no reduce
    // launch.  Null: the reduce kernel merges them.
    int32_t* counters;
    int64_t batch, hq, hkv, d, num_blocks, bs, max_blocks;
    int64_t partition, num_splits;
    float sl2;             // scale * log2(e)
    void* stream;
};

struct CacheWriteArgs {
    const void* key;        // [num_tokens, hkv, head_dim], token stride key_stride elements
    const void* value;      // [num_tokens, hkv, head_dim], token stride value_stride elements
    void* k_cache;          // [num_blocks, hkv, bs, head_dim]
    void* v_cache;
    const int64_t* slots;   // [num_tokens]
    int64_t num_tokens, hkv, head_dim, num_blocks, bs;
    int64_t key_stride, value_stride;  // multiples of 8
    void* stream;
};

hipError_t prefill_launch(const PrefillArgs& a);
hipError_t decode_launch(const DecodeArgs& a);

// Size of the static per-GPU split-partials array behind
// ak_paged_decode_noalloc, and its device address on the current GPU
// (looked up once per device).
constexpr size_t kDecodeScratchBytes = size_t(32) << 20;
// Most splits merged in the decode kernel itself; more go to the reduce
// kernel, whose workgroups per row read them in parallel (measured at B = 1-4,
// Hq = 32, Hkv = 8: 8-16 splits merged in the kernel save 1.5 us a call, 32
// break even, 64 lose 3 us).
constexpr int64_t kFusedMaxSplits = 32;
// Split counters of the static per-GPU array: one per (sequence, kv head).
constexpr size_t kDecodeScratchCounters = size_t(1) << 18;
hipError_t decode_scratch(void** ptr, int32_t** counters);
hipError_t cache_write_launch(const CacheWriteArgs& a);
// XOR of the 16-byte words of src (bytes / 16 of them) into out[0..3].
hipError_t stream_checksum_launch(const void* src, size_t bytes, uint32_t* out, void* stream);

}  // namespace ak
