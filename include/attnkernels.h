/* attnkernels C-ABI: MI355X (gfx950) attention hot path.
 *
 * Plain pointers, sizes and a hipStream_t passed as void*; no torch types.
 * These are the entry points behind the reference's pybind module
 * `attnkernels_ext` (sonhoang/flash-attention-from-scratch
 * attnkernels/csrc/ext.cpp:3-10, 14-17); each function names the reference
 * interface it replaces.
 *
 * Conventions shared by every entry point
 *   - Tensors are dense, row-major, fp16 (IEEE binary16) unless stated, in
 *     device memory, and every pointer is 16-byte aligned.
 *   - Work is enqueued on `stream` (NULL = the null stream) and the call
 *     returns without synchronising, like the reference's launches.
 *   - The return value is AK_OK or one of the AK_ERR_* codes; on failure
 *     ak_last_error() returns a message for the calling thread, worded like
 *     the reference's TORCH_CHECK messages where one exists.
 *   - Validation happens before any HIP call, so a rejected call touches no GPU.
 */
#ifndef ATTNKERNELS_H
#define ATTNKERNELS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    AK_OK = 0,
    AK_ERR_INVALID_ARGUMENT = 1, /* null/misaligned pointer, negative size, bad split size */
    AK_ERR_UNSUPPORTED = 2,      /* head_dim / block_n / head-group combination not built */
    AK_ERR_WORKSPACE = 3,        /* workspace missing or smaller than required */
    AK_ERR_HIP = 4               /* the HIP runtime reported an error at launch */
};

/* Message describing the last failed call on this thread ("" if none). */
const char *ak_last_error(void);

/* ABI version of this library (major * 100 + minor). */
int ak_abi_version(void);

/* Prefill attention, O = softmax(scale * Q K^T [+ causal mask]) V.
 * q, k, v, o: fp16 [batch, heads, seq_len, head_dim]; head_dim 64 or 128.
 * Key j is masked for query i iff causal && j > i.
 *
 * ak_naive_attention replaces naive_attention (attnkernels/csrc/naive_attn.cu:65-86,
 *   ext.cpp:14); it runs the same flash kernel (no N x N score buffer).
 * ak_flash_simt replaces flash_simt (attnkernels/csrc/flash_simt.cu:209-221, ext.cpp:15).
 * ak_flash_wmma replaces flash_wmma (attnkernels/csrc/flash_wmma.cu:241-257, ext.cpp:16);
 *   block_n must be 32 or 64, as in the reference, and selects nothing else: the
 *   gfx950 kernel picks its own key tile. */
int ak_naive_attention(const void *q, const void *k, const void *v, void *o, int64_t batch,
                       int64_t heads, int64_t seq_len, int64_t head_dim, int causal,
                       double scale, void *stream);
int ak_flash_simt(const void *q, const void *k, const void *v, void *o, int64_t batch,
                  int64_t heads, int64_t seq_len, int64_t head_dim, int causal, double scale,
                  void *stream);
int ak_flash_wmma(const void *q, const void *k, const void *v, void *o, int64_t batch,
                  int64_t heads, int64_t seq_len, int64_t head_dim, int causal, double scale,
                  int64_t block_n, void *stream);

/* Prefill with grouped-query attention (GQA/MQA): q, o fp16 [batch, num_heads,
 * seq_len, head_dim]; k, v fp16 [batch, num_kv_heads, seq_len, head_dim]; query
 * head h reads kv head h / (num_heads / num_kv_heads).  The same kernel as
 * ak_flash_wmma; the reference requires num_kv_heads == num_heads
 * (attnkernels/__init__.py:57-58), where the two agree. */
int ak_prefill_gqa(const void *q, const void *k, const void *v, void *o, int64_t batch,
                   int64_t num_heads, int64_t num_kv_heads, int64_t seq_len, int64_t head_dim,
                   int causal, double scale, void *stream);

/* Prefill over packed variable-length sequences (no padding), GQA allowed.
 *   q, o: fp16 [total_rows, num_heads, head_dim]; k, v: fp16 [total_rows,
 *         num_kv_heads, head_dim]; sequence b is rows cu_seqlens[b] ..
 *         cu_seqlens[b+1] - 1 of all four (self-attention: same lengths for q, k)
 *   cu_seqlens: int32 [batch + 1], device memory, non-decreasing
 *   max_seqlen: host value >= every sequence length (it sizes the grid)
 * Each sequence attends only within itself; causal masks key j > query i of the
 * same sequence.  Sequence rows are clamped into [0, total_rows): inconsistent
 * offsets give wrong rows, never an access out of bounds; rows of a sequence
 * beyond max_seqlen are not written.  The reference's prefill is dense only
 * (attnkernels/__init__.py:53-61); this is the same kernel on a row-strided layout. */
int ak_prefill_varlen(const void *q, const void *k, const void *v, void *o,
                      const int32_t *cu_seqlens, int64_t batch, int64_t total_rows,
                      int64_t num_heads, int64_t num_kv_heads, int64_t max_seqlen,
                      int64_t head_dim, int causal, double scale, void *stream);

/* Bytes of device workspace ak_paged_decode needs for these sizes: the fp32
 * split partials o [B, Hq, S, D], m and l [B, Hq, S] with S = ceil(max_context_len /
 * partition), or 0 when S == 1.  Replaces the torch::empty partials of
 * launch_decode (attnkernels/csrc/paged_decode.cu:227-235).  Returns 0 for
 * invalid sizes. */
size_t ak_paged_decode_workspace_size(int64_t batch, int64_t num_heads, int64_t head_dim,
                                      int64_t max_context_len, int64_t partition);

/* Paged-KV decode with split-K, replacing paged_decode
 * (attnkernels/csrc/paged_decode.cu:256-277, ext.cpp:17).
 *   q:            fp16 [batch, num_heads, head_dim], one query token per sequence
 *   k_cache, v_cache: fp16 [num_blocks, num_kv_heads, block_size, head_dim]
 *   block_tables: int32 [batch, max_blocks_per_seq], physical page ids
 *   context_lens: int32 [batch], tokens of context (>= 1) per sequence; a
 *                 sequence with 0 (or less) gets a zero output row
 *   out:          fp16 [batch, num_heads, head_dim]
 *   max_context_len: host value >= every context length
 *   partition:    tokens per split, a positive multiple of 256
 *   workspace:    device memory of at least ak_paged_decode_workspace_size() bytes
 *                 (may be NULL when that size is 0); contents are scratch.
 * head_dim 64/128 and num_heads/num_kv_heads in {1, 2, 4, 8}.  Query head h
 * reads kv head h / (num_heads / num_kv_heads).  Page ids outside
 * [0, num_blocks) are never read (their tokens are left out of the softmax);
 * tokens at or beyond max_blocks_per_seq * block_size are ignored. */
int ak_paged_decode(const void *q, const void *k_cache, const void *v_cache,
                    const int32_t *block_tables, const int32_t *context_lens, void *out,
                    int64_t batch, int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                    int64_t num_blocks, int64_t block_size, int64_t max_blocks_per_seq,
                    int64_t max_context_len, double scale, int64_t partition, void *workspace,
                    size_t workspace_bytes, void *stream);

/* ak_paged_decode with the split merge in the decode kernel itself: no
 * separate reduce launch (about 4 us of a small decode step).  No counterpart
 * in the reference, which always launches paged_reduce_kernel
 * (attnkernels/csrc/paged_decode.cu:243-248).  The last split of each
 * (sequence, kv head) to finish merges the partials, which needs one int32
 * counter per (sequence, kv head):
 *   counters:     device int32 array of counters_len >= batch * num_kv_heads
 *                 elements, all zero before the first call; every call leaves
 *                 them zero, so one array serves any later call on the same
 *                 stream (calls that share it must not overlap).  NULL: the
 *                 reduce kernel merges, exactly as ak_paged_decode.
 * Launches with more than 32 splits merge in the reduce kernel either way
 * (its workgroups per row read the partials in parallel).  Arguments, results
 * and errors are otherwise those of ak_paged_decode. */
int ak_paged_decode_fused(const void *q, const void *k_cache, const void *v_cache,
                          const int32_t *block_tables, const int32_t *context_lens, void *out,
                          int64_t batch, int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                          int64_t num_blocks, int64_t block_size, int64_t max_blocks_per_seq,
                          int64_t max_context_len, double scale, int64_t partition, void *workspace,
                          size_t workspace_bytes, int32_t *counters, int64_t counters_len, void *stream);

/* Paged-KV decode that allocates nothing: ak_paged_decode without the
 * workspace arguments.  No counterpart in the reference; it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  The split partials live in
 * a static per-GPU device array of AK_PAGED_DECODE_NOALLOC_MAX_BYTES (32 MiB),
 * the split counters in another of 1 MiB; the call fails with
 * AK_ERR_WORKSPACE, before any HIP call, when ak_paged_decode_workspace_size()
 * for these sizes exceeds 32 MiB (e.g. 8 sequences x 32 query heads x 128
 * splits x D=128 need 17 MB).  With more than 262144 (sequence, kv head)
 * pairs the splits are merged by the reduce kernel instead.
 * The arrays belong to the library's code object: every process that loads it
 * holds these 33 MiB on each GPU where any of its kernels has run, until the
 * process ends, whether or not it calls this entry point.
 * The call calls no hipMalloc/hipFree; every call looks up the current
 * device's arrays (hipGetSymbolAddress, not an allocation), so no address
 * outlives a hipDeviceReset.  All calls on one GPU share the arrays: calls
 * that overlap on one GPU (other streams, other threads) race.  `stream` must
 * belong to the current device.  Arguments, results and errors are otherwise
 * those of ak_paged_decode. */
#define AK_PAGED_DECODE_NOALLOC_MAX_BYTES ((size_t)32 << 20)
int ak_paged_decode_noalloc(const void *q, const void *k_cache, const void *v_cache,
                            const int32_t *block_tables, const int32_t *context_lens, void *out,
                            int64_t batch, int64_t num_heads, int64_t num_kv_heads,
                            int64_t head_dim, int64_t num_blocks, int64_t block_size,
                            int64_t max_blocks_per_seq, int64_t max_context_len, double scale,
                            int64_t partition, void *stream);

/* Read-only streaming checksum: XORs the bytes / 16 16-byte words of src into
 * out[0..3] (uint32, device memory the caller zeroes first).  No counterpart
 * in the reference's kernels: it is the read ceiling of bench.py's measured
 * ceilings, as the reference's bench measures a device copy
 * (bench/bench.py:119-131).  bytes a multiple of 16, src 16-byte aligned. */
int ak_stream_checksum(const void *src, size_t bytes, uint32_t *out, void *stream);

/* Paged KV-cache writer ("reshape and cache"): appends new tokens' keys and
 * values to the paged cache that ak_paged_decode reads.  No counterpart in the
 * reference, which only reads the cache (attnkernels/csrc/paged_decode.cu:95-96);
 * the layout written is the reference's (attnkernels/reference.py:21-44).
 *   key, value:   [num_tokens, num_kv_heads, head_dim], 2-byte elements (fp16 or
 *                 bf16, copied bit for bit); token t starts key_stride (value_stride)
 *                 elements after token t-1, heads are contiguous (a row of a
 *                 larger projection output may be passed with its stride)
 *   k_cache, v_cache: [num_blocks, num_kv_heads, block_size, head_dim], same dtype
 *   slot_mapping: int64 [num_tokens]; token t is written to page
 *                 slot / block_size, row slot % block_size.  Negative slots
 *                 (padding) and slots >= num_blocks * block_size are skipped.
 * head_dim a multiple of 8 up to 512; strides multiples of 8 and >= num_kv_heads *
 * head_dim.  Two tokens with the same slot: one of them wins. */
int ak_reshape_and_cache(const void *key, const void *value, void *k_cache, void *v_cache,
                         const int64_t *slot_mapping, int64_t num_tokens, int64_t num_kv_heads,
                         int64_t head_dim, int64_t num_blocks, int64_t block_size,
                         int64_t key_stride, int64_t value_stride, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* ATTNKERNELS_H */
