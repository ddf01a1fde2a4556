// C-ABI entry points (include/attnkernels.h): argument validation, the
// reference's error wording, and dispatch to the HIP launchers.  Validation
// runs before any HIP call, so a rejected call never touches the GPU.
#include <climits>
#include <cmath>
#include <cstdio>
#include <string>

#include "attn_kernels.hpp"
#include "attnkernels.h"

static_assert(AK_PAGED_DECODE_NOALLOC_MAX_BYTES == ak::kDecodeScratchBytes,
              "the header states the static scratch size");

namespace {

thread_local std::string g_last_error;
constexpr double kLog2e = 1.4426950408889634;
constexpr int64_t kChunk = 256;  // partitions are multiples of it (paged_decode.cu:37)

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

int ok() {
    g_last_error.clear();
    return AK_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int hip_status(hipError_t e, const char* who) {
    if (e == hipSuccess) return ok();
    return fail(AK_ERR_HIP, std::string(who) + ": HIP error: " + hipGetErrorString(e));
}

// Shared by every prefill entry point.  kv_heads divides heads (GQA); cu is
// null for the dense [B, H, N, D] layout, else the packed layout's sequence
// starts with total_rows rows in q/k/v and seq_len the longest sequence.
int prefill(const char* who, const void* q, const void* k, const void* v, void* o, int64_t batch,
            int64_t heads, int64_t kv_heads, int64_t seq_len, int64_t head_dim, int causal, double scale,
            const int32_t* cu, int64_t total_rows, void* stream) {
    if (batch < 0 || heads < 0 || seq_len < 0 || kv_heads < 0 || total_rows < 0)
        return fail(AK_ERR_INVALID_ARGUMENT, std::string(who) + ": negative size");
    if (kv_heads == 0 ? heads != 0 : heads % kv_heads != 0)
        return fail(AK_ERR_INVALID_ARGUMENT, std::string(who) + ": num_heads must be a multiple of num_kv_heads");
    if (batch * heads * seq_len == 0 || (cu && total_rows == 0)) return ok();  // nothing to compute
    if (!q || !k || !v || !o) return fail(AK_ERR_INVALID_ARGUMENT, std::string(who) + ": null pointer");
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
        return fail(AK_ERR_INVALID_ARGUMENT, std::string(who) + ": pointers must be 16-byte aligned");
    // Workgroups = query-tile units (128 or 256 rows, causal: pairs) x batch x
    // heads: an int, counted here for the smaller tile.
    const int64_t tiles = (seq_len + 127) / 128, units = causal ? (tiles + 1) / 2 : tiles;
    if (seq_len > INT_MAX / 2 || total_rows > INT_MAX / 2 || batch * heads > INT_MAX / units)
        return fail(AK_ERR_INVALID_ARGUMENT, std::string(who) + ": size out of range");
    ak::PrefillArgs a{};
    a.q = q;
    a.k = k;
    a.v = v;
    a.o = o;
    a.bh = batch * heads;
    a.hq = heads;
    a.hkv = kv_heads;
    a.cu = cu;
    a.total_rows = total_rows;
    a.n = seq_len;
    a.d = (int)head_dim;
    a.causal = causal != 0;
    // |scale| * log2(e), kept >= 1e-30 so that masked scores (-inf) still map to
    // 2^-inf = 0; below that every score rounds to the same weight anyway.
    a.sl2 = (float)std::fmax(std::fabs(scale) * kLog2e, 1e-30);
    a.qflip = std::signbit(scale) && scale != 0.0 ? 0x80008000u : 0u;
    a.stream = stream;
    return hip_status(ak::prefill_launch(a), who);
}

// Validation shared by both decode entry points, in the reference's order
// (paged_decode.cu:260-262, 275), and the launch arguments except the split
// partials.  batch == 0 passes validation with nothing to launch.
int decode_args(const void* q, const void* k_cache, const void* v_cache, const int32_t* block_tables,
                const int32_t* context_lens, void* out, int64_t batch, int64_t num_heads, int64_t num_kv_heads,
                int64_t head_dim, int64_t num_blocks, int64_t block_size, int64_t max_blocks_per_seq,
                int64_t max_context_len, double scale, int64_t partition, void* stream, ak::DecodeArgs& a) {
    if (num_kv_heads <= 0 || num_heads <= 0 || num_heads % num_kv_heads != 0)
        return fail(AK_ERR_INVALID_ARGUMENT, "num_heads must be a multiple of num_kv_heads");
    if (partition <= 0 || partition % kChunk != 0)
        return fail(AK_ERR_INVALID_ARGUMENT, "partition size must be a positive multiple of 256");
    const int64_t G = num_heads / num_kv_heads;
    if ((head_dim != 64 && head_dim != 128) || (G != 1 && G != 2 && G != 4 && G != 8))
        return fail(AK_ERR_UNSUPPORTED,
                    "paged_decode: head_dim must be 64/128 and num_heads/num_kv_heads in {1,2,4,8}");
    if (batch < 0 || num_blocks < 0 || block_size <= 0 || max_blocks_per_seq < 0)
        return fail(AK_ERR_INVALID_ARGUMENT, "paged_decode: invalid size");
    if (batch == 0) return ok();
    if (max_context_len < 1)
        return fail(AK_ERR_INVALID_ARGUMENT, "paged_decode: max_context_len must be >= 1");
    if (max_blocks_per_seq < 1 || num_blocks < 1)
        return fail(AK_ERR_INVALID_ARGUMENT, "paged_decode: empty block table or cache");
    if (!q || !k_cache || !v_cache || !block_tables || !context_lens || !out)
        return fail(AK_ERR_INVALID_ARGUMENT, "paged_decode: null pointer");
    if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned16(out))
        return fail(AK_ERR_INVALID_ARGUMENT, "paged_decode: q, caches and out must be 16-byte aligned");
    if ((reinterpret_cast<uintptr_t>(block_tables) & 3u) || (reinterpret_cast<uintptr_t>(context_lens) & 3u))
        return fail(AK_ERR_INVALID_ARGUMENT, "paged_decode: int32 arrays must be 4-byte aligned");
    if (max_context_len > INT_MAX - partition || partition > INT_MAX || num_blocks > INT_MAX ||
        max_blocks_per_seq * block_size > INT_MAX || batch > 65535 || num_kv_heads > 65535)
        return fail(AK_ERR_INVALID_ARGUMENT, "paged_decode: size out of range");
    const int64_t splits = (max_context_len + partition - 1) / partition;
    if (splits > 65535) return fail(AK_ERR_INVALID_ARGUMENT, "paged_decode: more than 65535 splits");
    a.q = q;
    a.k_cache = k_cache;
    a.v_cache = v_cache;
    a.block_tables = block_tables;
    a.context_lens = context_lens;
    a.out = out;
    a.batch = batch;
    a.hq = num_heads;
    a.hkv = num_kv_heads;
    a.d = head_dim;
    a.num_blocks = num_blocks;
    a.bs = block_size;
    a.max_blocks = max_blocks_per_seq;
    a.partition = partition;
    a.num_splits = splits;
    a.sl2 = (float)(scale * kLog2e);
    a.stream = stream;
    return ok();
}

// Bytes of the split partials in one fp32 buffer: o [B, Hq, S, D], m [B, Hq, S], l [B, Hq, S].
size_t partials_bytes(int64_t batch, int64_t num_heads, int64_t splits, int64_t head_dim) {
    return (size_t)batch * (size_t)num_heads * (size_t)splits * (size_t)(head_dim + 2) * sizeof(float);
}

void set_partials(ak::DecodeArgs& a, void* buf) {
    float* ws = static_cast<float*>(buf);
    const size_t rows = (size_t)a.batch * (size_t)a.hq * (size_t)a.num_splits;
    a.o_part = ws;
    a.m_part = ws + rows * (size_t)a.d;
    a.l_part = a.m_part + rows;
}

}  // namespace

extern "C" {

const char* ak_last_error(void) { return g_last_error.c_str(); }

int ak_abi_version(void) { return 101; }

int ak_naive_attention(const void* q, const void* k, const void* v, void* o, int64_t batch,
                       int64_t heads, int64_t seq_len, int64_t head_dim, int causal, double scale,
                       void* stream) {
    if (head_dim != 64 && head_dim != 128)
        return fail(AK_ERR_UNSUPPORTED, "naive_attention: head_dim must be 64 or 128");
    return prefill("naive_attention", q, k, v, o, batch, heads, heads, seq_len, head_dim, causal, scale, nullptr, 0,
                   stream);
}

int ak_flash_simt(const void* q, const void* k, const void* v, void* o, int64_t batch, int64_t heads,
                  int64_t seq_len, int64_t head_dim, int causal, double scale, void* stream) {
    if (head_dim != 64 && head_dim != 128)
        return fail(AK_ERR_UNSUPPORTED, "flash_simt: head_dim must be 64 or 128");
    return prefill("flash_simt", q, k, v, o, batch, heads, heads, seq_len, head_dim, causal, scale, nullptr, 0,
                   stream);
}

int ak_flash_wmma(const void* q, const void* k, const void* v, void* o, int64_t batch, int64_t heads,
                  int64_t seq_len, int64_t head_dim, int causal, double scale, int64_t block_n,
                  void* stream) {
    if ((head_dim != 64 && head_dim != 128) || (block_n != 32 && block_n != 64))
        return fail(AK_ERR_UNSUPPORTED, "flash_wmma: head_dim must be 64 or 128 and block_n 32 or 64");
    return prefill("flash_wmma", q, k, v, o, batch, heads, heads, seq_len, head_dim, causal, scale, nullptr, 0,
                   stream);
}

int ak_prefill_gqa(const void* q, const void* k, const void* v, void* o, int64_t batch, int64_t num_heads,
                   int64_t num_kv_heads, int64_t seq_len, int64_t head_dim, int causal, double scale,
                   void* stream) {
    if (head_dim != 64 && head_dim != 128)
        return fail(AK_ERR_UNSUPPORTED, "prefill_gqa: head_dim must be 64 or 128");
    return prefill("prefill_gqa", q, k, v, o, batch, num_heads, num_kv_heads, seq_len, head_dim, causal, scale,
                   nullptr, 0, stream);
}

int ak_prefill_varlen(const void* q, const void* k, const void* v, void* o, const int32_t* cu_seqlens,
                      int64_t batch, int64_t total_rows, int64_t num_heads, int64_t num_kv_heads,
                      int64_t max_seqlen, int64_t head_dim, int causal, double scale, void* stream) {
    if (head_dim != 64 && head_dim != 128)
        return fail(AK_ERR_UNSUPPORTED, "prefill_varlen: head_dim must be 64 or 128");
    if (batch > 0 && (!cu_seqlens || (reinterpret_cast<uintptr_t>(cu_seqlens) & 3u)))
        return fail(AK_ERR_INVALID_ARGUMENT, "prefill_varlen: cu_seqlens must be a 4-byte aligned int32 array");
    return prefill("prefill_varlen", q, k, v, o, batch, num_heads, num_kv_heads, max_seqlen, head_dim, causal,
                   scale, batch > 0 ? cu_seqlens : nullptr, total_rows, stream);
}

size_t ak_paged_decode_workspace_size(int64_t batch, int64_t num_heads, int64_t head_dim,
                                      int64_t max_context_len, int64_t partition) {
    if (batch < 0 || num_heads < 0 || head_dim <= 0 || max_context_len < 1 || partition <= 0) return 0;
    const int64_t splits = (max_context_len + partition - 1) / partition;
    if (splits <= 1) return 0;
    return partials_bytes(batch, num_heads, splits, head_dim);
}

int ak_paged_decode(const void* q, const void* k_cache, const void* v_cache, const int32_t* block_tables,
                    const int32_t* context_lens, void* out, int64_t batch, int64_t num_heads,
                    int64_t num_kv_heads, int64_t head_dim, int64_t num_blocks, int64_t block_size,
                    int64_t max_blocks_per_seq, int64_t max_context_len, double scale, int64_t partition,
                    void* workspace, size_t workspace_bytes, void* stream) {
    return ak_paged_decode_fused(q, k_cache, v_cache, block_tables, context_lens, out, batch, num_heads,
                                 num_kv_heads, head_dim, num_blocks, block_size, max_blocks_per_seq,
                                 max_context_len, scale, partition, workspace, workspace_bytes, nullptr, 0, stream);
}

int ak_paged_decode_fused(const void* q, const void* k_cache, const void* v_cache, const int32_t* block_tables,
                          const int32_t* context_lens, void* out, int64_t batch, int64_t num_heads,
                          int64_t num_kv_heads, int64_t head_dim, int64_t num_blocks, int64_t block_size,
                          int64_t max_blocks_per_seq, int64_t max_context_len, double scale, int64_t partition,
                          void* workspace, size_t workspace_bytes, int32_t* counters, int64_t counters_len,
                          void* stream) {
    ak::DecodeArgs a{};
    const int rc = decode_args(q, k_cache, v_cache, block_tables, context_lens, out, batch, num_heads, num_kv_heads,
                               head_dim, num_blocks, block_size, max_blocks_per_seq, max_context_len, scale,
                               partition, stream, a);
    if (rc != AK_OK || batch == 0) return rc;
    if (counters && (counters_len < batch * num_kv_heads || (reinterpret_cast<uintptr_t>(counters) & 3u)))
        return fail(AK_ERR_INVALID_ARGUMENT, "paged_decode: counters must be a 4-byte aligned int32 array of at least "
                                             "batch * num_kv_heads = " + std::to_string(batch * num_kv_heads) +
                                             " elements");
    if (a.num_splits > 1) {
        const size_t need = ak_paged_decode_workspace_size(batch, num_heads, head_dim, max_context_len, partition);
        if (!workspace || workspace_bytes < need)
            return fail(AK_ERR_WORKSPACE, "paged_decode: workspace of " + std::to_string(need) +
                                              " bytes required, got " + std::to_string(workspace_bytes));
        if (!aligned16(workspace))
            return fail(AK_ERR_INVALID_ARGUMENT, "paged_decode: workspace must be 16-byte aligned");
        set_partials(a, workspace);
        a.counters = counters;
    }
    return hip_status(ak::decode_launch(a), "paged_decode");
}

int ak_paged_decode_noalloc(const void* q, const void* k_cache, const void* v_cache, const int32_t* block_tables,
                            const int32_t* context_lens, void* out, int64_t batch, int64_t num_heads,
                            int64_t num_kv_heads, int64_t head_dim, int64_t num_blocks, int64_t block_size,
                            int64_t max_blocks_per_seq, int64_t max_context_len, double scale, int64_t partition,
                            void* stream) {
    ak::DecodeArgs a{};
    const int rc = decode_args(q, k_cache, v_cache, block_tables, context_lens, out, batch, num_heads, num_kv_heads,
                               head_dim, num_blocks, block_size, max_blocks_per_seq, max_context_len, scale,
                               partition, stream, a);
    if (rc != AK_OK || batch == 0) return rc;
    if (a.num_splits > 1) {
        const size_t need = partials_bytes(batch, num_heads, a.num_splits, head_dim);
        if (need > ak::kDecodeScratchBytes)
            return fail(AK_ERR_WORKSPACE, "paged_decode_noalloc: the split partials need " + std::to_string(need) +
                                              " bytes, more than the static scratch of " +
                                              std::to_string(ak::kDecodeScratchBytes) +
                                              " bytes; use a larger partition or ak_paged_decode with a workspace");
        // The scratch array of the current device: the stream must run there.
        if (stream) {
            int cur = 0;
            hipDevice_t sdev = 0;
            hipError_t e = hipGetDevice(&cur);
            if (e == hipSuccess) e = hipStreamGetDevice((hipStream_t)stream, &sdev);
            if (e != hipSuccess) return hip_status(e, "paged_decode_noalloc");
            if ((int)sdev != cur)
                return fail(AK_ERR_INVALID_ARGUMENT,
                            "paged_decode_noalloc: the stream must belong to the current device");
        }
        void* ws = nullptr;
        int32_t* counters = nullptr;
        const hipError_t e = ak::decode_scratch(&ws, &counters);
        if (e != hipSuccess) return hip_status(e, "paged_decode_noalloc");
        set_partials(a, ws);
        // counters for every (sequence, kv head) fit the static array: merged in
        // the decode kernel; otherwise by the reduce kernel
        if ((size_t)batch * (size_t)num_kv_heads <= ak::kDecodeScratchCounters) a.counters = counters;
    }
    return hip_status(ak::decode_launch(a), "paged_decode_noalloc");
}

int ak_reshape_and_cache(const void* key, const void* value, void* k_cache, void* v_cache,
                         const int64_t* slot_mapping, int64_t num_tokens, int64_t num_kv_heads,
                         int64_t head_dim, int64_t num_blocks, int64_t block_size, int64_t key_stride,
                         int64_t value_stride, void* stream) {
    if (num_tokens < 0 || num_kv_heads <= 0 || num_blocks < 0 || block_size <= 0)
        return fail(AK_ERR_INVALID_ARGUMENT, "reshape_and_cache: invalid size");
    if (head_dim <= 0 || head_dim % 8 != 0 || head_dim > 512)
        return fail(AK_ERR_UNSUPPORTED, "reshape_and_cache: head_dim must be a multiple of 8 up to 512");
    const int64_t row = num_kv_heads * head_dim;
    if (key_stride < row || value_stride < row || key_stride % 8 || value_stride % 8)
        return fail(AK_ERR_INVALID_ARGUMENT,
                    "reshape_and_cache: token strides must be multiples of 8 and >= num_kv_heads * head_dim");
    if (num_tokens == 0 || num_blocks == 0) return ok();  // nothing to write, or no slot in range
    if (!key || !value || !k_cache || !v_cache || !slot_mapping)
        return fail(AK_ERR_INVALID_ARGUMENT, "reshape_and_cache: null pointer");
    if (!aligned16(key) || !aligned16(value) || !aligned16(k_cache) || !aligned16(v_cache) ||
        (reinterpret_cast<uintptr_t>(slot_mapping) & 7u))
        return fail(AK_ERR_INVALID_ARGUMENT, "reshape_and_cache: tensors must be 16-byte aligned");
    // Grid: x = token (< 2^31), y = groups of 256 chunks of one token (<= 65535).
    if (num_kv_heads * (head_dim / 8) > 65535LL * 256 || block_size > INT_MAX ||
        num_blocks > INT64_MAX / block_size / row || num_tokens > INT_MAX)
        return fail(AK_ERR_INVALID_ARGUMENT, "reshape_and_cache: size out of range");
    ak::CacheWriteArgs a{};
    a.key = key;
    a.value = value;
    a.k_cache = k_cache;
    a.v_cache = v_cache;
    a.slots = slot_mapping;
    a.num_tokens = num_tokens;
    a.hkv = num_kv_heads;
    a.head_dim = head_dim;
    a.num_blocks = num_blocks;
    a.bs = block_size;
    a.key_stride = key_stride;
    a.value_stride = value_stride;
    a.stream = stream;
    return hip_status(ak::cache_write_launch(a), "reshape_and_cache");
}

int ak_stream_checksum(const void* src, size_t bytes, uint32_t* out, void* stream) {
    if (bytes % 16 != 0) return fail(AK_ERR_INVALID_ARGUMENT, "stream_checksum: bytes must be a multiple of 16");
    if (bytes > 0 && (!src || !aligned16(src)))
        return fail(AK_ERR_INVALID_ARGUMENT, "stream_checksum: src must be a 16-byte aligned device pointer");
    if (!out || (reinterpret_cast<uintptr_t>(out) & 3u))
        return fail(AK_ERR_INVALID_ARGUMENT, "stream_checksum: out must be a 4-byte aligned device pointer");
    return hip_status(ak::stream_checksum_launch(src, bytes, out, stream), "stream_checksum");
}

}  // extern "C"
