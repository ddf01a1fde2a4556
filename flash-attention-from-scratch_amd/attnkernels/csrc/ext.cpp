// Thin PyTorch-ROCm glue: the pybind module `attnkernels_ext` with the
// reference's four functions (attnkernels/csrc/ext.cpp:3-17) plus the paged
// cache writer reshape_and_cache and the GQA / varlen prefill, each allocating
// its output (and split-K workspace) from the caching allocator and calling
// the C-ABI in include/attnkernels.h on the caller's current HIP stream.
#include <torch/extension.h>

// PyTorch-ROCm reports GPU tensors with device type "cuda"; these are its
// guard and stream accessors for that device type.
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>

#include <map>
#include <mutex>
#include <utility>
#include <vector>

#include "attnkernels.h"

namespace {

void check_rc(int rc) { TORCH_CHECK(rc == AK_OK, ak_last_error()); }

void check_prefill(const torch::Tensor& q, const torch::Tensor& k, const torch::Tensor& v) {
    for (const auto* t : {&q, &k, &v}) {
        TORCH_CHECK(t->is_cuda() && t->scalar_type() == torch::kHalf && t->dim() == 4 && t->is_contiguous(),
                    "q, k, v must be contiguous fp16 GPU tensors of shape [B, H, N, D]");
        TORCH_CHECK(t->device() == q.device(), "q, k, v must be on the same device");
    }
    TORCH_CHECK(q.sizes() == k.sizes() && q.sizes() == v.sizes(),
                "q, k, v must have the same shape (self-attention prefill)");
}

void* stream_of(const torch::Tensor& t) {
    return at::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.device().index()).stream();
}

// Split counters of the decode kernels' in-kernel merge, one array per
// (device, stream): zeroed when allocated, and every decode call leaves its
// counters at zero, so the calls on a stream (which run in order) share it.
// A stream that needs more counters gets a new, larger array; the smaller one
// is kept, because a captured graph may still use it.
// The cache is never destroyed: its tensors would otherwise be freed during
// static destruction, after torch's allocator or the HIP runtime may be gone.
torch::Tensor split_counters(const torch::Tensor& q, int64_t n) {
    static std::mutex mu;
    static auto* cache = new std::map<std::pair<int, void*>, std::vector<torch::Tensor>>();
    std::lock_guard<std::mutex> lock(mu);
    auto& arrays = (*cache)[{(int)q.device().index(), stream_of(q)}];
    if (arrays.empty() || arrays.back().numel() < n) {
        const int64_t grow = arrays.empty() ? 0 : 2 * arrays.back().numel();
        arrays.push_back(torch::zeros({std::max(n, std::max<int64_t>(grow, 4096))}, q.options().dtype(torch::kInt)));
    }
    return arrays.back();
}

}  // namespace

torch::Tensor naive_attention(torch::Tensor q, torch::Tensor k, torch::Tensor v, bool causal, double scale) {
    check_prefill(q, k, v);
    const at::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
    auto o = torch::empty_like(q);
    check_rc(ak_naive_attention(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), q.size(0), q.size(1),
                                q.size(2), q.size(3), causal, scale, stream_of(q)));
    return o;
}

torch::Tensor flash_simt(torch::Tensor q, torch::Tensor k, torch::Tensor v, bool causal, double scale) {
    check_prefill(q, k, v);
    const at::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
    auto o = torch::empty_like(q);
    check_rc(ak_flash_simt(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), q.size(0), q.size(1),
                           q.size(2), q.size(3), causal, scale, stream_of(q)));
    return o;
}

torch::Tensor flash_wmma(torch::Tensor q, torch::Tensor k, torch::Tensor v, bool causal, double scale,
                         int64_t block_n) {
    check_prefill(q, k, v);
    const at::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
    auto o = torch::empty_like(q);
    check_rc(ak_flash_wmma(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), q.size(0), q.size(1),
                           q.size(2), q.size(3), causal, scale, block_n, stream_of(q)));
    return o;
}

// Dense prefill with fewer kv heads than query heads (GQA/MQA).
torch::Tensor flash_gqa(torch::Tensor q, torch::Tensor k, torch::Tensor v, bool causal, double scale) {
    for (const auto* t : {&q, &k, &v}) {
        TORCH_CHECK(t->is_cuda() && t->scalar_type() == torch::kHalf && t->dim() == 4 && t->is_contiguous(),
                    "q, k, v must be contiguous fp16 GPU tensors of shape [B, H, N, D]");
        TORCH_CHECK(t->device() == q.device(), "q, k, v must be on the same device");
    }
    TORCH_CHECK(k.sizes() == v.sizes() && k.size(0) == q.size(0) && k.size(2) == q.size(2) && k.size(3) == q.size(3),
                "k and v must be [B, H_kv, N, D] with q's B, N and D");
    const at::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
    auto o = torch::empty_like(q);
    check_rc(ak_prefill_gqa(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), q.size(0), q.size(1), k.size(1),
                            q.size(2), q.size(3), causal, scale, stream_of(q)));
    return o;
}

// Packed variable-length prefill: q [T, H, D], k/v [T, H_kv, D], cu_seqlens int32 [B + 1].
torch::Tensor flash_varlen(torch::Tensor q, torch::Tensor k, torch::Tensor v, torch::Tensor cu, int64_t max_seqlen,
                           bool causal, double scale) {
    for (const auto* t : {&q, &k, &v}) {
        TORCH_CHECK(t->is_cuda() && t->scalar_type() == torch::kHalf && t->dim() == 3 && t->is_contiguous(),
                    "q, k, v must be contiguous fp16 GPU tensors of shape [total, H, D]");
        TORCH_CHECK(t->device() == q.device(), "q, k, v must be on the same device");
    }
    TORCH_CHECK(k.sizes() == v.sizes() && k.size(0) == q.size(0) && k.size(2) == q.size(2),
                "k and v must be [total, H_kv, D] with q's total and D");
    TORCH_CHECK(cu.scalar_type() == torch::kInt && cu.dim() == 1 && cu.is_contiguous() && cu.size(0) >= 1 &&
                    cu.device() == q.device(),
                "cu_seqlens must be a contiguous int32 tensor [B + 1] on q's device");
    const at::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
    auto o = torch::empty_like(q);
    check_rc(ak_prefill_varlen(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), cu.data_ptr<int32_t>(),
                               cu.size(0) - 1, q.size(0), q.size(1), k.size(1), max_seqlen, q.size(2), causal, scale,
                               stream_of(q)));
    return o;
}

torch::Tensor paged_decode(torch::Tensor q, torch::Tensor kc, torch::Tensor vc, torch::Tensor bt,
                           torch::Tensor ctx, int64_t max_ctx, double scale, int64_t partition) {
    TORCH_CHECK(q.is_cuda() && q.scalar_type() == torch::kHalf && q.dim() == 3 && q.is_contiguous(),
                "q must be a contiguous fp16 GPU tensor [B, H, D]");
    TORCH_CHECK(kc.is_cuda() && kc.scalar_type() == torch::kHalf && kc.dim() == 4 && kc.is_contiguous() &&
                    vc.sizes() == kc.sizes() && vc.scalar_type() == torch::kHalf && vc.is_contiguous(),
                "k_cache and v_cache must be contiguous fp16 GPU tensors [num_blocks, H_kv, block_size, D]");
    TORCH_CHECK(kc.size(3) == q.size(2), "head_dim of q and the cache must match");
    TORCH_CHECK(bt.scalar_type() == torch::kInt && bt.dim() == 2 && bt.is_contiguous() && bt.size(0) == q.size(0),
                "block_tables must be a contiguous int32 tensor [B, max_blocks]");
    TORCH_CHECK(ctx.scalar_type() == torch::kInt && ctx.dim() == 1 && ctx.is_contiguous() && ctx.size(0) == q.size(0),
                "context_lens must be a contiguous int32 tensor [B]");
    for (const auto* t : {&kc, &vc, &bt, &ctx})
        TORCH_CHECK(t->device() == q.device(), "all paged_decode tensors must be on the same device");
    const at::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
    auto out = torch::empty_like(q);
    const int64_t B = q.size(0), hq = q.size(1), D = q.size(2), hkv = kc.size(1);
    const size_t ws_bytes = ak_paged_decode_workspace_size(B, hq, D, max_ctx, partition);
    torch::Tensor ws, counters;
    if (ws_bytes > 0) {
        ws = torch::empty({(int64_t)ws_bytes}, q.options().dtype(torch::kByte));
        counters = split_counters(q, B * hkv);
    }
    check_rc(ak_paged_decode_fused(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), bt.data_ptr<int32_t>(),
                                   ctx.data_ptr<int32_t>(), out.data_ptr(), B, hq, hkv, D, kc.size(0), kc.size(2),
                                   bt.size(1), max_ctx, scale, partition, ws_bytes ? ws.data_ptr() : nullptr,
                                   ws_bytes, ws_bytes ? counters.data_ptr<int32_t>() : nullptr,
                                   ws_bytes ? counters.numel() : 0, stream_of(q)));
    return out;
}

// In place: writes key/value rows into the caches (no counterpart in the
// reference, whose decode only reads the cache).
void reshape_and_cache(torch::Tensor key, torch::Tensor value, torch::Tensor kc, torch::Tensor vc,
                       torch::Tensor slots) {
    TORCH_CHECK(key.is_cuda() && key.dim() == 3 && value.dim() == 3 && key.sizes() == value.sizes(),
                "key and value must be GPU tensors [num_tokens, H_kv, D] of the same shape");
    TORCH_CHECK(key.element_size() == 2 && value.scalar_type() == key.scalar_type() &&
                    kc.scalar_type() == key.scalar_type() && vc.scalar_type() == key.scalar_type(),
                "key, value and the caches must share one 2-byte dtype (fp16 or bf16)");
    TORCH_CHECK(key.stride(2) == 1 && key.stride(1) == key.size(2) && value.stride(2) == 1 &&
                    value.stride(1) == value.size(2),
                "key and value must have contiguous heads (any token stride)");
    TORCH_CHECK(kc.dim() == 4 && kc.is_contiguous() && vc.is_contiguous() && vc.sizes() == kc.sizes() &&
                    kc.size(1) == key.size(1) && kc.size(3) == key.size(2),
                "k_cache and v_cache must be contiguous [num_blocks, H_kv, block_size, D] matching key");
    TORCH_CHECK(slots.scalar_type() == torch::kLong && slots.dim() == 1 && slots.is_contiguous() &&
                    slots.size(0) == key.size(0),
                "slot_mapping must be a contiguous int64 tensor [num_tokens]");
    for (const auto* t : {&value, &kc, &vc, &slots})
        TORCH_CHECK(t->device() == key.device(), "all reshape_and_cache tensors must be on the same device");
    const at::hip::HIPGuardMasqueradingAsCUDA guard(key.device());
    const int64_t T = key.size(0);
    check_rc(ak_reshape_and_cache(key.data_ptr(), value.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                                  slots.data_ptr<int64_t>(), T, key.size(1), key.size(2), kc.size(0), kc.size(2),
                                  T > 1 ? key.stride(0) : key.size(1) * key.size(2),
                                  T > 1 ? value.stride(0) : value.size(1) * value.size(2), stream_of(key)));
}

// XOR checksum of a tensor's bytes (a multiple of 16): the read-only
// streaming kernel behind bench.py's HBM read ceiling.
// out (int32[4] on x's device) accumulates the XOR when given: the caller
// zeroes it; without it a zeroed one is made.
torch::Tensor stream_checksum(torch::Tensor x, c10::optional<torch::Tensor> out_opt) {
    TORCH_CHECK(x.is_cuda() && x.is_contiguous() && x.nbytes() % 16 == 0,
                "stream_checksum: a contiguous GPU tensor of a multiple of 16 bytes");
    const at::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    torch::Tensor out;
    if (out_opt.has_value()) {
        out = *out_opt;
        TORCH_CHECK(out.device() == x.device() && out.scalar_type() == torch::kInt && out.numel() == 4 &&
                        out.is_contiguous(),
                    "stream_checksum: out must be a contiguous int32[4] on the input's device");
    } else {
        out = torch::zeros({4}, x.options().dtype(torch::kInt));
    }
    check_rc(ak_stream_checksum(x.data_ptr(), x.nbytes(), reinterpret_cast<uint32_t*>(out.data_ptr<int32_t>()),
                                stream_of(x)));
    return out;
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.doc() = "gfx950 attention kernels: MFMA flash prefill, paged split-K decode";
    m.def("naive_attention", &naive_attention, "prefill attention (served by the MFMA flash kernel)");
    m.def("flash_simt", &flash_simt, "prefill attention (served by the MFMA flash kernel)");
    m.def("flash_wmma", &flash_wmma, "tiled attention with online softmax on MFMA matrix cores");
    m.def("paged_decode", &paged_decode, "decode attention over a paged KV cache, split-K");
    m.def("stream_checksum", &stream_checksum, "XOR checksum of a tensor's bytes (read-only streaming ceiling)",
          py::arg("x"), py::arg("out") = py::none());
    m.def("reshape_and_cache", &reshape_and_cache, "write new tokens' K/V rows into the paged caches");
    m.def("flash_gqa", &flash_gqa, "dense prefill with grouped-query attention");
    m.def("flash_varlen", &flash_varlen, "prefill over packed variable-length sequences");
}
