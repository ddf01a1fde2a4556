// Paged KV-cache writer ("reshape and cache"): the step after a decode or a
// prefill that appends the new tokens' keys and values to the paged cache the
// decode kernel reads.  Not in the reference; its cache layout is the
// reference's (k/v cache [num_blocks, num_kv_heads, block_size, head_dim],
// attnkernels/reference.py:21-44, read at paged_decode.cu:95-96).
//
// Token t goes to page slot / block_size, row slot % block_size, for
// slot = slot_mapping[t]; a negative slot (padding) or one past the pool is
// skipped.  The move is a bit copy of 16-byte chunks, so fp16 and bf16 share
// the kernel.  HBM-bound: each chunk is read once (non-temporal) and written
// once; one lane per chunk, consecutive lanes on consecutive chunks of one
// token, so a token's Hkv * head_dim elements move in whole 64-byte lines.
#include <hip/hip_runtime.h>

#include "attn_kernels.hpp"

namespace ak {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kMaxWriteThreads = 256;

// One workgroup per (token, group of up to 256 chunks): the token index, its
// slot and the page arithmetic are wave-uniform (scalar registers); each lane
// moves one 16-byte chunk of K and one of V.
template <int CPR, bool POW2_BS>  // CPR = head_dim / 8 (0: runtime value)
__global__ void __launch_bounds__(kMaxWriteThreads)
cache_write_kernel(const u32x4* __restrict__ key, const u32x4* __restrict__ value, u32x4* __restrict__ k_cache,
                   u32x4* __restrict__ v_cache, const int64_t* __restrict__ slots, int hkv, int cpr_rt,
                   int64_t key_stride, int64_t value_stride, int64_t num_slots, int bs, int bs_shift) {
    const int cpr = CPR ? CPR : cpr_rt;
    const int64_t t = blockIdx.x;
    const int r = (int)(blockIdx.y * blockDim.x + threadIdx.x);  // = h * cpr + c: heads are contiguous
    const int64_t slot = slots[t];
    if (r >= hkv * cpr || slot < 0 || slot >= num_slots) return;
    const int64_t page = POW2_BS ? slot >> bs_shift : slot / bs;
    const int64_t row = slot - page * bs;
    const int h = r / cpr, c = r - h * cpr;
    const int64_t dst = ((page * hkv + h) * bs + row) * cpr + c;
    const u32x4 kx = __builtin_nontemporal_load(key + t * key_stride + r);
    const u32x4 vx = __builtin_nontemporal_load(value + t * value_stride + r);
    k_cache[dst] = kx;
    v_cache[dst] = vx;
}

template <int CPR>
static void launch_cw(const CacheWriteArgs& a, dim3 grid, int threads, bool pow2, int shift) {
    const auto* k = static_cast<const u32x4*>(a.key);
    const auto* v = static_cast<const u32x4*>(a.value);
    auto* kc = static_cast<u32x4*>(a.k_cache);
    auto* vc = static_cast<u32x4*>(a.v_cache);
    const int cpr = (int)(a.head_dim / 8);
    const hipStream_t s = (hipStream_t)a.stream;
    if (pow2)
        hipLaunchKernelGGL((cache_write_kernel<CPR, true>), grid, dim3(threads), 0, s, k, v, kc, vc, a.slots,
                           (int)a.hkv, cpr, a.key_stride / 8, a.value_stride / 8, a.num_blocks * a.bs, (int)a.bs,
                           shift);
    else
        hipLaunchKernelGGL((cache_write_kernel<CPR, false>), grid, dim3(threads), 0, s, k, v, kc, vc, a.slots,
                           (int)a.hkv, cpr, a.key_stride / 8, a.value_stride / 8, a.num_blocks * a.bs, (int)a.bs,
                           shift);
}

hipError_t cache_write_launch(const CacheWriteArgs& a) {
    const int per_token = (int)(a.hkv * (a.head_dim / 8));
    if (a.num_tokens == 0 || per_token == 0) return hipSuccess;
    const int threads = per_token >= kMaxWriteThreads ? kMaxWriteThreads : (per_token + 63) / 64 * 64;
    const dim3 grid((unsigned)a.num_tokens, (unsigned)((per_token + threads - 1) / threads));
    const bool pow2 = (a.bs & (a.bs - 1)) == 0;
    const int shift = pow2 ? __builtin_ctzll((unsigned long long)a.bs) : 0;
    if (a.head_dim == 128)
        launch_cw<16>(a, grid, threads, pow2, shift);
    else if (a.head_dim == 64)
        launch_cw<8>(a, grid, threads, pow2, shift);
    else
        launch_cw<0>(a, grid, threads, pow2, shift);
    return hipGetLastError();
}

}  // namespace ak
