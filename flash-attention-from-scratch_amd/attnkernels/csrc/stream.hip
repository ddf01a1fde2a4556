// Read-only streaming checksum: the HBM read ceiling bench.py reports beside
// the decode kernels' rates.
//
// The reference reports its kernels against a measured device copy
// (bench/bench.py:119-131).  On MI355X a copy (read + write) and the vendor
// reductions and GEMV (3.7-5.7 TB/s read) all stream slower than the paged
// decode kernels read, so they bound nothing; this kernel only reads.  Each
// workgroup reads one contiguous chunk of the buffer, every lane keeping 16
// non-temporal 16-byte loads in flight; one workgroup per CU.  Of the shapes
// measured on a 2 GiB buffer (grid-stride or chunked, 1-16 workgroups per CU,
// 128-1024 threads, 4-16 loads in flight) this one read fastest, 7.1 TB/s;
// more workgroups per CU read slower.  The XOR of all 16-byte words is the
// result (independent of order, so a test can recompute it on the host).
#include "attn_kernels.hpp"
#include "wave.hpp"

namespace ak {

constexpr int kStreamThreads = 256, kStreamUnroll = 16;

__global__ void __launch_bounds__(kStreamThreads)
stream_checksum_kernel(const u32x4* __restrict__ src, size_t words, size_t per_block, uint32_t* __restrict__ out) {
    constexpr size_t kGroup = (size_t)kStreamThreads * kStreamUnroll;
    const size_t lo = min(words, (size_t)blockIdx.x * per_block), hi = min(words, lo + per_block);
    size_t i = lo + threadIdx.x;
    u32x4 acc = {0u, 0u, 0u, 0u};
    // Whole groups: this lane's kStreamUnroll words of the group, all loads
    // issued before any is used.  The lane's words are lo + tid + m * threads.
    for (; i + (kStreamUnroll - 1) * kStreamThreads < hi; i += kGroup) {
        u32x4 w[kStreamUnroll];
#pragma unroll
        for (int k = 0; k < kStreamUnroll; ++k) w[k] = __builtin_nontemporal_load(src + i + k * kStreamThreads);
#pragma unroll
        for (int k = 0; k < kStreamUnroll; ++k) acc ^= w[k];
    }
    for (; i < hi; i += kStreamThreads) acc ^= __builtin_nontemporal_load(src + i);
    // XOR over the wave, then one agent-scope atomic per wave and word.
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        uint32_t x = acc[j];
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) x ^= (uint32_t)__shfl_xor((int)x, off, kWave);
        if ((threadIdx.x & (kWave - 1)) == 0 && x)
            __hip_atomic_fetch_xor(out + j, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

hipError_t stream_checksum_launch(const void* src, size_t bytes, uint32_t* out, void* stream) {
    const size_t words = bytes / 16;
    if (words == 0) return hipSuccess;
    int dev = 0, cus = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return e;
    // one workgroup per CU, fewer for a small buffer; chunks are whole groups
    constexpr size_t kGroup = (size_t)kStreamThreads * kStreamUnroll;
    const size_t groups = (words + kGroup - 1) / kGroup;
    const size_t grid = groups < (size_t)cus ? groups : (size_t)cus;
    const size_t per_block = (groups + grid - 1) / grid * kGroup;
    hipLaunchKernelGGL(stream_checksum_kernel, dim3((unsigned)grid), dim3(kStreamThreads), 0, (hipStream_t)stream,
                       static_cast<const u32x4*>(src), words, per_block, out);
    return hipGetLastError();
}

}  // namespace ak
