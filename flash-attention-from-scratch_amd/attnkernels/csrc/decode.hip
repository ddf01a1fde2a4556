// Paged-KV split-K decode ("flash-decoding") and its LSE-merge reduce, gfx950.
//
// Same contract as the reference's kernel pair (paged_decode.cu:39-216): the
// cache is [num_blocks, hkv, bs, D], token t of sequence b lives in page
// block_tables[b][t / bs] at offset t % bs; a workgroup handles one
// (split, kv head, sequence) and all G query heads that share the kv head, so
// every K/V byte is read once; it writes the normalised partial o and (m, l) in
// the log2 domain, or the fp16 output directly when there is one split; the
// reduce merges partials with M = max m_s, w_s = l_s 2^(m_s - M),
// O = sum w_s o_s / sum w_s.
//
// The kernel is built for HBM bandwidth, with no matrix cores:
//   * a token row of one page is D*2 contiguous bytes; D/8 lanes cover it with
//     one 16-byte load each, so one wave-wide load reads 4 (D=128) or 8 (D=64)
//     tokens = 1 KB; a D=128 lane keeps 16 K loads and 16 V loads in flight (4
//     waves per workgroup; with head groups 8 and 8, or 4 and 4 with 4 query
//     heads per kv head), a D=64 lane 4 and 4 (8 waves with one query head per
//     kv head, 4 with head groups): the fastest shape of each head size on
//     ragged and long-context paged caches, as measured on MI355X;
//   * the dot product is v_dot2_f32_f16 on the raw fp16 q and k, reduced over
//     the D/8 lanes of a token with DPP row permutes, then scaled by
//     scale*log2(e) in fp32;
//   * each group of D/8 lanes runs its own online softmax over the tokens it
//     loads (no cross-lane traffic in the loop); the groups of a wave and the
//     waves of a workgroup are merged once, at the end, by the same LSE rule;
//   * with head groups and 16-token pages, a wave's chunk is 1, 2 or 4 whole
//     pages: their ids are wave-uniform scalar loads and each K/V load is a
//     page base plus a lane offset plus an immediate, with no per-token page
//     arithmetic or masking; the context's tail, other page sizes and
//     out-of-range page ids take the checked per-token loads.
#include "attn_kernels.hpp"
#include "wave.hpp"

#include <mutex>
#include <type_traits>

namespace ak {

template <int D, int G>
struct DecodeTile {
    // Waves per workgroup.  With head groups a workgroup's fixed costs (page
    // ids, then K/V, before any work; the merge at the end) grow with G while
    // fewer of them fit on a CU, so D=64 takes 4 waves there: a 256-token
    // split is then 2 pipelined chunks per wave instead of 1 (1.1-2.1x at the
    // default partition on MI355X, equal at the best one).
    static constexpr int NW = D == 128 || G >= 2 ? 4 : 8;
    static constexpr int THREADS = NW * kWave;   // 256 or 512
    static constexpr int LPT = D / 8;            // lanes per token row
    static constexpr int TPL = kWave / LPT;      // tokens per wave-wide load
    // Loads in flight per lane, per cache.  D=128 with head groups spends the
    // registers on q and the accumulators instead, for more waves per SIMD: 8
    // with 2 query heads per kv head (127 VGPRs, 4 waves, against 229 and 2 at
    // 16) and with 8; 4 with 4 (115 VGPRs, 4 waves, against 162 and 3 at 8).
    static constexpr int U = D == 128 ? (G == 1 ? 16 : G == 4 ? 4 : 8) : 4;
    static constexpr int TOK = U * TPL;         // tokens per wave iteration
    // Page size of the fast path: a wave iteration then covers PPI whole pages
    // (its first token is a multiple of TOK, itself a multiple of 16).
    static constexpr int FAST_BS = 16;
    static constexpr int PPI = TOK / FAST_BS;
    static_assert(TOK % FAST_BS == 0 && FAST_BS % TPL == 0, "whole pages per wave iteration");
};

__device__ __forceinline__ float dot8(f16x8 a, f16x8 b) {
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const f16x2 x = {a[2 * j], a[2 * j + 1]};
        const f16x2 y = {b[2 * j], b[2 * j + 1]};
        s = __builtin_amdgcn_fdot2(x, y, s, false);
    }
    return s;
}

template <int D, int G>
__global__ void __launch_bounds__((DecodeTile<D, G>::THREADS))
paged_decode_kernel(const f16* __restrict__ q, const f16* __restrict__ kc, const f16* __restrict__ vc,
                    const int* __restrict__ block_tables, const int* __restrict__ ctx_lens,
                    f16* __restrict__ out, float* __restrict__ o_part, float* __restrict__ m_part,
                    float* __restrict__ l_part, int hkv, int bs, int bs_shift, int max_blocks,
                    int num_blocks, int partition, int num_splits, float sl2) {
    using T = DecodeTile<D, G>;
    __shared__ float red_acc[T::NW][G][D];
    __shared__ float red_m[T::NW][G], red_l[T::NW][G];

    // kv head fastest: neighbouring workgroups read neighbouring 4 KB head
    // blocks of the same pages.
    const int kvh = blockIdx.x, split = blockIdx.y, b = blockIdx.z;
    const int hq = hkv * G;
    const int start = split * partition;
    const int tid = threadIdx.x, lane = tid & 63, w = uniform(tid >> 6);
    const int gi = lane / T::LPT, li = lane % T::LPT;
    const int* bt = block_tables + (size_t)b * max_blocks;
    const int max_tok = max_blocks * bs;  // never index past the table row

    // Page ids of this lane's tokens in the chunk starting at t0, for tokens
    // below lim (-1 elsewhere).  They are loaded one chunk ahead, behind the
    // current chunk's K/V loads, so a chunk costs one memory round trip.
    auto load_pages = [&](int t0, int lim, int (&pg)[T::U]) {
#pragma unroll
        for (int u = 0; u < T::U; ++u) {
            const int t = t0 + u * T::TPL + gi;
            const int pi = bs_shift >= 0 ? (t >> bs_shift) : (t / bs);
            pg[u] = t < lim ? bt[pi] : -1;
        }
    };
    // The context length, q and the first chunk's page ids are loaded together:
    // the page loads are bounded by the table row, not by the (not yet known)
    // context length, which only masks them afterwards.
    const int ctx_raw = ctx_lens[b];
    f16x8 qv[G];  // q of the G heads of this kv head, raw fp16 (scaled after the dot product)
#pragma unroll
    for (int h = 0; h < G; ++h)
        qv[h] = *reinterpret_cast<const f16x8*>(q + ((size_t)b * hq + kvh * G + h) * D + li * 8);
    const int stride = T::NW * T::TOK;
    int pg[T::U];
    load_pages(start + w * T::TOK, min(start + partition, max_tok), pg);
    // Fast path (page size 16, a chunk wholly inside the context): the chunk's
    // PPI page ids are wave-uniform scalar loads, and every K/V load is one
    // instruction, page base (SGPR) + lane offset + immediate.  Loaded one
    // chunk ahead like pg; the first chunk's together with pg.  Head groups
    // only: with one query head per kv head the loop is not issue-bound, and
    // the checked loads measured 1% faster there (MI355X, same box); with 4 or
    // 8 heads this path is 4-11% faster.
    const bool fast_bs = G >= 2 && bs == T::FAST_BS;
    int spg[T::PPI];
    auto load_spages = [&](int t0) {
#pragma unroll
        for (int p = 0; p < T::PPI; ++p) spg[p] = bt[uniform((t0 >> 4) + p)];
    };
    if (fast_bs && start + w * T::TOK + T::TOK <= min(start + partition, max_tok)) load_spages(start + w * T::TOK);

    const int ctx = min(ctx_raw, max_tok);
    if (start >= ctx) {  // whole workgroup: this split is past the context
        // A sequence with no context (outside the >= 1 contract) gets a zero row,
        // as the reduce gives it when there are several splits.
        if (num_splits == 1)
            for (int idx = tid; idx < G * D; idx += T::THREADS)
                out[((size_t)b * hq + kvh * G + idx / D) * D + idx % D] = (f16)0.f;
        return;
    }
    const int end = min(ctx, start + partition);

    float m[G], l[G], acc[G][8];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        m[h] = -INFINITY;
        l[h] = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[h][i] = 0.f;
    }
    const size_t page_stride = (size_t)hkv * bs * D;
    const size_t head_off = (size_t)kvh * bs * D + li * 8;

    // Scores, online softmax and P V of one chunk: kr/vr hold token
    // t0 + u*TPL + gi of each u; tokens with !valid[u] drop out.
    auto consume = [&](const f16x8 (&kr)[T::U], const f16x8 (&vr)[T::U], const bool (&valid)[T::U], auto masked) {
        constexpr bool MASKED = decltype(masked)::value;
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float s[T::U];
            float mx = -INFINITY;
#pragma unroll
            for (int u = 0; u < T::U; ++u) {
                const float dsum = group_sum<T::LPT>(dot8(qv[h], kr[u]));
                s[u] = !MASKED || valid[u] ? dsum * sl2 : -INFINITY;
                mx = fmaxf(mx, s[u]);
            }
            const float m_new = fmaxf(m[h], mx);
            const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
            const float alpha = exp2_fast(m[h] - m_use);
            float psum = 0.f;
#pragma unroll
            for (int u = 0; u < T::U; ++u) {
                s[u] = exp2_fast(s[u] - m_use);
                psum += s[u];
            }
            l[h] = l[h] * alpha + psum;
            m[h] = m_new;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                float a = acc[h][i] * alpha;
#pragma unroll
                for (int u = 0; u < T::U; ++u) a = fmaf(s[u], (float)vr[u][i], a);
                acc[h][i] = a;
            }
        }
    };
    // Byte offset of this lane's 16 bytes inside a 16-token page of its kv head.
    const uint32_t lane_off = (uint32_t)(((size_t)kvh * T::FAST_BS * D + gi * D + li * 8) * sizeof(f16));

    // Fast loop: whole chunks of 16-token pages with valid page ids.  Its page
    // ids are prefetched as spg while the next chunk is also a fast one, else
    // as pg for the checked loop, which takes the rest (the context's tail,
    // other page sizes, out-of-range page ids).
    int t0 = start + w * T::TOK;
    while (fast_bs && t0 + T::TOK <= end) {
        bool pages_ok = true;
#pragma unroll
        for (int p = 0; p < T::PPI; ++p) pages_ok = pages_ok && (unsigned)spg[p] < (unsigned)num_blocks;
        if (!pages_ok) {
            load_pages(t0, end, pg);
            break;
        }
        f16x8 kr[T::U], vr[T::U];
#pragma unroll
        for (int u = 0; u < T::U; ++u) {
            const int p = u * T::TPL / T::FAST_BS, row = u * T::TPL % T::FAST_BS;
            const size_t pbase = (size_t)spg[p] * page_stride * sizeof(f16);
            const uint32_t off = lane_off + (uint32_t)(row * D * sizeof(f16));
            // K/V are streamed once: non-temporal loads keep them out of the caches' way.
            kr[u] = __builtin_nontemporal_load(
                reinterpret_cast<const f16x8*>(reinterpret_cast<const char*>(kc) + pbase + off));
            vr[u] = __builtin_nontemporal_load(
                reinterpret_cast<const f16x8*>(reinterpret_cast<const char*>(vc) + pbase + off));
        }
        const int tn = t0 + stride;
        if (tn + T::TOK <= end) load_spages(tn);
        else load_pages(tn, end, pg);
        const bool unused[T::U] = {};  // unmasked: every token of a whole-page chunk is valid
        consume(kr, vr, unused, std::false_type{});
        t0 = tn;
    }
    for (; t0 < end; t0 += stride) {
        f16x8 kr[T::U], vr[T::U];
        bool valid[T::U];
#pragma unroll
        for (int u = 0; u < T::U; ++u) {
            const int t = t0 + u * T::TPL + gi;
            const int po = bs_shift >= 0 ? (t & (bs - 1)) : (t % bs);
            const bool ok = t < end && (unsigned)pg[u] < (unsigned)num_blocks;  // bad page ids are never read
            const size_t off = (size_t)(ok ? pg[u] : 0) * page_stride + head_off + (size_t)po * D;
            valid[u] = ok;
            kr[u] = ok ? __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(kc + off)) : f16x8{};
            vr[u] = ok ? __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(vc + off)) : f16x8{};
        }
        load_pages(t0 + stride, end, pg);
        consume(kr, vr, valid, std::true_type{});
    }

    // Merge the token groups of the wave (lanes that share li), then the waves.
#pragma unroll
    for (int off = T::LPT; off < kWave; off <<= 1) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const float mo = __shfl_xor(m[h], off, kWave);
            const float lo = __shfl_xor(l[h], off, kWave);
            const float M = fmaxf(m[h], mo);
            const float Mu = (M == -INFINITY) ? 0.f : M;
            const float ws = exp2_fast(m[h] - Mu), wo = exp2_fast(mo - Mu);
            l[h] = l[h] * ws + lo * wo;
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[h][i] = acc[h][i] * ws + __shfl_xor(acc[h][i], off, kWave) * wo;
            m[h] = M;
        }
    }
    if (gi == 0) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
#pragma unroll
            for (int i = 0; i < 8; ++i) red_acc[w][h][li * 8 + i] = acc[h][i];
            if (li == 0) {
                red_m[w][h] = m[h];
                red_l[w][h] = l[h];
            }
        }
    }
    __syncthreads();
    for (int idx = tid; idx < G * D; idx += T::THREADS) {
        const int h = idx / D, d = idx % D;
        float M = -INFINITY;
#pragma unroll
        for (int v = 0; v < T::NW; ++v) M = fmaxf(M, red_m[v][h]);
        // A split whose every token sits on an out-of-range page has no valid
        // token in any wave: M stays -inf, and subtracting it would give
        // 2^(-inf + inf) = NaN.  Such a split yields o = 0, l = 0, m = -inf,
        // which the reduce weighs 0.
        const float Mu = M == -INFINITY ? 0.f : M;
        float L = 0.f, o = 0.f;
#pragma unroll
        for (int v = 0; v < T::NW; ++v) {
            const float wv = exp2_fast(red_m[v][h] - Mu);  // waves without tokens: 2^-inf = 0
            L += red_l[v][h] * wv;
            o += red_acc[v][h][d] * wv;
        }
        o = L > 0.f ? o / L : 0.f;
        const size_t row = (size_t)b * hq + kvh * G + h;
        if (num_splits == 1) {
            out[row * D + d] = (f16)o;
        } else {
            o_part[(row * num_splits + split) * D + d] = o;
            if (d == 0) {
                m_part[row * num_splits + split] = M;
                l_part[row * num_splits + split] = L;
            }
        }
    }
}

// LSE merge of the split partials (paged_decode.cu:204-215): one 256-thread
// workgroup per (sequence, query head) row; ns = ceil(ctx/P) partials are
// merged, with ctx clamped to the table row's capacity max_tok exactly as the
// decode kernel clamps it (a split starting past max_tok writes no partial),
// and ns clamped to the number of launched splits.  Partials with l = 0 (no
// readable token in the split) carry no weight; a row with no weight at all
// is written as zeros.  Every partial is read by
// an independent load (no serial chain over splits): pass 1 takes the block
// max of m; pass 2 has D/4 threads per partial row, each with a float4 of o,
// and 256/(D/4) partial rows in flight per step; the groups are summed in LDS.
template <int D>
__global__ void __launch_bounds__(256)
paged_reduce_kernel(const float* __restrict__ o_part, const float* __restrict__ m_part,
                    const float* __restrict__ l_part, const int* __restrict__ ctx_lens,
                    f16* __restrict__ out, int hq, int partition, int num_splits, int max_tok) {
    constexpr int THREADS = 256, TPR = D / 4, GROUPS = THREADS / TPR;
    __shared__ float red_max[THREADS / kWave];
    __shared__ f32x4 red_acc[GROUPS][TPR];
    __shared__ float red_den[GROUPS];
    const size_t row = blockIdx.x;
    const int b = (int)(row / hq);
    const int ctx = min(ctx_lens[b], max_tok);
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    int ns = ctx > 0 ? (int)(((long long)ctx + partition - 1) / partition) : 0;
    ns = min(ns, num_splits);
    const float* mp = m_part + row * num_splits;
    const float* lp = l_part + row * num_splits;
    const f32x4* op = reinterpret_cast<const f32x4*>(o_part + row * num_splits * D);

    float M = -INFINITY;
    for (int s = tid; s < ns; s += THREADS) M = fmaxf(M, mp[s]);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) M = fmaxf(M, __shfl_xor(M, off, kWave));
    if (lane == 0) red_max[w] = M;
    __syncthreads();
    M = fmaxf(fmaxf(red_max[0], red_max[1]), fmaxf(red_max[2], red_max[3]));
    if (M == -INFINITY) M = 0.f;  // every partial empty: all weights are 0 below

    const int g = tid / TPR, j = tid % TPR;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    float den = 0.f;
#pragma unroll 4
    for (int s = g; s < ns; s += GROUPS) {
        const float ls = lp[s];
        const float wgt = ls > 0.f ? ls * exp2_fast(mp[s] - M) : 0.f;
        acc += wgt * op[(size_t)s * TPR + j];
        den += wgt;
    }
    red_acc[g][j] = acc;
    if (j == 0) red_den[g] = den;
    __syncthreads();
    if (tid < TPR) {
        f32x4 sum = red_acc[0][tid];
        float dsum = red_den[0];
#pragma unroll
        for (int k = 1; k < GROUPS; ++k) {
            sum += red_acc[k][tid];
            dsum += red_den[k];
        }
        const float inv = dsum > 0.f ? 1.f / dsum : 0.f;
        f16* dst = out + row * D + tid * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[i] = (f16)(sum[i] * inv);
    }
}

template <int D, int G>
static hipError_t launch_decode(const DecodeArgs& a) {
    using T = DecodeTile<D, G>;
    int bs_shift = -1;
    for (int s = 0; s < 31; ++s)
        if ((int64_t(1) << s) == a.bs) bs_shift = s;
    const hipStream_t stream = (hipStream_t)a.stream;
    dim3 grid((unsigned)a.hkv, (unsigned)a.num_splits, (unsigned)a.batch);
    hipLaunchKernelGGL((paged_decode_kernel<D, G>), grid, dim3(T::THREADS), 0, stream, (const f16*)a.q,
                       (const f16*)a.k_cache, (const f16*)a.v_cache, a.block_tables, a.context_lens,
                       (f16*)a.out, a.o_part, a.m_part, a.l_part, (int)a.hkv, (int)a.bs, bs_shift,
                       (int)a.max_blocks, (int)a.num_blocks, (int)a.partition, (int)a.num_splits, a.sl2);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.num_splits == 1) return e;
    hipLaunchKernelGGL((paged_reduce_kernel<D>), dim3((unsigned)(a.batch * a.hq)), dim3(256), 0, stream,
                       a.o_part, a.m_part, a.l_part, a.context_lens, (f16*)a.out, (int)a.hq,
                       (int)a.partition, (int)a.num_splits, (int)(a.max_blocks * a.bs));
    return hipGetLastError();
}

// Split partials of ak_paged_decode_noalloc: one static array per GPU, held
// until the process ends, so that callers that cannot allocate (graph capture,
// tight serving loops) need no workspace.  Every call on a GPU shares that
// GPU's array; calls that overlap on one GPU race.  Nothing in it has to start
// at zero: the reduce reads only partials the same call's decode kernel wrote.
static __device__ __align__(256) float scratch[kDecodeScratchBytes / sizeof(float)];

// Device address of this GPU's scratch array.  In host code `scratch` names a
// host-side stand-in, never the device memory: the address comes from
// hipGetSymbolAddress, called once per device with that device current, and
// only that pointer is handed to kernels.
hipError_t decode_scratch(void** ptr) {
    constexpr int kMaxDevices = 64;
    static std::mutex mu;
    static void* addr[kMaxDevices] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        addr[dev] = p;
    }
    *ptr = addr[dev];
    return hipSuccess;
}

hipError_t decode_launch(const DecodeArgs& a) {
    const int64_t G = a.hq / a.hkv;
#define AK_DECODE(DD, GG) \
    if (a.d == DD && G == GG) return launch_decode<DD, GG>(a);
    AK_DECODE(64, 1) AK_DECODE(64, 2) AK_DECODE(64, 4) AK_DECODE(64, 8)
    AK_DECODE(128, 1) AK_DECODE(128, 2) AK_DECODE(128, 4) AK_DECODE(128, 8)
#undef AK_DECODE
    return hipErrorInvalidValue;
}

}  // namespace ak
