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
// The kernels are built for HBM bandwidth:
//   * in the dot-product kernels a token row of one page (D*2 contiguous
//     bytes) is covered by D/8 lanes (a lane group) with one 16-byte load each,
//     so one wave-wide load reads 4 (D=128) or 8 (D=64) tokens = 1 KB;
//   * their dot products are v_dot2_f32_f16 on the raw fp16 q and k, scaled by
//     scale*log2(e) in fp32 afterwards;
//   * with one query head per kv head (paged_decode_kernel) a D=128 lane keeps
//     16 K loads and 16 V loads in flight, a D=64 lane 4 and 4; each lane
//     group reduces its dot products with a DPP tree and runs its own online
//     softmax over the tokens it loads;
//   * with two or four heads per kv head (paged_decode_gqa_kernel, below)
//     the arithmetic per byte grows G-fold, and the lane groups share the
//     reduction, the exponentials and P V out by a butterfly (see there);
//   * with eight (paged_decode_gqa_mfma_kernel) both products run on the
//     matrix cores, 16x16x32 MFMAs over page pairs, with the K and V loads laid
//     out as the MFMA operands (see there);
//   * the lane groups of a wave and the waves of a workgroup are merged once,
//     at the end, by the same LSE rule.
#include "attn_kernels.hpp"
#include "wave.hpp"

#include <type_traits>

namespace ak {

// Agent-coherent (sc1) loads and stores of split partials: relaxed atomics at
// agent scope reach the device-wide coherence point without the whole-cache
// writeback and invalidate that release/acquire fences cost on gfx950.
__device__ __forceinline__ void coherent_store(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float coherent_load(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ f32x4 coherent_load4(const float* p) {  // 16-byte aligned
    const uint64_t a = __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t b = __hip_atomic_load(reinterpret_cast<const uint64_t*>(p) + 1, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
    const f32x2 x = __builtin_bit_cast(f32x2, a), y = __builtin_bit_cast(f32x2, b);
    return f32x4{x[0], x[1], y[0], y[1]};
}

// Merge of the ns split partials of one (sequence, kv head) into its G output
// rows row0 .. row0 + G - 1, by one workgroup: the LSE rule of the reduce
// kernel below (paged_decode.cu:204-215), M = max m_s, w_s = l_s 2^(m_s - M),
// O = sum w_s o_s / sum w_s, with partials of l = 0 weighted 0.  A thread owns
// 4 head dims of one row (a unit) and every SG-th split; its loads for NB of
// them at a time are issued together and merged by a running maximum, and the
// SG split groups of a unit are merged through LDS.
template <int D, int G, int THREADS>
__device__ __forceinline__ void merge_splits(const float* o_part, const float* m_part, const float* l_part,
                                             f16* out, size_t row0, int num_splits, int ns, int tid) {
    // NB: loads per batch, enough for the most splits merged here in one batch,
    // but no more than the kernel's main loop has registers for (8, or 16 for
    // the four- and eight-head kernels)
    constexpr int UNITS = G * D / 4, SG = THREADS / UNITS;
    constexpr int NB_CAP = G >= 4 ? 16 : 8, NB_ALL = (int)((kFusedMaxSplits + SG - 1) / SG);
    constexpr int NB = NB_ALL < NB_CAP ? NB_ALL : NB_CAP;
    static_assert(SG >= 1 && SG * UNITS == THREADS, "units tile the workgroup");
    __shared__ float mg_m[THREADS], mg_l[THREADS];
    __shared__ f32x4 mg_o[THREADS];
    const int u = tid % UNITS, sg = tid / UNITS;
    const int h = u / (D / 4), d4 = u % (D / 4);
    const size_t row = row0 + h;
    const float* mp = m_part + row * num_splits;
    const float* lp = l_part + row * num_splits;
    const float* op = o_part + row * num_splits * D + d4 * 4;
    float M = -INFINITY, L = 0.f;
    f32x4 O = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = sg; s0 < ns; s0 += SG * NB) {
        float ms[NB], ls[NB];
        f32x4 os[NB];
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int s = s0 + j * SG;
            const bool in = s < ns;
            ms[j] = in ? coherent_load(mp + s) : -INFINITY;
            ls[j] = in ? coherent_load(lp + s) : 0.f;
            os[j] = in ? coherent_load4(op + (size_t)s * D) : f32x4{0.f, 0.f, 0.f, 0.f};
        }
        float mb = M;
#pragma unroll
        for (int j = 0; j < NB; ++j) mb = fmaxf(mb, ls[j] > 0.f ? ms[j] : -INFINITY);
        if (mb == -INFINITY) continue;  // no weighted partial yet
        const float a = exp2_fast(M - mb);  // 0 while M = -inf
        L *= a;
        O *= a;
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const float wgt = ls[j] > 0.f ? ls[j] * exp2_fast(ms[j] - mb) : 0.f;
            L += wgt;
            O += wgt * os[j];
        }
        M = mb;
    }
    if constexpr (SG > 1) {
        mg_m[tid] = M;
        mg_l[tid] = L;
        mg_o[tid] = O;
        __syncthreads();
        if (sg == 0) {
            float Mx = M;
#pragma unroll
            for (int k = 1; k < SG; ++k) Mx = fmaxf(Mx, mg_m[k * UNITS + u]);
            const float Mu = Mx == -INFINITY ? 0.f : Mx;
            L = 0.f;
            O = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k = 0; k < SG; ++k) {
                const float wgt = exp2_fast(mg_m[k * UNITS + u] - Mu);  // groups without weight: 2^-inf = 0
                L += mg_l[k * UNITS + u] * wgt;
                O += wgt * mg_o[k * UNITS + u];
            }
        }
    }
    if (sg == 0) {
        const float inv = L > 0.f ? 1.f / L : 0.f;  // a row with no weight at all is written as zeros
        f16* dst = out + row * D + d4 * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[i] = (f16)(O[i] * inv);
    }
}

// Split epilogue of both decode kernels.  red_acc / red_m / red_l hold the
// workgroup's per-wave (acc, m, l) of the kv head's G query heads (m in the
// log2 domain; the stored l is L * lscale).  The waves are merged by the LSE
// rule, then:
//   * one split in the launch (num_splits == 1), or (fused) one split with
//     tokens for this sequence: the fp16 output rows;
//   * reduce path (counters == null): the split's partial (normalised o, m, l)
//     for the reduce kernel;
//   * fused path: the partial with agent-coherent stores, then, once they are
//     complete, the (sequence, kv head) counter.  The split that takes it to
//     ns - 1 is the last to arrive: every other partial is complete, so it
//     merges all ns of them into the output and resets the counter to zero
//     for the next call.  No workgroup waits for another.
template <int D, int G, int NW>
__device__ __forceinline__ void split_epilogue(const float (&red_acc)[NW][G][D], const float (&red_m)[NW][G],
                                               const float (&red_l)[NW][G], float lscale, f16* __restrict__ out,
                                               float* __restrict__ o_part, float* __restrict__ m_part,
                                               float* __restrict__ l_part, int32_t* __restrict__ counters, int b,
                                               int kvh, int hkv, int split, int num_splits, int ns, int tid) {
    constexpr int THREADS = NW * kWave;
    __shared__ int last;
    const int hq = hkv * G;
    const bool direct = num_splits == 1 || (counters && ns == 1);
    const bool fused = counters && !direct;
    for (int idx = tid; idx < G * D; idx += THREADS) {
        const int h = idx / D, d = idx % D;
        float M = -INFINITY;
#pragma unroll
        for (int v = 0; v < NW; ++v) M = fmaxf(M, red_m[v][h]);
        // A split whose every token sits on an out-of-range page has no valid
        // token in any wave: M stays -inf, and subtracting it would give
        // 2^(-inf + inf) = NaN.  Such a split yields o = 0, l = 0, m = -inf,
        // which the merge weighs 0.
        const float Mu = M == -INFINITY ? 0.f : M;
        float L = 0.f, o = 0.f;
#pragma unroll
        for (int v = 0; v < NW; ++v) {
            const float wv = exp2_fast(red_m[v][h] - Mu);  // waves without tokens: 2^-inf = 0
            L += red_l[v][h] * wv;
            o += red_acc[v][h][d] * wv;
        }
        o = L > 0.f ? o / L : 0.f;
        const size_t row = (size_t)b * hq + kvh * G + h;
        const size_t slot = row * num_splits + split;
        if (direct) {
            out[row * D + d] = (f16)o;
        } else if (!fused) {
            o_part[slot * D + d] = o;
            if (d == 0) {
                m_part[slot] = M;
                l_part[slot] = L * lscale;
            }
        } else {
            coherent_store(o_part + slot * D + d, o);
            if (d == 0) {
                coherent_store(m_part + slot, M);
                coherent_store(l_part + slot, L * lscale);
            }
        }
    }
    if (!fused) return;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's partial stores are complete
    __syncthreads();
    int32_t* cnt = counters + (size_t)b * hkv + kvh;
    if (tid == 0) last = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == ns - 1;
    __syncthreads();
    if (!last) return;
    merge_splits<D, G, THREADS>(o_part, m_part, l_part, out, (size_t)b * hq + (size_t)kvh * G, num_splits, ns, tid);
    if (tid == 0) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Splits of sequence b that hold tokens (the reduce kernel reads as many).
__device__ __forceinline__ int splits_with_tokens(int ctx, int partition, int num_splits) {
    const int ns = ctx > 0 ? (int)(((long long)ctx + partition - 1) / partition) : 0;
    return min(ns, num_splits);
}

// One query head per kv head (the reference's decode configurations).
template <int D>
struct DecodeTile {
    static constexpr int NW = D == 128 ? 4 : 8;  // waves per workgroup
    static constexpr int THREADS = NW * kWave;   // 256 or 512
    static constexpr int LPT = D / 8;            // lanes per token row
    static constexpr int TPL = kWave / LPT;      // tokens per wave-wide load
    static constexpr int U = D == 128 ? 16 : 4;  // loads in flight per lane, per cache
    static constexpr int TOK = U * TPL;          // tokens per wave iteration
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

template <int D>
__global__ void __launch_bounds__((DecodeTile<D>::THREADS))
paged_decode_kernel(const f16* __restrict__ q, const f16* __restrict__ kc, const f16* __restrict__ vc,
                    const int* __restrict__ block_tables, const int* __restrict__ ctx_lens,
                    f16* __restrict__ out, float* __restrict__ o_part, float* __restrict__ m_part,
                    float* __restrict__ l_part, int32_t* __restrict__ counters, int hkv, int bs, int bs_shift,
                    int max_blocks, int num_blocks, int partition, int num_splits, float sl2) {
    using T = DecodeTile<D>;
    constexpr int G = 1;
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
    // The context length first: a workgroup past a short context (most of a
    // skewed batch's grid) exits after that one scalar load, without the U
    // vector loads of its page ids, which would hold its slot for a vector
    // round trip (measured: a skewed batch's step 12% faster, cfg4 and cfg5
    // unchanged).  The page ids and q follow the check.
    const int ctx_raw = ctx_lens[b];
    const int stride = T::NW * T::TOK;
    int pg[T::U];

    const int ctx = min(ctx_raw, max_tok);
    if (start >= ctx) {  // whole workgroup: this split is past the context
        // A sequence with no context (outside the >= 1 contract) gets a zero row,
        // as the reduce gives it when there are several splits.
        if (num_splits == 1 || (counters && split == 0))
            for (int idx = tid; idx < D; idx += T::THREADS) out[((size_t)b * hq + kvh) * D + idx] = (f16)0.f;
        return;
    }
    const int end = min(ctx, start + partition);
    load_pages(start + w * T::TOK, end, pg);
    // q of this head, raw fp16 (scaled after the dot product)
    const f16x8 qv = *reinterpret_cast<const f16x8*>(q + ((size_t)b * hq + kvh) * D + li * 8);

    float m[G] = {-INFINITY}, l[G] = {0.f}, acc[G][8] = {};
    const size_t page_stride = (size_t)hkv * bs * D;
    const size_t head_off = (size_t)kvh * bs * D + li * 8;

    // One chunk: token t0 + u*TPL + gi in kr[u]/vr[u]; tokens with !valid[u]
    // drop out.  Each group of D/8 lanes reduces its dot products with a DPP
    // tree and runs its own online softmax.
    for (int t0 = start + w * T::TOK; t0 < end; t0 += stride) {
        f16x8 kr[T::U], vr[T::U];
        bool valid[T::U];
#pragma unroll
        for (int u = 0; u < T::U; ++u) {
            const int t = t0 + u * T::TPL + gi;
            const int po = bs_shift >= 0 ? (t & (bs - 1)) : (t % bs);
            const bool ok = t < end && (unsigned)pg[u] < (unsigned)num_blocks;  // bad page ids are never read
            const size_t off = (size_t)(ok ? pg[u] : 0) * page_stride + head_off + (size_t)po * D;
            valid[u] = ok;
            // K/V are streamed once: non-temporal loads keep them out of the caches' way.
            kr[u] = ok ? __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(kc + off)) : f16x8{};
            vr[u] = ok ? __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(vc + off)) : f16x8{};
        }
        load_pages(t0 + stride, end, pg);
        float sc[T::U];
        float mx = -INFINITY;
#pragma unroll
        for (int u = 0; u < T::U; ++u) {
            const float dsum = group_sum<T::LPT>(dot8(qv, kr[u]));
            sc[u] = valid[u] ? dsum * sl2 : -INFINITY;
            mx = fmaxf(mx, sc[u]);
        }
        const float m_new = fmaxf(m[0], mx);
        const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
        const float alpha = exp2_fast(m[0] - m_use);
        float psum = 0.f;
#pragma unroll
        for (int u = 0; u < T::U; ++u) {
            sc[u] = exp2_fast(sc[u] - m_use);
            psum += sc[u];
        }
        l[0] = l[0] * alpha + psum;
        m[0] = m_new;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float a = acc[0][i] * alpha;
#pragma unroll
            for (int u = 0; u < T::U; ++u) a = fmaf(sc[u], (float)vr[u][i], a);
            acc[0][i] = a;
        }
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
    split_epilogue<D, G, T::NW>(red_acc, red_m, red_l, 1.f, out, o_part, m_part, l_part, counters, b, kvh, hkv,
                                split, num_splits, splits_with_tokens(ctx, partition, num_splits), tid);
}

// ---------------------------------------------------------------------------
// Grouped-query decode on dot products: G = 2 or 4 query heads per kv head
// (eight go to the matrix-core kernel further below).
//
// The kernel above, given head groups, runs out of VALU issue before HBM: each
// (head, token) dot product is reduced over its D/8 lanes by a DPP tree, every
// lane of the group then exponentiates the same score, and P V converts V to
// fp32 and spends one FMA per (head, token, dim).  This kernel reads the cache
// exactly as that one does (D/8 lanes per token row, one 16-byte K and V load
// per lane per token, scalar page ids, one 16-token page per wave chunk) and
// reorganises the arithmetic of a chunk:
//   * reduce-scatter: a lane's G*U partial dot products (8 dims each) are
//     summed across its lane group by a butterfly that halves the list at
//     every lane bit: the lane keeps one half and adds the partner's copy of it
//     (DPP), so the G*U sums cost about G*U DPP adds instead of log2(D/8) * G*U,
//     and every lane ends with the full scores of one head and two tokens.  So
//     that each step is one DPP add with no selects, a lane holds its q heads
//     and its token slots in a lane-dependent order: register r holds value
//     r ^ f(lane), where f toggles the bit resolved at each butterfly stage;
//   * every score is exponentiated once, against a per-wave, per-head reference
//     max m that moves only when a score exceeds it by more than 8 (base 2), so
//     that P = 2^(s - m + 7) stays below 2^15 and is exact enough in fp16 (the
//     2^7 keeps small weights out of fp16's subnormal range; it cancels in o/l);
//   * P goes to fp16, two tokens per register, and is all-gathered across the
//     lane group by the inverse butterfly; P V is v_dot2_f32_f16 over token
//     pairs (V repacked pairwise with v_perm), into fp32 accumulators; l sums
//     the same fp16 P values, so rounding P only perturbs the weights.
// Lanes of one group hold the same head order, so the groups of a wave merge
// register by register at the end (lane permutes, no LDS), and the waves of the
// workgroup through LDS as above.

// Issue priority from a wave's progress through its split: 3 over the first
// quarter of its tokens, falling to 0 over the last, so that a wave running
// ahead of the others on its SIMD yields issue slots to those behind it.  Of
// two workgroups sharing a CU, the hardware otherwise favours the older one:
// measured per workgroup (B=8 x 8192 tokens, G=8, 512 workgroups, two per CU),
// in every CU the older finished its loop 9.5-11.5 us before the younger,
// which then streamed alone.  Only for launches whose workgroups are all
// resident at once (gqa_balance): when some wait for a slot, letting the
// oldest finish first frees slots sooner (one and a third rounds: -7% to -10%).
__device__ __forceinline__ void progress_priority(int done, int total) {
    const int q = (done * 4) / max(1, total);
    if (q <= 0) __builtin_amdgcn_s_setprio(3);
    else if (q == 1) __builtin_amdgcn_s_setprio(2);
    else if (q == 2) __builtin_amdgcn_s_setprio(1);
    else __builtin_amdgcn_s_setprio(0);
}

template <int D, int G, int NW_>
struct GqaTile {
    static constexpr int NW = NW_;               // waves per workgroup
    static constexpr int THREADS = NW * kWave;
    static constexpr int LPT = D / 8;            // lanes per token row (a lane group)
    static constexpr int TPL = kWave / LPT;      // tokens per wave-wide load
    static constexpr int U = 16 / TPL;           // K (and V) loads per lane per chunk
    static constexpr int TOK = U * TPL;          // tokens per wave chunk: one 16-token page
    static constexpr int LB = D == 128 ? 4 : 3;  // log2(LPT): butterfly stages of a lane group
    static constexpr int N = G * U;              // partial dot products per lane per chunk
    static constexpr int LOGN = G * U == 4 ? 2 : G * U == 8 ? 3 : G * U == 16 ? 4 : 5;
    static constexpr int S = LB < LOGN - 1 ? LB : LOGN - 1;  // stages that scatter
    static constexpr int HB = G == 2 ? 1 : G == 4 ? 2 : 3;   // head bits of a value index
    static_assert(D == 128 || D == 64, "head dim");
    static_assert(G == 2 || G == 4, "head group");
    static_assert((N >> S) == 2, "two scores per lane after the scatter");
    static_assert(S >= HB, "the scatter resolves every head bit");
};

// The butterfly's partner at stage s is lane ^ mask(s) inside the lane group.
// 16-lane groups: masks 8, 7, 2, 1 (DPP row_ror:8, row_half_mirror, quad_perm
// [2,3,0,1], quad_perm [1,0,3,2]); 8-lane groups: 7, 2, 1.  They are linearly
// independent over GF(2), so every lane has unique coordinates c_s in them.
template <int LB>
__device__ constexpr int bfly_dpp(int s) {
    constexpr int k16[4] = {0x128, kDppHalfMirror, kDppXor2, kDppXor1};
    return k16[s + 4 - LB];
}
template <int LB>
__device__ __forceinline__ int bfly_coord(int li, int s) {
    // li = XOR_s c_s * mask(s) with masks (8,) 7, 2, 1: bit 3 only in 8, bit 2
    // only in 7, bit 1 in 7 and 2, bit 0 in 7 and 1.
    const int l2 = (li >> 2) & 1;
    const int c[4] = {(li >> 3) & 1, l2, ((li >> 1) & 1) ^ l2, (li & 1) ^ l2};
    return c[s + 4 - LB];
}

// Lane mask, inside a lane group, from a lane holding head h to a lane that
// holds head h ^ a: the masks of the stages that resolve the head bits set in a.
template <int LB, int N, int G>
__device__ constexpr int head_lane_mask(int a) {
    constexpr int k16[4] = {8, 7, 2, 1};
    int m = 0;
    for (int s = 0; s < LB && (N >> (s + 1)) >= 2; ++s) {
        const int bit = N >> (s + 1);  // value-index bit resolved at stage s
        if (bit < 2 * G && (a & (bit >> 1))) m ^= k16[s + 4 - LB];
    }
    return m;
}

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t x) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, 0xF, 0xF, false);
}

template <int I, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (I < E) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, E>(f);
    }
}

// x combined by op with the value of lane l ^ MASK (MASK = 8, 16 or 32): DPP
// row_ror:8, or v_permlane16/32_swap on two copies of x (inline asm, as in the
// prefill kernel: the builtin with identical inputs kept one register).  The
// s_nop covers the VALU-write -> permlane-read hazard.
template <int MASK, class Op>
__device__ __forceinline__ float xor_combine(float x, Op op) {
    static_assert(MASK == 8 || MASK == 16 || MASK == 32, "lane mask");
    if constexpr (MASK == 8) {
        return op(x, dpp<0x128>(x));
    } else {
        float a = x, b = x;
        if constexpr (MASK == 16)
            asm volatile("s_nop 2\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
        else
            asm volatile("s_nop 2\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
        return op(a, b);
    }
}
// x combined over the TPL lane groups of the wave (lanes l ^ LPT, l ^ 2 LPT, ...).
template <int LPT, class Op>
__device__ __forceinline__ float across_groups(float x, Op op) {
    if constexpr (LPT == 8) x = xor_combine<8>(x, op);
    x = xor_combine<16>(x, op);
    return xor_combine<32>(x, op);
}

template <int D, int G, int NW, bool PIPE>
__global__ void __launch_bounds__((GqaTile<D, G, NW>::THREADS))
paged_decode_gqa_kernel(const f16* __restrict__ q, const f16* __restrict__ kc, const f16* __restrict__ vc,
                        const int* __restrict__ block_tables, const int* __restrict__ ctx_lens,
                        f16* __restrict__ out, float* __restrict__ o_part, float* __restrict__ m_part,
                        float* __restrict__ l_part, int32_t* __restrict__ counters, int hkv, int bs,
                        int bs_shift, int max_blocks, int num_blocks, int partition, int num_splits, float sl2,
                        int balance) {
    using T = GqaTile<D, G, NW>;
    constexpr int U = T::U, N = T::N, S = T::S, LB = T::LB;
    // P = 2^(s - m + kPShift): the largest P the fast path accepts is 2^kPMax.
    constexpr float kPShift = 7.f, kPMax = 32768.f;
    __shared__ float red_acc[T::NW][G][D];
    __shared__ float red_m[T::NW][G], red_l[T::NW][G];

    const int kvh = blockIdx.x, split = blockIdx.y, b = blockIdx.z;
    const int hq = hkv * G;
    const int start = split * partition;
    const int tid = threadIdx.x, lane = tid & 63, w = uniform(tid >> 6);
    const int gi = lane / T::LPT, li = lane % T::LPT;
    const int* bt = block_tables + (size_t)b * max_blocks;
    const int max_tok = max_blocks * bs;

    // Value index of a partial dot product: j = (slot >> 1) * 2G + head * 2 +
    // (slot & 1).  Stage s of the butterfly resolves bit N >> (s + 1), top
    // first, so a slot's high bit (if U = 4) is resolved by the first stage,
    // whose partner mask 8 is the cache-line bit of the lane (lanes 0-7 and
    // 8-15 read the two 128-byte halves of a 256-byte row): the 8 lanes of a
    // cache line always read the same token row, and every load instruction
    // reads whole lines.  This lane's offset f into the value index:
    int f = 0;
#pragma unroll
    for (int s = 0; s < S; ++s) f ^= bfly_coord<LB>(li, s) ? (N >> (s + 1)) : 0;
    constexpr int LG = G == 2 ? 1 : G == 4 ? 2 : 3;
    auto head_of = [](int j) { return (j >> 1) & (G - 1); };
    auto slot_of = [](int j) { return ((j >> (1 + LG)) << 1) | (j & 1); };
    const int fh = head_of(f), fu = slot_of(f);

    // Page ids of this lane's token slots (slot u holds token t0 + (u ^ fu) *
    // TPL + gi) below lim, -1 elsewhere; loaded one chunk ahead.
    auto load_pages = [&](int t0, int lim, int (&pg)[U]) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int t = t0 + (u ^ fu) * T::TPL + gi;
            const int pi = bs_shift >= 0 ? (t >> bs_shift) : (t / bs);
            pg[u] = t < lim ? bt[pi] : -1;
        }
    };
    const int ctx_raw = ctx_lens[b];
    const int stride = T::NW * T::TOK;
    int pg[U];
    const bool fast_bs = bs == T::TOK;

    const int ctx = min(ctx_raw, max_tok);
    if (start >= ctx) {
        if (num_splits == 1 || (counters && split == 0))
            for (int idx = tid; idx < G * D; idx += T::THREADS)
                out[((size_t)b * hq + kvh * G + idx / D) * D + idx % D] = (f16)0.f;
        return;
    }
    const int end = min(ctx, start + partition);
    // The first page id and q after the context check: a workgroup past a
    // short context exits after its one scalar load (the check's wait would
    // also wait for a page id loaded beside it; a skewed batch's step 3%
    // faster, uniform batches unchanged).
    int spg = 0;
    if (fast_bs && start + w * T::TOK + T::TOK <= min(start + partition, max_tok))
        spg = bt[uniform((start + w * T::TOK) >> 4)];
    f16x8 qv[G];  // register a: query head a ^ fh
#pragma unroll
    for (int a = 0; a < G; ++a)
        qv[a] = *reinterpret_cast<const f16x8*>(q + ((size_t)b * hq + kvh * G + (a ^ fh)) * D + li * 8);

    // Per-wave reference max of this lane's head (fh), this lane's share of l
    // for that head, and the accumulators (register a: head a ^ fh, dims
    // li*8 .. li*8+7, this lane group's tokens).
    float m_own = -INFINITY, l_own = 0.f;
    float acc[G][8];
#pragma unroll
    for (int a = 0; a < G; ++a)
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[a][i] = 0.f;
    const size_t page_stride = (size_t)hkv * bs * D;
    const size_t head_off = (size_t)kvh * bs * D + li * 8;

    // Scores of a chunk: the full dot products of head fh with this lane's own
    // slots 0 and 1 (after which the K registers are free).
    auto scores = [&](const f16x8 (&kr)[U], float (&xs)[2]) {
        // Partial dot products: x[r] = q(head head_of(r) ^ fh) . k(slot slot_of(r) ^ fu), 8 dims.
        float x[N];
#pragma unroll
        for (int r = 0; r < N; ++r) x[r] = dot8(qv[head_of(r)], kr[slot_of(r)]);
        // Reduce-scatter over the lane group; the remaining stages (lane bits
        // left after every head bit and every slot bit but the lowest is
        // resolved) sum the two remaining values in full.
        static_for<0, S>([&](auto st) {
            constexpr int s = decltype(st)::value, half = (N >> s) / 2;
#pragma unroll
            for (int r = 0; r < half; ++r) x[r] += dpp<bfly_dpp<LB>(s)>(x[r + half]);
        });
        static_for<S, LB>([&](auto st) {
            constexpr int s = decltype(st)::value;
            x[0] += dpp<bfly_dpp<LB>(s)>(x[0]);
            x[1] += dpp<bfly_dpp<LB>(s)>(x[1]);
        });
        xs[0] = x[0];
        xs[1] = x[1];
    };
    // Online softmax and P V of a chunk, from its scores and its V registers;
    // tokens with !valid[r] (this lane's slots 0 and 1) drop out when MASKED.
    auto finish = [&](const float (&x)[2], const f16x8 (&vr)[U], const bool (&valid)[U], auto masked) {
        constexpr bool MASKED = decltype(masked)::value;
        float p[2];
        float bias = kPShift - m_own;
#pragma unroll
        for (int r = 0; r < 2; ++r)
            p[r] = exp2_fast(!MASKED || valid[r] ? fmaf(x[r], sl2, bias) : -INFINITY);
        const bool ok = p[0] <= kPMax && p[1] <= kPMax;  // false for inf and NaN
        if (__builtin_amdgcn_ballot_w64(!ok)) {
            // Move the reference max of every head of the wave to its running
            // max (first chunk: m = -inf; later: a score above m + 8).
            float mx = -INFINITY;
#pragma unroll
            for (int r = 0; r < 2; ++r) mx = fmaxf(mx, !MASKED || valid[r] ? x[r] * sl2 : -INFINITY);
            auto fmax2 = [](float u, float v) { return fmaxf(u, v); };
            static_for<0, LB>([&](auto st) {
                constexpr int s = decltype(st)::value;
                if constexpr (s >= S || (N >> (s + 1)) >= 2 * G) mx = fmaxf(mx, dpp<bfly_dpp<LB>(s)>(mx));
            });
            mx = across_groups<T::LPT>(mx, fmax2);
            const float m_new = fmaxf(m_own, mx);
            const float m_use = m_new == -INFINITY ? 0.f : m_new;
            const float alpha = exp2_fast(m_own - m_use);  // 0 while m was -inf
            l_own *= alpha;
            m_own = m_new;
            // Every lane of head fh holds the same alpha; the accumulators of
            // head a ^ fh take theirs from the lane of the group that holds
            // that head (a lane shuffle: no memory, nothing to order).
            static_for<0, G>([&](auto ai) {
                constexpr int a = decltype(ai)::value;
                const float al = a == 0 ? alpha : __shfl_xor(alpha, head_lane_mask<LB, N, G>(a), kWave);
#pragma unroll
                for (int i = 0; i < 8; ++i) acc[a][i] *= al;
            });
            bias = kPShift - m_use;
#pragma unroll
            for (int r = 0; r < 2; ++r)
                p[r] = exp2_fast(!MASKED || valid[r] ? fmaf(x[r], sl2, bias) : -INFINITY);
        }
        const f16x2 pp = {(f16)p[0], (f16)p[1]};
        l_own = __builtin_amdgcn_fdot2(pp, f16x2{(f16)1.f, (f16)1.f}, l_own, false);
        // All-gather P over the lane group (the scatter's stages in reverse):
        // register k = pr * G + a then holds the pair of head a ^ fh, slots
        // (2 pr) ^ fu and +1, i.e. the tokens in V registers 2 pr and 2 pr + 1.
        uint32_t P[N / 2];
        P[0] = __builtin_bit_cast(uint32_t, pp);
        static_for<0, S>([&](auto st) {
            constexpr int s = S - 1 - decltype(st)::value, m = N >> (s + 2);
#pragma unroll
            for (int k = 0; k < m; ++k) P[k + m] = dpp_u32<bfly_dpp<LB>(s)>(P[k]);
        });
        // P V over token pairs: vp[i] = (v(slot 2pr)[i], v(slot 2pr+1)[i]).
#pragma unroll
        for (int pr = 0; pr < U / 2; ++pr) {
            const auto lo = __builtin_bit_cast(u32x4, vr[2 * pr]);
            const auto hi = __builtin_bit_cast(u32x4, vr[2 * pr + 1]);
            f16x2 vp[8];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                vp[2 * k] = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(hi[k], lo[k], 0x05040100u));
                vp[2 * k + 1] = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(hi[k], lo[k], 0x07060302u));
            }
#pragma unroll
            for (int a = 0; a < G; ++a) {
                const f16x2 pa = __builtin_bit_cast(f16x2, P[pr * G + a]);
#pragma unroll
                for (int i = 0; i < 8; ++i) acc[a][i] = __builtin_amdgcn_fdot2(pa, vp[i], acc[a][i], false);
            }
        }
    };
    // Byte offset of slot u's 16 bytes inside a 16-token page of this kv head.
    uint32_t lane_off[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
        lane_off[u] = (uint32_t)(((size_t)kvh * T::TOK * D + ((u ^ fu) * T::TPL + gi) * D + li * 8) * sizeof(f16));

    // Whole-page chunks: the chunk's page id is one wave-uniform scalar load
    // (prefetched one chunk ahead) and every K/V load is page base + lane
    // offset.  The checked loop takes the rest: the context's tail, an
    // out-of-range page id, and every chunk when pages are not 16 tokens.
    int t0 = start + w * T::TOK;
    {
        auto load_kv = [&](const f16* cache, int pid, f16x8 (&r)[U]) {
            const char* base = reinterpret_cast<const char*>(cache) + (size_t)pid * page_stride * sizeof(f16);
#pragma unroll
            for (int u = 0; u < U; ++u)  // streamed once: non-temporal
                r[u] = __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(base + lane_off[u]));
        };
        const bool unused[U] = {};
        if constexpr (PIPE) {
            // Software-pipelined: chunk t0 + stride's K and V are issued before
            // chunk t0 is computed (page ids one chunk further ahead), in two
            // register sets that swap roles every chunk.  A step computes chunk
            // t0 and returns whether the next chunk was issued; when it was not
            // (tail, bad page id), t0 is that chunk and the checked loop takes it.
            auto step = [&](const f16x8 (&kcur)[U], const f16x8 (&vcur)[U], f16x8 (&knext)[U],
                            f16x8 (&vnext)[U], int& spn) {
                const int tn = t0 + stride;
                const bool issued = tn + T::TOK <= end && (unsigned)spn < (unsigned)num_blocks;
                if (issued) {
                    load_kv(kc, spn, knext);
                    load_kv(vc, spn, vnext);
                    const int tnn = tn + stride;
                    if (tnn + T::TOK <= end) spn = bt[uniform(tnn >> 4)];
                }
                if (balance) progress_priority(t0 - start, end - start);
                float x[2];
                scores(kcur, x);
                finish(x, vcur, unused, std::false_type{});
                t0 = tn;
                return issued;
            };
            if (fast_bs && t0 + T::TOK <= end && (unsigned)spg < (unsigned)num_blocks) {
                f16x8 ka[U], va[U], kb[U], vb[U];
                load_kv(kc, spg, ka);
                load_kv(vc, spg, va);
                int spn = -1;
                if (t0 + stride + T::TOK <= end) spn = bt[uniform((t0 + stride) >> 4)];
                while (step(ka, va, kb, vb, spn) && step(kb, vb, ka, va, spn)) {
                }
            }
        } else {
            while (fast_bs && t0 + T::TOK <= end && (unsigned)spg < (unsigned)num_blocks) {
                f16x8 kr[U], vr[U];
                load_kv(kc, spg, kr);
                load_kv(vc, spg, vr);
                const int tn = t0 + stride;
                if (tn + T::TOK <= end) spg = bt[uniform(tn >> 4)];
                if (balance) progress_priority(t0 - start, end - start);
                float x[2];
                scores(kr, x);
                finish(x, vr, unused, std::false_type{});
                t0 = tn;
            }
        }
    }
    __builtin_amdgcn_s_setprio(0);
    if (t0 < end) load_pages(t0, end, pg);
    for (; t0 < end; t0 += stride) {
        f16x8 kr[U], vr[U];
        bool valid[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int t = t0 + (u ^ fu) * T::TPL + gi;
            const int po = bs_shift >= 0 ? (t & (bs - 1)) : (t % bs);
            const bool ok = t < end && (unsigned)pg[u] < (unsigned)num_blocks;
            const size_t off = (size_t)(ok ? pg[u] : 0) * page_stride + head_off + (size_t)po * D;
            valid[u] = ok;
            kr[u] = ok ? __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(kc + off)) : f16x8{};
            vr[u] = ok ? __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(vc + off)) : f16x8{};
        }
        load_pages(t0 + stride, end, pg);
        float x[2];
        scores(kr, x);
        finish(x, vr, valid, std::true_type{});
    }

    // Merge the wave: l over the lanes of each head (the stages that resolved
    // slot bits; the plain stages hold copies), then everything over the lane
    // groups.  m is already per wave and head, so these are plain sums.
    auto add2 = [](float u, float v) { return u + v; };
    static_for<0, S>([&](auto st) {
        constexpr int s = decltype(st)::value;
        if constexpr ((N >> (s + 1)) >= 2 * G) l_own += dpp<bfly_dpp<LB>(s)>(l_own);
    });
    l_own = across_groups<T::LPT>(l_own, add2);
#pragma unroll
    for (int a = 0; a < G; ++a)
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[a][i] = across_groups<T::LPT>(acc[a][i], add2);
    if (gi == 0) {
#pragma unroll
        for (int a = 0; a < G; ++a)
#pragma unroll
            for (int i = 0; i < 8; ++i) red_acc[w][a ^ fh][li * 8 + i] = acc[a][i];
        red_m[w][fh] = m_own;
        red_l[w][fh] = l_own;
    }
    __syncthreads();
    // m in the log2 domain of the scores: the kPShift on P cancels in o and is
    // taken out of l here.
    split_epilogue<D, G, T::NW>(red_acc, red_m, red_l, 1.f / 128.f, out, o_part, m_part, l_part, counters, b, kvh,
                                hkv, split, num_splits, splits_with_tokens(ctx, partition, num_splits), tid);
}

// Eight query heads per kv head on the matrix cores
// (paged_decode_gqa_mfma_kernel).  A wave takes two 16-token pages per
// iteration and runs both products on v_mfma_f32_16x16x32_f16, the head group
// padded to the MFMA's 16 rows (rows G..15 hold zeros or values nobody reads):
//   * S^T = K Q^T per page: A = K (lane l: token l%16 of the page, head dims
//     32s + 8(l/16) .. +7 for step s < D/32, one 16-byte load each), B = Q^T
//     (lane l: query head l%16, the same dims, loaded once), so lane
//     (n = l%16, g = l/16) ends with the raw scores of head n, tokens
//     4g .. 4g+3 of the page;
//   * O += P V per page pair, k = 32 tokens: A = P (lane (n, g): head n, the
//     8 tokens 4g .. 4g+3 of both pages: exactly the scores the lane holds),
//     B = V, where column n stands for head dims DPL n + j in the j-th of
//     DPL = D/16 products: the lane loads its 8 tokens' DPL dims (16 or 8
//     bytes each; one load instruction reads 4 whole token rows) and regroups
//     them per dim with v_perm; accumulator j then holds heads 4g + r, dim
//     DPL n + j;
//   * softmax as in the dot-product kernel: one exponential per score against
//     a per-head reference max (the same in the head's four lanes) that moves
//     only when a score exceeds it by more than 8 (base 2), so that fp16
//     P = 2^(s - m + 7) stays below 2^15; l sums the fp16 P values.
// The VALU work per page is the V regrouping and the softmax, about 40
// instructions against about 300 for eight heads on dot products.  Measured
// on MI355X against the dot-product kernel at the default partition (calls
// back to back / after a 512 MiB flush): G = 8, B = 8 x 8192 tokens, D = 128
// +3% / +3%, D = 64 +5-8% / +4-8%; B = 1 x 1024 tokens +3% / +15%.  With
// two or four heads per kv head it is no faster (-5% to +1%: B = 1-4, 4096-
// 16384 tokens lose 4-5% back to back), so those keep the dot products.
template <int D, int G, int NW_>
struct GqaMfmaTile {
    static constexpr int NW = NW_;         // waves per workgroup
    static constexpr int THREADS = NW * kWave;
    static constexpr int KS = D / 32;      // S^T = K Q^T steps of 32 head dims
    static constexpr int DPL = D / 16;     // head dims of a V row per lane = P V products per page pair
    static constexpr int TOK = 32;         // tokens per wave iteration: two 16-token pages
    static_assert(D == 128 || D == 64, "head dim");
    static_assert(G >= 2 && G <= 16, "head group within the MFMA's 16 rows");
};

// At most 168 VGPRs (amdgpu_waves_per_eu(3)), so that three waves share a
// SIMD (the compiler otherwise moves the accumulators to AGPRs and holds 172
// registers, two waves); a 128-register bound spills at D = 128.
template <int D, int G, int NW>
__global__ void __launch_bounds__((GqaMfmaTile<D, G, NW>::THREADS)) __attribute__((amdgpu_waves_per_eu(3)))
paged_decode_gqa_mfma_kernel(const f16* __restrict__ q, const f16* __restrict__ kc, const f16* __restrict__ vc,
                             const int* __restrict__ block_tables, const int* __restrict__ ctx_lens,
                             f16* __restrict__ out, float* __restrict__ o_part, float* __restrict__ m_part,
                             float* __restrict__ l_part, int32_t* __restrict__ counters, int hkv, int bs,
                             int bs_shift, int max_blocks, int num_blocks, int partition, int num_splits,
                             float sl2, int balance) {
    using T = GqaMfmaTile<D, G, NW>;
    constexpr int KS = T::KS, DPL = T::DPL;
    typedef _Float16 vrow_t __attribute__((ext_vector_type(DPL)));
    typedef uint32_t vrow_u __attribute__((ext_vector_type(DPL / 2)));
    constexpr float kPShift = 7.f, kPMax = 32768.f;
    __shared__ float red_acc[NW][G][D];
    __shared__ float red_m[NW][G], red_l[NW][G];

    const int kvh = blockIdx.x, split = blockIdx.y, b = blockIdx.z;
    const int hq = hkv * G;
    const int start = split * partition;
    const int tid = threadIdx.x, lane = tid & 63, w = uniform(tid >> 6);
    const int n = lane & 15, g = lane >> 4;
    const int* bt = block_tables + (size_t)b * max_blocks;
    const int max_tok = max_blocks * bs;
    const int ctx_raw = ctx_lens[b];
    const int stride = NW * T::TOK;
    const bool fast_bs = bs == 16;
    int t0 = start + w * T::TOK;

    const int ctx = min(ctx_raw, max_tok);
    if (start >= ctx) {
        if (num_splits == 1 || (counters && split == 0))
            for (int idx = tid; idx < G * D; idx += T::THREADS)
                out[((size_t)b * hq + kvh * G + idx / D) * D + idx % D] = (f16)0.f;
        return;
    }
    const int end = min(ctx, start + partition);
    // The first pair's page ids and the Q^T fragments after the context
    // check, so that a workgroup past a short context (most of a skewed
    // batch's grid) exits after its one scalar load.
    int spa = -1, spb = -1;  // page ids of the pair at t0 (wave-uniform), loaded one pair ahead
    if (fast_bs && t0 + T::TOK <= min(start + partition, max_tok)) {
        spa = bt[uniform(t0 >> 4)];
        spb = bt[uniform((t0 >> 4) + 1)];
    }

    // Q^T fragments: head n (zeros for n >= G), dims 32 s + 8 g .. +7.
    f16x8 qf[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) qf[s] = f16x8{};
    if (n < G) {
        const f16* qrow = q + ((size_t)b * hq + kvh * G + n) * D + 8 * g;
#pragma unroll
        for (int s = 0; s < KS; ++s) qf[s] = *reinterpret_cast<const f16x8*>(qrow + 32 * s);
    }

    // Reference max of head n (the same in the head's four lanes), this
    // lane's share of l for head n, and acc[j][r]: head 4g + r, dim DPL n + j.
    float m_own = -INFINITY, l_own = 0.f;
    f32x4 acc[DPL];
#pragma unroll
    for (int j = 0; j < DPL; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // One page pair: scores, online softmax and P V.  Score i of the lane is
    // token 4g + i of page A (i < 4) or 4g + i - 4 of page B, the tokens of V
    // rows va[i] / vb[i - 4]; tokens with !valid[i] drop out when MASKED.
    auto step = [&](const f16x8 (&ka)[KS], const f16x8 (&kb)[KS], const vrow_t (&va)[4], const vrow_t (&vb)[4],
                    const bool (&valid)[8], auto masked) {
        constexpr bool MASKED = decltype(masked)::value;
        f32x4 sa = {0.f, 0.f, 0.f, 0.f}, sb = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            sa = mfma16x16x32(ka[s], qf[s], sa);
            sb = mfma16x16x32(kb[s], qf[s], sb);
        }
        const float x[8] = {sa[0], sa[1], sa[2], sa[3], sb[0], sb[1], sb[2], sb[3]};
        float p[8];
        float bias = kPShift - m_own;
#pragma unroll
        for (int i = 0; i < 8; ++i) p[i] = exp2_fast(!MASKED || valid[i] ? fmaf(x[i], sl2, bias) : -INFINITY);
        bool ok = true;
#pragma unroll
        for (int i = 0; i < 8; ++i) ok = ok && p[i] <= kPMax;  // false for inf and NaN
        if (__builtin_amdgcn_ballot_w64(!ok)) {
            // Move every head's reference max to its running max (first
            // pair: m = -inf; later: a score above m + 8).  The padding heads
            // (n >= G, scores 0) move once, on the first pair, like the rest.
            auto fmax2 = [](float u, float v) { return fmaxf(u, v); };
            float mx = -INFINITY;
#pragma unroll
            for (int i = 0; i < 8; ++i) mx = fmaxf(mx, !MASKED || valid[i] ? x[i] * sl2 : -INFINITY);
            mx = xor_combine<16>(mx, fmax2);
            mx = xor_combine<32>(mx, fmax2);
            const float m_new = fmaxf(m_own, mx);
            const float m_use = m_new == -INFINITY ? 0.f : m_new;
            const float alpha = exp2_fast(m_own - m_use);  // 0 while m was -inf
            l_own *= alpha;
            m_own = m_new;
            // accumulator row r is head 4g + r, whose alpha lane 4g + r holds
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float al = __shfl(alpha, 4 * g + r, kWave);
#pragma unroll
                for (int j = 0; j < DPL; ++j) acc[j][r] *= al;
            }
            bias = kPShift - m_use;
#pragma unroll
            for (int i = 0; i < 8; ++i) p[i] = exp2_fast(!MASKED || valid[i] ? fmaf(x[i], sl2, bias) : -INFINITY);
        }
        f16x8 pa;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const f16x2 pk = {(f16)p[2 * k], (f16)p[2 * k + 1]};
            l_own = __builtin_amdgcn_fdot2(pk, f16x2{(f16)1.f, (f16)1.f}, l_own, false);
            pa[2 * k] = pk[0];
            pa[2 * k + 1] = pk[1];
        }
        // V fragment j: the 8 tokens' dim DPL n + j, two tokens per register.
        vrow_u vu[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            vu[i] = __builtin_bit_cast(vrow_u, va[i]);
            vu[i + 4] = __builtin_bit_cast(vrow_u, vb[i]);
        }
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
            const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
            u32x4 f;
#pragma unroll
            for (int k = 0; k < 4; ++k) f[k] = __builtin_amdgcn_perm(vu[2 * k + 1][j >> 1], vu[2 * k][j >> 1], sel);
            acc[j] = mfma16x16x32(pa, __builtin_bit_cast(f16x8, f), acc[j]);
        }
    };

    const size_t page_stride = (size_t)hkv * bs * D;  // elements
    // Whole pairs of 16-token pages: two wave-uniform page ids (loaded one
    // pair ahead), every K/V load at page base + lane offset.
    {
        const uint32_t kv_off = (uint32_t)(kvh * 16 * D);
        uint32_t koff[KS], voff[4];  // byte offsets inside a page
#pragma unroll
        for (int s = 0; s < KS; ++s) koff[s] = (kv_off + n * D + 32 * s + 8 * g) * 2;
#pragma unroll
        for (int r = 0; r < 4; ++r) voff[r] = (kv_off + (4 * g + r) * D + DPL * n) * 2;
        const bool unused[8] = {};
        while (fast_bs && t0 + T::TOK <= end && (unsigned)spa < (unsigned)num_blocks &&
               (unsigned)spb < (unsigned)num_blocks) {
            f16x8 ka[KS], kb[KS];
            vrow_t va[4], vb[4];
            const char* kpa = reinterpret_cast<const char*>(kc + (size_t)spa * page_stride);
            const char* kpb = reinterpret_cast<const char*>(kc + (size_t)spb * page_stride);
            const char* vpa = reinterpret_cast<const char*>(vc + (size_t)spa * page_stride);
            const char* vpb = reinterpret_cast<const char*>(vc + (size_t)spb * page_stride);
#pragma unroll
            for (int s = 0; s < KS; ++s) {  // streamed once: non-temporal
                ka[s] = __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(kpa + koff[s]));
                kb[s] = __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(kpb + koff[s]));
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                va[r] = __builtin_nontemporal_load(reinterpret_cast<const vrow_t*>(vpa + voff[r]));
                vb[r] = __builtin_nontemporal_load(reinterpret_cast<const vrow_t*>(vpb + voff[r]));
            }
            const int tn = t0 + stride;
            if (tn < end) {  // the next pair's page ids (page B only if it holds a token)
                spa = bt[uniform(tn >> 4)];
                spb = tn + 16 < end ? bt[uniform((tn >> 4) + 1)] : -1;
            }
            if (balance) progress_priority(t0 - start, end - start);
            step(ka, kb, va, vb, unused, std::false_type{});
            t0 = tn;
        }
        __builtin_amdgcn_s_setprio(0);
        // The pair that holds the end of the context: the same page-base loads
        // with the page ids already loaded, rows past the end left zero and
        // masked out of the softmax.  (Through the checked path below, each
        // lane would look up its 10 token rows' page ids first: one more
        // dependent memory round trip for every sequence.)
        const bool hasb = t0 + 16 < end;
        if (fast_bs && t0 < end && t0 + T::TOK > end && (unsigned)spa < (unsigned)num_blocks &&
            (!hasb || (unsigned)spb < (unsigned)num_blocks)) {
            f16x8 ka[KS], kb[KS];
            vrow_t va[4], vb[4];
            bool valid[8];
            const int pb = hasb ? spb : spa;  // no row of page B is read when it holds no token
            const char* kpa = reinterpret_cast<const char*>(kc + (size_t)spa * page_stride);
            const char* vpa = reinterpret_cast<const char*>(vc + (size_t)spa * page_stride);
            const char* kpb = reinterpret_cast<const char*>(kc + (size_t)pb * page_stride);
            const char* vpb = reinterpret_cast<const char*>(vc + (size_t)pb * page_stride);
            const bool ka_ok = t0 + n < end, kb_ok = t0 + 16 + n < end;
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                ka[s] = ka_ok ? __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(kpa + koff[s])) : f16x8{};
                kb[s] = kb_ok ? __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(kpb + koff[s])) : f16x8{};
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                valid[r] = t0 + 4 * g + r < end;
                valid[r + 4] = t0 + 16 + 4 * g + r < end;
                va[r] = valid[r] ? __builtin_nontemporal_load(reinterpret_cast<const vrow_t*>(vpa + voff[r]))
                                 : vrow_t{};
                vb[r] = valid[r + 4] ? __builtin_nontemporal_load(reinterpret_cast<const vrow_t*>(vpb + voff[r]))
                                     : vrow_t{};
            }
            step(ka, kb, va, vb, valid, std::true_type{});
            t0 += stride;
        }
    }
    // The rest (context tail, out-of-range page ids, pages not of 16 tokens):
    // every token row located on its own; rows that are not read are zeros.
    for (; t0 < end; t0 += stride) {
        auto locate = [&](int t, bool& ok) -> size_t {  // element offset of token t's row
            const int pi = bs_shift >= 0 ? (t >> bs_shift) : (t / bs);
            const int po = bs_shift >= 0 ? (t & (bs - 1)) : (t % bs);
            const int pid = t < end ? bt[pi] : -1;
            ok = t < end && (unsigned)pid < (unsigned)num_blocks;
            return ok ? (size_t)pid * page_stride + ((size_t)kvh * bs + po) * D : 0;
        };
        f16x8 ka[KS], kb[KS];
        vrow_t va[4], vb[4];
        bool valid[8], kok;
        const size_t kao = locate(t0 + n, kok);
#pragma unroll
        for (int s = 0; s < KS; ++s)
            ka[s] = kok ? *reinterpret_cast<const f16x8*>(kc + kao + 32 * s + 8 * g) : f16x8{};
        const size_t kbo = locate(t0 + 16 + n, kok);
#pragma unroll
        for (int s = 0; s < KS; ++s)
            kb[s] = kok ? *reinterpret_cast<const f16x8*>(kc + kbo + 32 * s + 8 * g) : f16x8{};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const size_t oa = locate(t0 + 4 * g + r, valid[r]);
            va[r] = valid[r] ? *reinterpret_cast<const vrow_t*>(vc + oa + DPL * n) : vrow_t{};
            const size_t ob = locate(t0 + 16 + 4 * g + r, valid[r + 4]);
            vb[r] = valid[r + 4] ? *reinterpret_cast<const vrow_t*>(vc + ob + DPL * n) : vrow_t{};
        }
        step(ka, kb, va, vb, valid, std::true_type{});
    }

    // Merge the wave: l over the four lanes of each head, then the G heads'
    // rows to LDS for the workgroup's merge.
    auto add2 = [](float u, float v) { return u + v; };
    l_own = xor_combine<16>(l_own, add2);
    l_own = xor_combine<32>(l_own, add2);
    if (g == 0 && n < G) {
        red_m[w][n] = m_own;
        red_l[w][n] = l_own;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int h = 4 * g + r;
        if (h < G)
#pragma unroll
            for (int j = 0; j < DPL; ++j) red_acc[w][h][DPL * n + j] = acc[j][r];
    }
    __syncthreads();
    split_epilogue<D, G, NW>(red_acc, red_m, red_l, 1.f / 128.f, out, o_part, m_part, l_part, counters, b, kvh,
                             hkv, split, num_splits, splits_with_tokens(ctx, partition, num_splits), tid);
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

// Software pipelining of the dot-product grouped-query kernel's main loop (the
// next chunk's K and V issued before this chunk is computed).  Measured on
// MI355X, back-to-back calls at the default partition: D = 64 with 4 query
// heads per kv head +4% to +6.5%; D = 128 -2% to +3%, so only D = 64 with
// four heads pipelines.  (The matrix-core kernel for eight heads gains nothing
// from it: -1% to +1%.)
constexpr bool gqa_pipelined(int d, int g) { return d == 64 && g >= 4; }

// Waves per workgroup of both grouped-query kernels.  A dot-product wave
// reads one 16-token page per round trip to memory, so a split of P tokens
// costs P / (16 NW) dependent round trips; with many workgroups per CU they
// overlap, but in a small grid (one sequence, few kv heads) they are the
// kernel's critical path.  Measured on MI355X (one call after a 512 MiB flush,
// G = 2, 4, 8, D = 64 and 128): grids under 512 workgroups run 0.3-1.9 us
// faster with 8 waves than with 4 (B=1 ctx 1024: 11.8 vs 13.7 us; ctx 16384:
// 20.8 vs 21.4 us), and 16 waves are slower than 8 everywhere; from 512
// workgroups up, 4 waves win.  The matrix-core kernel (two pages per round
// trip) measured the same way picks the same: 4 waves at B = 8 x 8192 tokens
// (8 waves -2%), 8 at B = 1 (equal or better).
template <int G>
static int gqa_waves(const DecodeArgs& a) {
    const int64_t wgs = a.batch * a.hkv * a.num_splits;
    return wgs * 4 >= kGqaManyWaves ? 4 : 8;
}

// Whether all `wgs` workgroups of a launch of KERNEL are resident at once,
// the case in which the grouped-query kernels balance their waves by issue
// priority (progress_priority).  Workgroups per CU come from the runtime's
// occupancy calculator (registers, LDS, waves), once per kernel; the CU count
// from the current device.  Host-side queries only: nothing is allocated or
// enqueued.
template <auto KERNEL>
static bool one_round(int threads, int64_t wgs) {
    static const int per_cu = [threads] {
        int n = 0;
        return hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(KERNEL), threads, 0) ==
                       hipSuccess
                   ? n
                   : 0;
    }();
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return false;
    return per_cu > 0 && wgs <= (int64_t)per_cu * cus;
}

template <int D, int G>
static hipError_t launch_decode(const DecodeArgs& a) {
    int bs_shift = -1;
    for (int s = 0; s < 31; ++s)
        if ((int64_t(1) << s) == a.bs) bs_shift = s;
    const hipStream_t stream = (hipStream_t)a.stream;
    dim3 grid((unsigned)a.hkv, (unsigned)a.num_splits, (unsigned)a.batch);
    // Few enough splits: the last split of each (sequence, kv head) merges them
    // in the decode kernel (no reduce launch); otherwise the reduce kernel does.
    int32_t* counters = a.counters && a.num_splits > 1 && a.num_splits <= kFusedMaxSplits ? a.counters : nullptr;
    if constexpr (G == 1)
        hipLaunchKernelGGL((paged_decode_kernel<D>), grid, dim3(DecodeTile<D>::THREADS), 0, stream, (const f16*)a.q,
                           (const f16*)a.k_cache, (const f16*)a.v_cache, a.block_tables, a.context_lens,
                           (f16*)a.out, a.o_part, a.m_part, a.l_part, counters, (int)a.hkv, (int)a.bs, bs_shift,
                           (int)a.max_blocks, (int)a.num_blocks, (int)a.partition, (int)a.num_splits, a.sl2);
    else {
        const int64_t wgs = a.batch * a.hkv * a.num_splits;
        auto launch = [&](auto nw) {
            constexpr int NW = decltype(nw)::value, THREADS = GqaTile<D, G, NW>::THREADS;
            const int balance = one_round<paged_decode_gqa_kernel<D, G, NW, gqa_pipelined(D, G)>>(THREADS, wgs);
            hipLaunchKernelGGL((paged_decode_gqa_kernel<D, G, NW, gqa_pipelined(D, G)>), grid, dim3(THREADS), 0,
                               stream, (const f16*)a.q, (const f16*)a.k_cache, (const f16*)a.v_cache,
                               a.block_tables, a.context_lens, (f16*)a.out, a.o_part, a.m_part, a.l_part, counters,
                               (int)a.hkv, (int)a.bs, bs_shift, (int)a.max_blocks, (int)a.num_blocks,
                               (int)a.partition, (int)a.num_splits, a.sl2, balance);
        };
        auto launch_mfma = [&](auto nw) {
            constexpr int NW = decltype(nw)::value, THREADS = GqaMfmaTile<D, G, NW>::THREADS;
            const int balance = one_round<paged_decode_gqa_mfma_kernel<D, G, NW>>(THREADS, wgs);
            hipLaunchKernelGGL((paged_decode_gqa_mfma_kernel<D, G, NW>), grid, dim3(THREADS), 0, stream,
                               (const f16*)a.q, (const f16*)a.k_cache, (const f16*)a.v_cache, a.block_tables,
                               a.context_lens, (f16*)a.out, a.o_part, a.m_part, a.l_part, counters, (int)a.hkv,
                               (int)a.bs, bs_shift, (int)a.max_blocks, (int)a.num_blocks, (int)a.partition,
                               (int)a.num_splits, a.sl2, balance);
        };
        const bool many = gqa_waves<G>(a) == 4;
        if constexpr (G == 8) {
            if (many)
                launch_mfma(std::integral_constant<int, 4>{});
            else
                launch_mfma(std::integral_constant<int, 8>{});
        } else if (many)
            launch(std::integral_constant<int, 4>{});
        else
            launch(std::integral_constant<int, 8>{});
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.num_splits == 1 || counters) return e;
    hipLaunchKernelGGL((paged_reduce_kernel<D>), dim3((unsigned)(a.batch * a.hq)), dim3(256), 0, stream,
                       a.o_part, a.m_part, a.l_part, a.context_lens, (f16*)a.out, (int)a.hq,
                       (int)a.partition, (int)a.num_splits, (int)(a.max_blocks * a.bs));
    return hipGetLastError();
}

// Split partials of ak_paged_decode_noalloc: one static array per GPU, held
// until the process ends, so that callers that cannot allocate (graph capture,
// tight serving loops) need no workspace.  Every call on a GPU shares that
// GPU's array; calls that overlap on one GPU race.  The partials need no
// initial contents: a merge reads only partials the same call wrote.  The
// split counters (one per sequence and kv head) start at zero, as every
// static device array does, and every call leaves them at zero.
static __device__ __align__(256) float scratch[kDecodeScratchBytes / sizeof(float)];
static __device__ __align__(256) int32_t scratch_counters[kDecodeScratchCounters];

// Device addresses of this GPU's scratch arrays.  In host code `scratch` and
// `scratch_counters` name host-side stand-ins, never the device memory: the
// addresses come from hipGetSymbolAddress with the device current, and only
// those pointers are handed to kernels.  They are looked up again on every
// call (a lookup allocates nothing), so they stay valid across a
// hipDeviceReset that reloads the module.
hipError_t decode_scratch(void** ptr, int32_t** counters) {
    void* p = nullptr;
    void* c = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e == hipSuccess) e = hipGetSymbolAddress(&c, HIP_SYMBOL(scratch_counters));
    if (e != hipSuccess) return e;
    if (!p || !c) return hipErrorInvalidSymbol;
    *ptr = p;
    *counters = static_cast<int32_t*>(c);
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
