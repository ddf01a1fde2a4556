// Flash prefill on CDNA4 f16 MFMA (gfx950).
//
// One kernel serves the reference's three prefill entry points
// (naive_attn.cu:65-86, flash_simt.cu:209-221, flash_wmma.cu:241-257): same
// inputs, same online-softmax algorithm (flash_wmma.cu:114-194), same masking
// and guards, built for wave64 and the 32x32x16 matrix core instead of warps.
//
// Layout choices
//   * A workgroup is 8 waves and owns BM = 256 query rows of one (batch, head);
//     each wave owns 32 of them, so no softmax row is shared between waves.
//     Eight waves share each K/V tile in LDS: half the LDS traffic per query
//     row of a 4-wave workgroup, and each wave issues only 2 one-KB loads per
//     K and per V tile.  Short sequences and small grids use 4-wave workgroups
//     (128 rows, two per CU; at D = 64 with 64-key tiles, three per CU)
//     instead: see prefill_waves.
//   * Scores are computed transposed, S^T = K Q^T, with K as the MFMA A operand
//     (16-byte LDS reads of K rows) and Q as the B operand (kept in VGPRs for
//     the whole kernel).  In the accumulator a lane then holds one query column
//     and 16 keys per 32x32 block, so the row max / sum are in-lane plus one
//     exchange with lane l^32.
//   * O^T = V^T P^T.  P^T comes straight from the S^T accumulators (converted
//     to f16, no LDS round trip): accumulator rows 8c..8c+7 of a lane half are
//     keys 16c + {0..3, 8..11} (+4 for the upper half).  The V^T operand is
//     read from the row-major V tile with ds_read_b64_tr_b16, which hands each
//     lane 4 consecutive keys of one head dim; two such reads give the keys
//     16c + 4h + {0..3} and 16c + 8 + 4h + {0..3} that line up with P's k.  The
//     head dims a lane reads are permuted (bits 2/3 of d swapped) so that its
//     O^T accumulators hold 8 contiguous head dims (16-byte output stores).
//   * K and V tiles go from global memory straight into LDS
//     (global_load_lds_dwordx4: no staging registers, no register transposes),
//     each in a ring of two tiles, one barrier per tile.  Rows are unpadded;
//     16-byte chunks are XOR-swizzled by row so that the K operand reads, the
//     transposed V reads and the DMA writes are all free of bank conflicts.
//     64 KB per workgroup (32 KB for the 64-key D = 64 tiles).  At about 230
//     VGPRs a SIMD holds two waves, so a CU runs one 8-wave workgroup, or two
//     4-wave workgroups, at a time; the D = 64 4-wave kernel stays under 168
//     VGPRs, and a CU holds three of its workgroups.
//   * The key loop is software-pipelined inside each wave: while the matrix
//     core computes the scores of tile t+1, the VALU turns the scores of tile
//     t into P (exponentials, fp16 conversion, row sums), then P V of tile t
//     follows.  sched_group_barrier fixes that interleave.  K is therefore
//     loaded two tiles ahead and V one tile ahead.
//   * Causal: a workgroup processes query tile j and tile nqt-1-j, so every
//     workgroup has the same amount of work; waves skip key tiles that lie
//     entirely above their diagonal; masking runs only on diagonal/tail tiles.
//   * Workgroup ids are remapped so that the query tiles of one (batch, head)
//     run on the same XCD and share its L2.
#include "attn_kernels.hpp"
#include "wave.hpp"

#include <type_traits>

#define AK_LDS __attribute__((address_space(3)))
#define AK_GLOBAL __attribute__((address_space(1)))

namespace ak {

typedef short s16x4 __attribute__((ext_vector_type(4)));

template <int D, int NWAVES = 8>
struct PrefillTile {
    static constexpr int NW = NWAVES;            // waves per workgroup: 8, or 4 for short sequences
    static constexpr int THREADS = NW * kWave;   // 512 or 256
    static constexpr int QW = 32;                // query rows per wave
    static constexpr int BM = NW * QW;           // query rows per workgroup
    static constexpr int CPR = D / 8;            // 16-byte chunks per K/V row
    // Keys per tile: a K tile is 16 KB (64 keys at D = 128, 128 at D = 64), except
    // for D = 64 in 4-wave workgroups, whose 64-key tiles keep the wave under
    // 168 VGPRs, so that a CU holds three of those workgroups (+5-9% on short
    // sequences; with 8 waves the 128-key tile is 2-4% faster).
    static constexpr int BN = D == 64 && NW == 4 ? 64 : 8192 / D;
    static constexpr int TILE = BN * D;          // halves per K (or V) tile
    static constexpr int STAGE = 2 * TILE;       // K + V
    static constexpr int RPI = 512 / D;          // rows per 1 KB load instruction
    static constexpr int LPW = TILE * 2 / 1024 / NW;  // 1 KB load instructions per wave per tile
    static constexpr int RPL = 128 / D;          // rows per 256-byte LDS bank line
    static constexpr int KB = BN / 32;           // 32-key blocks of S^T
    static constexpr int DC = D / 16;            // k-steps of K Q^T
    static constexpr int DT = D / 32;            // 32-row tiles of O^T
    static constexpr int PC = BN / 16;           // k-steps of V^T P^T
    static_assert(LPW >= 1 && LPW * NW * 1024 == TILE * 2, "the waves split each tile into whole KBs");
    static_assert(D % 32 == 0 && BN % 32 == 0, "tile shapes");
};

// Physical 16-byte chunk of logical chunk c in row r.  K: rows of one 256-byte
// bank line sequence get distinct chunks, so 16 lanes reading one logical
// chunk of 16 consecutive rows hit 16 different bank groups.  V: groups of 4
// consecutive rows get disjoint 64-byte blocks, which is what one transposed
// read of 4 rows x 16 head dims per 16 lanes needs.
template <int D>
__device__ __forceinline__ int k_chunk(int r, int c) {
    using T = PrefillTile<D>;
    return c ^ ((r / T::RPL) % T::CPR);
}
template <int D>
__device__ __forceinline__ int v_chunk(int r, int c) {
    using T = PrefillTile<D>;
    return c ^ (4 * ((r / T::RPL) % (T::CPR / 4)));
}

// Global -> LDS for one K (or V) tile, keys [k0, k0 + BN), asynchronous
// (vmcnt).  Each wave writes LPW contiguous KB of the tile; lane l fills the
// 16-byte slot l of a KB.  Row r starts r * rs elements after src.  Rows past n
// are clamped to row n-1: in bounds, and masked to -inf later.
//
// The load is issued as inline asm (M0 = LDS destination, set by the operand
// constraint; s_nop 0 is the one wait state an M0 write needs before an LDS
// DMA).  Issued through the builtin, the compiler's wait-count model treats the
// LDS counter as out of order for the whole loop and waits lgkmcnt(0) before
// every MFMA that reads a K or V fragment; hidden from it, the fragment reads
// get partial waits.  The compiler then no longer orders anything after these
// loads: every reader of the tile waits in wait_loads_and_sync (vmcnt(0), then
// the barrier), and the buffer a load overwrites was last read before the
// barrier that precedes it.
template <int D, bool IS_V, int NW>
__device__ __forceinline__ void load_kv(const f16* __restrict__ src, f16* dst, int k0, int n, int rs, int w,
                                        int lane) {
    using T = PrefillTile<D, NW>;
#pragma unroll
    for (int j = 0; j < T::LPW; ++j) {
        const int blk = w * T::LPW + j;
        const int row = blk * T::RPI + lane / T::CPR, p = lane % T::CPR;
        const int c = IS_V ? v_chunk<D>(row, p) : k_chunk<D>(row, p);
        const f16* g = src + (size_t)min(k0 + row, n - 1) * rs + c * 8;
        const uint32_t l = __builtin_amdgcn_readfirstlane((uint32_t)(size_t)(AK_LDS void*)(dst + blk * 512));
        asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(l));
    }
}

__device__ __forceinline__ void wait_loads_and_sync() {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
}

// {own value, value of lane l^32} in some order, by v_permlane32_swap on two
// copies of x (no LDS traffic).  Issued as inline asm: with the builtin and
// identical inputs the compiler kept only one of the two swapped registers.
// The s_nop covers the VALU-write -> permlane-read hazard.
__device__ __forceinline__ f32x2 pair_values(float x) {
    float a = x, b = x;
    asm volatile("s_nop 2\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    return f32x2{a, b};
}
__device__ __forceinline__ float pair_max(float x) {
    const f32x2 v = pair_values(x);
    return fmaxf(v[0], v[1]);
}
__device__ __forceinline__ float pair_sum(float x) {
    const f32x2 v = pair_values(x);
    return v[0] + v[1];
}

// The subtracted row maximum only moves when the tile's maximum exceeds it by
// more than this many powers of two, so O is rescaled rarely.  Softmax is
// invariant to the value subtracted; P stays <= 2^8, exact enough in fp16.
constexpr float kRescaleSlack = 8.f;

// S^T = K Q^T for one key tile: KB blocks of 32 keys x 32 queries; lane reads
// key row 32b+col, chunk 2dc+half.
template <int D, int NW>
__device__ __forceinline__ void qk_tile(const f16* __restrict__ ks, const f16x8 (&qf)[(PrefillTile<D, NW>::DC)],
                                        f32x16 (&s)[(PrefillTile<D, NW>::KB)], int lane) {
    using T = PrefillTile<D, NW>;
    const int col = lane & 31, half = lane >> 5;
#pragma unroll
    for (int b = 0; b < T::KB; ++b) s[b] = f32x16{};
    // D = 128: head-dim step outermost, so consecutive MFMAs share the Q operand
    // and write independent accumulators (+0.5-0.7% at N = 8192, bit-identical);
    // D = 64 was not faster that way.
    constexpr bool DC_OUTER = D == 128;
#pragma unroll
    for (int x = 0; x < T::KB * T::DC; ++x) {
        const int b = DC_OUTER ? x % T::KB : x / T::DC, dc = DC_OUTER ? x / T::KB : x % T::DC;
        const int r = b * 32 + col;
        s[b] = mfma32x32x16(*reinterpret_cast<const f16x8*>(ks + r * D + k_chunk<D>(r, 2 * dc + half) * 8), qf[dc],
                            s[b]);
    }
}

// Keys past n and, if causal, keys after the query -> -inf.
template <int D, int NW, bool CAUSAL>
__device__ __forceinline__ void mask_tile(f32x16 (&s)[(PrefillTile<D, NW>::KB)], int k0, int n, int qrow, int half) {
    using T = PrefillTile<D, NW>;
#pragma unroll
    for (int b = 0; b < T::KB; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int key = k0 + b * 32 + (r >> 2) * 8 + half * 4 + (r & 3);
            if (key >= n || (CAUSAL && key > qrow)) s[b][r] = -INFINITY;
        }
}

// Tile row maximum; moves the subtracted maximum (and rescales O and l) only
// when it grows by more than kRescaleSlack, which is rare after the first tile.
// Used on the diagonal (masked) tiles of causal D = 64 only.
template <int D, int NW>
__device__ __forceinline__ void max_tile(const f32x16 (&s)[(PrefillTile<D, NW>::KB)], f32x16 (&o)[(PrefillTile<D, NW>::DT)],
                                         float& ms_run, float& l_run, float sl2) {
    using T = PrefillTile<D, NW>;
    float mx = -INFINITY;
#pragma unroll
    for (int b = 0; b < T::KB; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[b][r]);
    const float mxs = pair_max(mx) * sl2;  // this tile's scaled row max (-inf if all masked)
    const bool grow = mxs > ms_run + kRescaleSlack;  // always true on the first tile
    if (__builtin_amdgcn_ballot_w64(grow)) {
        const float ms_new = grow ? mxs : ms_run;
        const float alpha = exp2_fast(ms_run - ms_new);  // 0 on the first tile, 1 if unchanged
        ms_run = ms_new;
        l_run *= alpha;
#pragma unroll
        for (int t = 0; t < T::DT; ++t) o[t] *= alpha;
    }
}

// P^T = 2^(S^T sl2 - ms) as the fp16 B operand, for key steps [C0, C1): k-step
// c = accumulator regs 8*(c%2).. of block c/2.  The row sum is taken over the
// same fp16 values the MFMA consumes, two at a time by v_dot2_f32_f16 against
// (1, 1), in the caller's 4 chains.  D = 64 splits a tile's steps in two: it
// has twice the scores per MFMA of D = 128, so half of them are exponentiated
// under the P V MFMAs instead of all under QK^T.
template <int D, int NW, int C0, int C1>
__device__ __forceinline__ void exp_part(const f32x16 (&s)[(PrefillTile<D, NW>::KB)], f16x8 (&pf)[(PrefillTile<D, NW>::PC)],
                                         float ms_run, float (&ps)[4], float sl2) {
    const f16x2 ones = {(f16)1.f, (f16)1.f};
#pragma unroll
    for (int c = C0; c < C1; ++c) {
#pragma unroll
        for (int i = 0; i < 8; ++i) pf[c][i] = (f16)exp2_fast(fmaf(s[c >> 1][(c & 1) * 8 + i], sl2, -ms_run));
#pragma unroll
        for (int i = 0; i < 4; ++i)
            ps[i] = __builtin_amdgcn_fdot2(f16x2{pf[c][2 * i], pf[c][2 * i + 1]}, ones, ps[i], false);
    }
}

// O^T += V^T P^T over key steps [C0, C1), key step outermost: the MFMAs of
// step c need only pf[c], so the exponentials of later steps can run under the
// MFMAs of earlier ones, and consecutive MFMAs share the P operand.  Transposed
// reads: in each 16-lane group, lane a points at row kb + a/4, head dims
// dbase + 4*sw(a%4) (sw swaps bits 0/1); lane i then receives keys kb..kb+3 of
// head dim dbase + 4*sw(i/4) + i%4.
template <int D, int NW, int C0, int C1>
__device__ __forceinline__ void pv_part(const f16* __restrict__ vs, const f16x8 (&pf)[(PrefillTile<D, NW>::PC)],
                                        f32x16 (&o)[(PrefillTile<D, NW>::DT)], int lane) {
    using T = PrefillTile<D, NW>;
    const int half = lane >> 5, a = lane & 15, gd = (lane >> 4) & 1;
    const int dsub = 16 * gd + 4 * (((a & 1) << 1) | ((a >> 1) & 1));
#pragma unroll
    for (int c = C0; c < C1; ++c) {
#pragma unroll
        for (int t = 0; t < T::DT; ++t) {
            const int dcol = t * 32 + dsub;
            f16x4 lohi[2];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int r = 16 * c + 8 * e + 4 * half + (a >> 2);
                const f16* p = vs + r * D + v_chunk<D>(r, dcol >> 3) * 8 + (dcol & 7);
                lohi[e] = __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((AK_LDS s16x4*)p));
            }
            const f16x8 va = {lohi[0][0], lohi[0][1], lohi[0][2], lohi[0][3],
                              lohi[1][0], lohi[1][1], lohi[1][2], lohi[1][3]};
            o[t] = mfma32x32x16(va, pf[c], o[t]);
        }
    }
}

// Exponents checked after the fact instead of taking the tile maximum first:
// P = 2^(S sl2 - m) is computed against the current subtracted maximum m, and
// only if a lane's sum over key steps [C0, C1) reaches 2^14 (some P near the
// top of fp16) or is not finite (the first tile, against m = -inf) does the
// wave come here.  Both lanes of each such row then move m to the maximum of
// those key steps, rescale O and l, and recompute P for them; rows that do not
// move recompute the same P.  D = 128 checks whole tiles; D = 64 checks each
// part of a tile before its P V MFMAs, and when the second part moves m the
// rescale also covers the first part's P V, already in O.  This saves the
// row-max pass (v_max3, a lane exchange and a compare per tile).
constexpr float kTileSumLimit = 16384.f;
template <int D, int NW, int C0, int C1>
__device__ __forceinline__ void settle_part(const f32x16 (&s)[(PrefillTile<D, NW>::KB)],
                                            f16x8 (&pf)[(PrefillTile<D, NW>::PC)],
                                            f32x16 (&o)[(PrefillTile<D, NW>::DT)], float& ms_run, float& l_run,
                                            float& l_part, bool bad, float sl2) {
    float mx = -INFINITY;
#pragma unroll
    for (int c = C0; c < C1; ++c)
#pragma unroll
        for (int i = 0; i < 8; ++i) mx = fmaxf(mx, s[c >> 1][(c & 1) * 8 + i]);
    const float mxs = pair_max(mx) * sl2;
    const bool move = pair_max(bad ? 1.f : 0.f) > 0.f && mxs > ms_run;
    if (move) {
        const float alpha = exp2_fast(ms_run - mxs);  // 0 on the first tile
        ms_run = mxs;
        l_run *= alpha;
#pragma unroll
        for (int t = 0; t < PrefillTile<D, NW>::DT; ++t) o[t] *= alpha;
    }
    float ps[4] = {0.f, 0.f, 0.f, 0.f};
    exp_part<D, NW, C0, C1>(s, pf, ms_run, ps, sl2);
    l_part = (ps[0] + ps[1]) + (ps[2] + ps[3]);
}

// Instruction interleave of one pipelined tile (sched_group_barrier masks:
// 0x008 MFMA, 0x002 VALU, 0x400 transcendental, 0x100 LDS read).  Per MFMA of
// the next tile's S: a few VALU ops and exponentials of this tile's P and the
// K read for a later MFMA; K reads run kKPrefetch ahead, V reads kVPrefetch.
// At D = 64 each P V MFMA also takes kValuPerPvMfma VALU ops and kExpPerMfma
// exponentials of the second half of P.
constexpr int kValuPerMfma = 3, kExpPerMfma = 2, kKPrefetch = 2, kVPrefetch = 4, kValuPerPvMfma = 4;

// Software-pipelined key loop: iteration t multiplies the scores of tile t
// (computed one iteration earlier) into O while the matrix core computes the
// scores of tile t+1, so the exponentials of one tile overlap the QK^T MFMAs
// of the next inside every wave.  K runs two tiles ahead in a 2-buffer ring,
// V one tile ahead in another; one barrier per tile.
template <int D, bool CAUSAL, int NW>
__device__ __forceinline__ void prefill_qtile(const f16* __restrict__ qb, const f16* __restrict__ kb,
                                              const f16* __restrict__ vb, f16* __restrict__ ob,
                                              f16* __restrict__ lds, int q0, int n, int qs, int ks, float sl2,
                                              uint32_t qflip) {
    using T = PrefillTile<D, NW>;
    const int tid = threadIdx.x;
    const int lane = tid & 63, w = uniform(tid >> 6);
    const int col = lane & 31, half = lane >> 5;
    const int qw0 = q0 + w * T::QW;
    const int qrow = qw0 + col;
    f16* kbuf = lds;                 // 2 K tiles
    f16* vbuf = lds + 2 * T::TILE;   // 2 V tiles

    const int kend = CAUSAL ? min(n, q0 + T::BM) : n;
    const int nkt = (kend + T::BN - 1) / T::BN;
    // Tiles before kt_mask need no masking for any wave of the workgroup: all
    // their keys are < n and (causal) <= the workgroup's first query row.
    const int kt_mask = min(nkt, CAUSAL ? q0 / T::BN : n / T::BN);

    load_kv<D, false, NW>(kb, kbuf, 0, n, ks, w, lane);
    load_kv<D, true, NW>(vb, vbuf, 0, n, ks, w, lane);
    if (nkt > 1) load_kv<D, false, NW>(kb, kbuf + T::TILE, T::BN, n, ks, w, lane);

    // Q as the MFMA B operand: col = query, k = head dim 16*dc + 8*half .. +7.
    f16x8 qf[T::DC];
#pragma unroll
    for (int dc = 0; dc < T::DC; ++dc) {
        // Rows past n are clamped to n-1: computed, never stored.
        f16x8 x = *reinterpret_cast<const f16x8*>(qb + (size_t)min(qrow, n - 1) * qs + dc * 16 + half * 8);
        if (qflip) {  // negative scale: fold the sign into Q exactly
            typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
            x = __builtin_bit_cast(f16x8, __builtin_bit_cast(u32x4, x) ^ qflip);
        }
        qf[dc] = x;
    }
    f32x16 o[T::DT];
#pragma unroll
    for (int t = 0; t < T::DT; ++t) o[t] = f32x16{};
    float ms_run = -INFINITY; // the scaled row maximum subtracted so far
    float l_run = 0.f;        // this lane's share of the row sum

    wait_loads_and_sync();
    // S(t) alternates between sx and sy (loop unrolled by 2: no copies).
    f32x16 sx[T::KB], sy[T::KB];
    qk_tile<D, NW>(kbuf, qf, sx, lane);

    // One tile: sc holds S(t); sn receives S(t+1), which the last tile skips.
    auto body = [&](int t, f32x16 (&sc)[T::KB], f32x16 (&sn)[T::KB], auto mask_tag, auto last_tag) {
        constexpr bool MASK = decltype(mask_tag)::value;
        constexpr bool LAST = decltype(last_tag)::value;  // the last tile: no next S to compute
        wait_loads_and_sync();  // K(t+1), V(t) landed; nobody reads K(t), V(t-1) any more
        if (t + 2 < nkt) load_kv<D, false, NW>(kb, kbuf + (t & 1) * T::TILE, (t + 2) * T::BN, n, ks, w, lane);
        // V(t+1) goes to the slot of V(t-1), last read before this barrier.  D = 64
        // issues it here; D = 128 after its QK^T phase, which spreads the CU's tile
        // loads over the tile (+1-2% at D = 128, -8-10% at D = 64).  Every body but
        // the last has a next tile (t + 1 < nkt), so the guard is compile-time: a
        // runtime branch after the QK^T phase let the compiler move the second
        // unrolled body's exponentials out of the QK^T interleave, below the branch.
        constexpr bool V_LATE = D == 128;
        if (!V_LATE && !LAST)
            load_kv<D, true, NW>(vb, vbuf + ((t + 1) & 1) * T::TILE, (t + 1) * T::BN, n, ks, w, lane);
        // Causal: a tile whose first key is after this wave's last row is skipped.
        const bool act = !MASK || !CAUSAL || t * T::BN <= qw0 + T::QW - 1;
        // The diagonal tiles of causal D = 64 take the tile's row maximum first; all
        // other tiles check the exponents after the fact (settle_part).
        // The split check on the masked tiles as well costs the causal D = 64 kernels
        // their register budget (spills at 8 waves, a third workgroup per CU at 4).
        constexpr bool MAX_FIRST = D == 64 && CAUSAL && MASK;
        if (act) {
            if constexpr (MASK) mask_tile<D, NW, CAUSAL>(sc, t * T::BN, n, qrow, half);
            if constexpr (MAX_FIRST) max_tile<D, NW>(sc, o, ms_run, l_run, sl2);
        }
        // The wave holds priority 1 while its QK^T MFMAs and exponentials run and
        // drops to 0 for P V and the max/barrier phase, so of the two waves on a
        // SIMD the one in the mixed MFMA+VALU phase issues first.  s_setprio ends
        // a scheduling region: each phase carries its own interleave.
        __builtin_amdgcn_s_setprio(1);
        if constexpr (!LAST) qk_tile<D, NW>(kbuf + ((t + 1) & 1) * T::TILE, qf, sn, lane);
        f16x8 pf[T::PC];
        float ps[4] = {0.f, 0.f, 0.f, 0.f};
        if (act) {
            if constexpr (D == 64) exp_part<D, NW, 0, T::PC / 2>(sc, pf, ms_run, ps, sl2);
            else exp_part<D, NW, 0, T::PC>(sc, pf, ms_run, ps, sl2);
            if constexpr (!LAST) {
                __builtin_amdgcn_sched_group_barrier(0x100, kKPrefetch, 0);
#pragma unroll
                for (int i = 0; i < T::KB * T::DC; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA (S of the next tile)
                    __builtin_amdgcn_sched_group_barrier(0x002, kValuPerMfma, 0);  // VALU (this tile's P)
                    __builtin_amdgcn_sched_group_barrier(0x400, kExpPerMfma, 0);  // exp
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // next K fragment read
                }
            }
        } else if constexpr (!LAST) {
            __builtin_amdgcn_sched_group_barrier(0x100, kKPrefetch, 0);
        }
        __builtin_amdgcn_s_setprio(0);
        if (V_LATE && !LAST)
            load_kv<D, true, NW>(vb, vbuf + ((t + 1) & 1) * T::TILE, (t + 1) * T::BN, n, ks, w, lane);
        if (act) {
            if constexpr (MAX_FIRST) {
                exp_part<D, NW, T::PC / 2, T::PC>(sc, pf, ms_run, ps, sl2);
                l_run += (ps[0] + ps[1]) + (ps[2] + ps[3]);
                pv_part<D, NW, 0, T::PC>(vbuf + (t & 1) * T::TILE, pf, o, lane);
                __builtin_amdgcn_sched_group_barrier(0x100, kVPrefetch, 0);
#pragma unroll
                for (int i = 0; i < T::DT * T::PC; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA (O += V^T P^T)
                    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // transposed V reads
                    __builtin_amdgcn_sched_group_barrier(0x002, kValuPerPvMfma, 0);  // second half of P
                    __builtin_amdgcn_sched_group_barrier(0x400, kExpPerMfma, 0);
                }
            } else if constexpr (D == 64) {
                // Each half of P is checked before its P V MFMAs: the first half was
                // formed under QK^T, the second is formed under the first half's P V.
                float l1 = (ps[0] + ps[1]) + (ps[2] + ps[3]);
                const bool bad1 = !(l1 < kTileSumLimit);
                if (__builtin_amdgcn_ballot_w64(bad1))
                    settle_part<D, NW, 0, T::PC / 2>(sc, pf, o, ms_run, l_run, l1, bad1, sl2);
                l_run += l1;
                float ps2[4] = {0.f, 0.f, 0.f, 0.f};
                exp_part<D, NW, T::PC / 2, T::PC>(sc, pf, ms_run, ps2, sl2);
                pv_part<D, NW, 0, T::PC / 2>(vbuf + (t & 1) * T::TILE, pf, o, lane);
                __builtin_amdgcn_sched_group_barrier(0x100, kVPrefetch, 0);
#pragma unroll
                for (int i = 0; i < T::DT * T::PC / 2; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA (first half of P V)
                    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // transposed V reads
                    __builtin_amdgcn_sched_group_barrier(0x002, 2 * kValuPerPvMfma, 0);  // second half of P
                    __builtin_amdgcn_sched_group_barrier(0x400, 2 * kExpPerMfma, 0);
                }
                float l2 = (ps2[0] + ps2[1]) + (ps2[2] + ps2[3]);
                const bool bad2 = !(l2 < kTileSumLimit);
                if (__builtin_amdgcn_ballot_w64(bad2))
                    settle_part<D, NW, T::PC / 2, T::PC>(sc, pf, o, ms_run, l_run, l2, bad2, sl2);
                l_run += l2;
                pv_part<D, NW, T::PC / 2, T::PC>(vbuf + (t & 1) * T::TILE, pf, o, lane);
                __builtin_amdgcn_sched_group_barrier(0x100, kVPrefetch, 0);
#pragma unroll
                for (int i = 0; i < T::DT * T::PC / 2; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA (second half of P V)
                    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // transposed V reads
                }
            } else {
                float l_tile = (ps[0] + ps[1]) + (ps[2] + ps[3]);
                const bool bad = !(l_tile < kTileSumLimit);
                if (__builtin_amdgcn_ballot_w64(bad))
                    settle_part<D, NW, 0, T::PC>(sc, pf, o, ms_run, l_run, l_tile, bad, sl2);
                l_run += l_tile;
                pv_part<D, NW, 0, T::PC>(vbuf + (t & 1) * T::TILE, pf, o, lane);
                __builtin_amdgcn_sched_group_barrier(0x100, kVPrefetch, 0);
#pragma unroll
                for (int i = 0; i < T::DT * T::PC; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA (O += V^T P^T)
                    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // transposed V reads
                }
            }
        }
        __builtin_amdgcn_s_setprio(0);
    };
    // Tiles 0 .. nkt-2 compute the next tile's S; the last tile's body has no
    // QK^T (nkt >= 1: every query tile has a key).
    const int um = min(kt_mask, nkt - 1);
    int t = 0;
    for (; t + 1 < um; t += 2) {
        body(t, sx, sy, std::false_type{}, std::false_type{});
        body(t + 1, sy, sx, std::false_type{}, std::false_type{});
    }
    if (t < um) {
        body(t, sx, sy, std::false_type{}, std::false_type{});
#pragma unroll
        for (int b = 0; b < T::KB; ++b) sx[b] = sy[b];
        ++t;
    }
    for (; t < nkt - 1; ++t) {
        body(t, sx, sy, std::true_type{}, std::false_type{});
#pragma unroll
        for (int b = 0; b < T::KB; ++b) sx[b] = sy[b];
    }
    if (t < kt_mask) body(t, sx, sy, std::false_type{}, std::true_type{});
    else body(t, sx, sy, std::true_type{}, std::true_type{});

    // O = O^T / l.  Lane holds query qrow, head dims 32t + 16hh + 8*half + i.
    const float l_tot = pair_sum(l_run);
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    if (qrow < n) {
        f16* orow = ob + (size_t)qrow * qs + half * 8;
#pragma unroll
        for (int t2 = 0; t2 < T::DT; ++t2)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                f16x8 v;
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] = (f16)(o[t2][hh * 8 + i] * inv);
                *reinterpret_cast<f16x8*>(orow + t2 * 32 + hh * 16) = v;
            }
    }
}

// One workgroup per (sequence, query head, query-tile unit).  Query head h
// reads kv head h / group.  Dense layout: q/o [B, Hq, N, D], k/v [B, Hkv, N, D].
// Packed layout (VARLEN): q/o [total, Hq, D], k/v [total, Hkv, D], sequence b
// being rows cu[b] .. cu[b+1]-1; the grid is sized for the longest sequence and
// the units past a shorter one exit before touching memory.
template <int D, bool CAUSAL, bool VARLEN, int NW>
__global__ void __launch_bounds__((PrefillTile<D, NW>::THREADS)) __attribute__((amdgpu_waves_per_eu(2)))
flash_prefill_kernel(const f16* __restrict__ Q, const f16* __restrict__ K, const f16* __restrict__ V,
                     f16* __restrict__ O, const int32_t* __restrict__ cu, int total_rows, int n_max,
                     int units_per_bh, int total_units, int hq, int group, float sl2, uint32_t qflip) {
    using T = PrefillTile<D, NW>;
    __shared__ __attribute__((aligned(1024))) f16 lds[2 * T::STAGE];
    // Dense: every (b, h) has the same units, so contiguous ranges per XCD are
    // balanced.  Varlen: the units past a short sequence are empty, so whole
    // GQA groups (all units of the query heads sharing a kv head) are dealt to
    // the XCDs round-robin instead.
    const int L = VARLEN ? xcd_chunk_remap((int)blockIdx.x, total_units, units_per_bh * group)
                         : xcd_remap((int)blockIdx.x, total_units);
    const int bh = L / units_per_bh, u = L % units_per_bh;
    const int b = bh / hq, h = bh - b * hq, hkv = hq / group, kvh = h / group;
    int n, qs, ks;
    size_t qbase, kvbase;
    if (VARLEN) {
        // Clamped into the tensors whatever the offsets hold: a bad cu gives a
        // wrong answer, never an access out of bounds.
        const int s0 = min(max(cu[b], 0), total_rows);
        n = min(max(cu[b + 1], s0), total_rows) - s0;
        qs = hq * D;
        ks = hkv * D;
        qbase = (size_t)s0 * qs + (size_t)h * D;
        kvbase = (size_t)s0 * ks + (size_t)kvh * D;
    } else {
        n = n_max;
        qs = ks = D;
        qbase = (size_t)bh * n * D;
        kvbase = ((size_t)b * hkv + kvh) * n * D;
    }
    const int nqt = (n + T::BM - 1) / T::BM;
    if (VARLEN && u >= (CAUSAL ? (nqt + 1) / 2 : nqt)) return;  // whole workgroup: past this sequence
    const f16 *Qb = Q + qbase, *Kb = K + kvbase, *Vb = V + kvbase;
    f16* Ob = O + qbase;
    if (CAUSAL) {
        // Pair the heaviest remaining tile with the lightest: equal work per workgroup.
        const int heavy = nqt - 1 - u;
        prefill_qtile<D, true, NW>(Qb, Kb, Vb, Ob, lds, heavy * T::BM, n, qs, ks, sl2, qflip);
        if (u != heavy) {
            __syncthreads();  // every wave is done with the buffers before they are refilled
            prefill_qtile<D, true, NW>(Qb, Kb, Vb, Ob, lds, u * T::BM, n, qs, ks, sl2, qflip);
        }
    } else {
        prefill_qtile<D, false, NW>(Qb, Kb, Vb, Ob, lds, u * T::BM, n, qs, ks, sl2, qflip);
    }
}

template <int D, bool CAUSAL, int NW>
static hipError_t launch_prefill_nw(const PrefillArgs& a) {
    using T = PrefillTile<D, NW>;
    const int nqt = (int)((a.n + T::BM - 1) / T::BM);  // a.n: the (longest) sequence length
    const int units = CAUSAL ? (nqt + 1) / 2 : nqt;
    const long long total = (long long)units * a.bh;
    if (total <= 0) return hipSuccess;
    const int group = (int)(a.hq / a.hkv);
    if (a.cu)
        hipLaunchKernelGGL((flash_prefill_kernel<D, CAUSAL, true, NW>), dim3((unsigned)total), dim3(T::THREADS), 0,
                           (hipStream_t)a.stream, (const f16*)a.q, (const f16*)a.k, (const f16*)a.v, (f16*)a.o,
                           a.cu, (int)a.total_rows, (int)a.n, units, (int)total, (int)a.hq, group, a.sl2, a.qflip);
    else
        hipLaunchKernelGGL((flash_prefill_kernel<D, CAUSAL, false, NW>), dim3((unsigned)total), dim3(T::THREADS), 0,
                           (hipStream_t)a.stream, (const f16*)a.q, (const f16*)a.k, (const f16*)a.v, (f16*)a.o,
                           a.cu, 0, (int)a.n, units, (int)total, (int)a.hq, group, a.sl2, a.qflip);
    return hipGetLastError();
}

// Workgroup size.  8 waves (256 rows) share each K/V tile among more rows and
// win on long sequences; 4 waves (128 rows, two workgroups per CU) halve the
// diagonal band a causal workgroup pays in full and double the workgroup count,
// which wins on short sequences and small grids.  Measured crossovers on
// MI355X: causal up to N = 2048 (+25% at 512, +5% at 2048, -4% at 8192),
// non-causal up to N = 1024 (+10% at 512, 0..+2% at 1024, -3..-6% beyond), and
// any grid of fewer 8-wave workgroups than half the CUs.
static int prefill_waves(int64_t n, bool causal, int64_t bh) {
    const int64_t nqt8 = (n + 255) / 256;
    const int64_t wg8 = (causal ? (nqt8 + 1) / 2 : nqt8) * bh;
    if (n <= (causal ? 2048 : 1024) || wg8 < 128) return 4;
    return 8;
}

template <int D, bool CAUSAL>
static hipError_t launch_prefill(const PrefillArgs& a) {
    return prefill_waves(a.n, CAUSAL, a.bh) == 4 ? launch_prefill_nw<D, CAUSAL, 4>(a)
                                                 : launch_prefill_nw<D, CAUSAL, 8>(a);
}

hipError_t prefill_launch(const PrefillArgs& a) {
    if (a.d == 64) return a.causal ? launch_prefill<64, true>(a) : launch_prefill<64, false>(a);
    return a.causal ? launch_prefill<128, true>(a) : launch_prefill<128, false>(a);
}

}  // namespace ak
