// Flash prefill on CDNA4 f16 MFMA (gfx950).
//
// One kernel serves the reference's three prefill entry points
// (naive_attn.cu:65-86, flash_simt.cu:209-221, flash_wmma.cu:241-257): same
// inputs, same online-softmax algorithm (flash_wmma.cu:114-194), same masking
// and guards, built for wave64 and the matrix core instead of warps.
//
// Layout choices
//   * A workgroup is 8 waves and owns BM = 256 query rows of one (batch, head);
//     each wave owns 32 of them, so no softmax row is shared between waves.
//     Eight waves share each K/V tile in LDS: half the LDS traffic per query
//     row of a 4-wave workgroup, and each wave issues only 2 one-KB loads per
//     K and per V tile.  Short sequences and small grids use 4-wave workgroups
//     (128 rows, two per CU; at D = 64 with 64-key tiles, three per CU)
//     instead: see prefill_waves.
//   * Two MFMA shapes, chosen per launch (prefill_mfma16): M = 32
//     (v_mfma_f32_32x32x16_f16) and M = 16 (v_mfma_f32_16x16x32_f16).  On
//     MI355X the 16x16 form costs less energy per FLOP: a matrix-core-only loop
//     at two waves per SIMD sustains 1.9-2.0 PFLOP/s on random fp16 data
//     against 1.2-1.6 for 32x32, and the D = 128 kernel runs at a 12% higher
//     clock with it.  It also issues twice the MFMA instructions, so it pays
//     only where the key loop is long: D = 128 with 8-wave workgroups, causal
//     N >= 6144 and non-causal N >= 3072.
//   * Scores are computed transposed, S^T = K Q^T, with K as the MFMA A operand
//     (16-byte LDS reads of K rows) and Q as the B operand (kept in VGPRs for
//     the whole kernel).
//       M = 32: a lane holds one query column and 16 keys per 32x32 block, so
//       the row max / sum are in-lane plus one exchange with lane l^32.
//       M = 16: a lane holds one query column and 4 keys per 16x16 block (lane
//       group g = lane / 16 holds keys 4g..4g+3); a lane owns two query rows
//       (one per 16-query block), each spread over the lanes l % 16 + 16 g.
//       Each K fragment feeds the two query blocks back to back.
//   * O^T = V^T P^T.  P^T comes straight from the S^T accumulators (converted
//     to f16, no LDS round trip), and the V^T operand is read from the
//     row-major V tile with ds_read_b64_tr_b16, which hands each lane 4
//     consecutive keys of one head dim; two such reads give the 8 keys whose P
//     the lane holds.
//       M = 32: accumulator rows 8c..8c+7 of a lane half are keys 16c +
//       {0..3, 8..11} (+4 for the upper half).  The head dims a lane reads are
//       permuted (bits 2/3 of d swapped) so that its O^T accumulators hold 8
//       contiguous head dims (16-byte output stores).
//       M = 16: for the 32-key step c, a lane's 8 B-operand elements are keys
//       32c + 16(i/4) + 4g + i%4; O^T accumulators hold 4 consecutive head dims
//       per 16-dim block (8-byte output stores).
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

template <int D, int NWAVES, int M>
struct PrefillTile {
    static_assert(M == 16 || M == 32, "MFMA shape");
    static constexpr int NW = NWAVES;            // waves per workgroup: 8, or 4 for short sequences
    static constexpr int THREADS = NW * kWave;   // 512 or 256
    static constexpr int QW = 32;                // query rows per wave
    static constexpr int QB = 32 / M;            // query blocks per wave (one per row a lane owns)
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
    static constexpr int KK = 512 / M;           // k (head dims or keys) per MFMA: 16 or 32
    static constexpr int KB = BN / M;            // key blocks of S^T
    static constexpr int DC = D / KK;            // k-steps of K Q^T
    static constexpr int DT = D / M;             // head-dim blocks of O^T
    static constexpr int PC = BN / KK;           // k-steps of V^T P^T
    static constexpr int NCH = 4 / QB;           // dot2 row-sum chains per row
    // Split P: D = 64 has twice the scores per MFMA of D = 128, so the key steps
    // past PC1 are exponentiated under the first half of P V instead of all
    // under QK^T.
    static constexpr bool SPLIT = D == 64;
    static constexpr int PC1 = SPLIT ? PC / 2 : PC;  // key steps whose P is formed under QK^T
    using Acc = std::conditional_t<M == 16, f32x4, f32x16>;
    static_assert(LPW >= 1 && LPW * NW * 1024 == TILE * 2, "the waves split each tile into whole KBs");
    static_assert(D % 32 == 0 && BN % 32 == 0, "tile shapes");
};

template <int D, int NW, int M>
using STile = typename PrefillTile<D, NW, M>::Acc[PrefillTile<D, NW, M>::KB][PrefillTile<D, NW, M>::QB];
template <int D, int NW, int M>
using OAcc = typename PrefillTile<D, NW, M>::Acc[PrefillTile<D, NW, M>::DT][PrefillTile<D, NW, M>::QB];
template <int D, int NW, int M>
using PFrag = f16x8[PrefillTile<D, NW, M>::PC][PrefillTile<D, NW, M>::QB];
template <int D, int NW, int M>
using QFrag = f16x8[PrefillTile<D, NW, M>::QB][PrefillTile<D, NW, M>::DC];

// Physical 16-byte chunk of logical chunk c in row r.  K: rows of one 256-byte
// bank line sequence get distinct chunks, so 16 lanes reading one logical
// chunk of 16 consecutive rows hit 16 different bank groups.  V: the
// transposed reads of one instruction take, per 16 lanes, 4 consecutive rows
// of 64 bytes (M = 32: the two 16-lane halves of a lane half read different
// 32-byte halves of them) or of 32 bytes (M = 16: the 16-lane groups read 4
// more rows each).  M = 32 gives groups of 4 consecutive rows disjoint 64-byte
// blocks; M = 16 XORs the chunk index with twice the row's index within 8
// bank lines, which puts the chunk pairs of 8 consecutive rows on 8 disjoint
// pairs of bank groups.
template <int D>
__device__ __forceinline__ int k_chunk(int r, int c) {
    constexpr int RPL = 128 / D, CPR = D / 8;
    return c ^ ((r / RPL) % CPR);
}
template <int D, int M>
__device__ __forceinline__ int v_chunk(int r, int c) {
    constexpr int RPL = 128 / D, CPR = D / 8;
    if constexpr (M == 16) return c ^ (2 * ((r / RPL) % (CPR / 2)));
    else return c ^ (4 * ((r / RPL) % (CPR / 4)));
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
//
// D = 128: a tile whose rows are all below n loads from a scalar base (the
// tile's first row) plus a 32-bit per-lane offset that is the same for every
// tile, so the address arithmetic is scalar; only a tile that crosses n takes
// the clamped per-lane 64-bit addresses.  Both issue LPW loads per wave.
// The branch splits a tile body into scheduling regions: the compiler then
// issues V(t+1) right after the next tile's QK^T MFMAs and this tile's
// exponentials after it, instead of interleaving them with those MFMAs.
// Measured on MI355X against per-lane addresses: non-causal N = 8192 +4-5%,
// causal N = 2048-8192 +0.4% to +2%; against the same scalar loads with the
// clamp folded into the offset (no branch, interleave kept) +1% to +4% at
// N >= 4096.  At D = 64 no gain, and the causal varlen kernel loses its third
// wave per SIMD to the extra registers, so D = 64 keeps the per-lane addresses.
template <int D, bool IS_V, int NW, int M>
__device__ __forceinline__ void load_kv(const f16* __restrict__ src, f16* dst, int k0, int n, int rs, int w,
                                        int lane) {
    using T = PrefillTile<D, NW, M>;
    if (D == 128 && k0 + T::BN <= n) {
        const f16* base = src + (size_t)k0 * rs;
#pragma unroll
        for (int j = 0; j < T::LPW; ++j) {
            const int blk = w * T::LPW + j;
            const int row = blk * T::RPI + lane / T::CPR, p = lane % T::CPR;
            const int c = IS_V ? v_chunk<D, M>(row, p) : k_chunk<D>(row, p);
            const uint32_t off = (uint32_t)(row * rs + c * 8) * (uint32_t)sizeof(f16);
            const uint32_t l = __builtin_amdgcn_readfirstlane((uint32_t)(size_t)(AK_LDS void*)(dst + blk * 512));
            // s_nop 4: five wait states, for an SGPR of `base` written by a
            // VALU instruction just before (the compiler restores spilled SGPRs
            // with v_readlane and cannot see the hazard inside this asm); they
            // also cover the M0 write.
            asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "{m0}"(l));
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < T::LPW; ++j) {
        const int blk = w * T::LPW + j;
        const int row = blk * T::RPI + lane / T::CPR, p = lane % T::CPR;
        const int c = IS_V ? v_chunk<D, M>(row, p) : k_chunk<D>(row, p);
        const f16* g = src + (size_t)min(k0 + row, n - 1) * rs + c * 8;
        const uint32_t l = __builtin_amdgcn_readfirstlane((uint32_t)(size_t)(AK_LDS void*)(dst + blk * 512));
        asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(l));
    }
}

__device__ __forceinline__ void wait_loads_and_sync() {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
}

// {own value, value of lane l^32} (v_permlane32_swap) or of lane l^16
// (v_permlane16_swap), in some order, by swapping two copies of x (no LDS
// traffic).  Issued as inline asm: with the builtin and identical inputs the
// compiler kept only one of the two swapped registers.  The s_nop covers the
// VALU-write -> permlane-read hazard.
template <int MASK>
__device__ __forceinline__ f32x2 pair_values(float x) {
    static_assert(MASK == 16 || MASK == 32, "permlane swap distance");
    float a = x, b = x;
    if constexpr (MASK == 32) asm volatile("s_nop 2\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    else asm volatile("s_nop 2\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    return f32x2{a, b};
}

// Maximum / sum over the lanes that share a query row: l and l^32 (M = 32),
// or the four lanes l % 16 + 16 g (M = 16).
template <int M>
__device__ __forceinline__ float row_max(float x) {
    if constexpr (M == 16) {
        const f32x2 v = pair_values<16>(x);
        x = fmaxf(v[0], v[1]);
    }
    const f32x2 v = pair_values<32>(x);
    return fmaxf(v[0], v[1]);
}
template <int M>
__device__ __forceinline__ float row_sum(float x) {
    if constexpr (M == 16) {
        const f32x2 v = pair_values<16>(x);
        x = v[0] + v[1];
    }
    const f32x2 v = pair_values<32>(x);
    return v[0] + v[1];
}

// Score register i of accumulator block (kb, qb): its key within the tile and
// its query within the wave's 32 rows.
template <int M>
__device__ __forceinline__ int score_key(int kb, int i, int lane) {
    if constexpr (M == 32) return kb * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
    else return kb * 16 + 4 * (lane >> 4) + i;
}
template <int M>
__device__ __forceinline__ int score_query(int qb, int lane) {
    if constexpr (M == 32) return lane & 31;
    else return qb * 16 + (lane & 15);
}

// Score register i of P^T k-step c (query block qb) in the S^T accumulators:
// M = 32 takes registers 8(c%2) + i of block c/2, M = 16 register i%4 of
// blocks 2c and 2c+1.
template <int D, int NW, int M>
__device__ __forceinline__ float p_score(const STile<D, NW, M>& s, int c, int qb, int i) {
    if constexpr (M == 32) return s[c >> 1][0][(c & 1) * 8 + i];
    else return s[2 * c + (i >> 2)][qb][i & 3];
}

// The subtracted row maximum only moves when the tile's maximum exceeds it by
// more than this many powers of two, so O is rescaled rarely.  Softmax is
// invariant to the value subtracted; P stays <= 2^8, exact enough in fp16.
constexpr float kRescaleSlack = 8.f;

// S^T = K Q^T for one key tile.
//   M = 32: KB blocks of 32 keys x 32 queries; lane reads key row 32b + l%32,
//   chunk 2dc + l/32.  D = 128: head-dim step outermost, so consecutive MFMAs
//   share the Q operand and write independent accumulators (+0.5-0.7% at
//   N = 8192, bit-identical); D = 64 was not faster that way.
//   M = 16: KB x 2 blocks of 16 keys x 16 queries; head-dim step outermost (8
//   MFMAs between two on one accumulator); each K fragment (lane: key row
//   16kb + l%16, logical chunk 4dc + l/16) feeds the two query blocks back to
//   back.
template <int D, int NW, int M>
__device__ __forceinline__ void qk_tile(const f16* __restrict__ ks, const QFrag<D, NW, M>& qf, STile<D, NW, M>& s,
                                        int lane) {
    using T = PrefillTile<D, NW, M>;
    if constexpr (M == 32) {
        const int col = lane & 31, half = lane >> 5;
#pragma unroll
        for (int b = 0; b < T::KB; ++b) s[b][0] = f32x16{};
        constexpr bool DC_OUTER = D == 128;
#pragma unroll
        for (int x = 0; x < T::KB * T::DC; ++x) {
            const int b = DC_OUTER ? x % T::KB : x / T::DC, dc = DC_OUTER ? x / T::KB : x % T::DC;
            const int r = b * 32 + col;
            s[b][0] = mfma32x32x16(*reinterpret_cast<const f16x8*>(ks + r * D + k_chunk<D>(r, 2 * dc + half) * 8),
                                   qf[0][dc], s[b][0]);
        }
    } else {
        const int c16 = lane & 15, g = lane >> 4;
#pragma unroll
        for (int kb = 0; kb < T::KB; ++kb)
#pragma unroll
            for (int qb = 0; qb < T::QB; ++qb) s[kb][qb] = f32x4{};
#pragma unroll
        for (int dc = 0; dc < T::DC; ++dc)
#pragma unroll
            for (int kb = 0; kb < T::KB; ++kb) {
                const int r = kb * 16 + c16;
                const f16x8 kf = *reinterpret_cast<const f16x8*>(ks + r * D + k_chunk<D>(r, 4 * dc + g) * 8);
#pragma unroll
                for (int qb = 0; qb < T::QB; ++qb) s[kb][qb] = mfma16x16x32(kf, qf[qb][dc], s[kb][qb]);
            }
    }
}

// Keys past n and, if causal, keys after the query -> -inf.
template <int D, int NW, int M, bool CAUSAL>
__device__ __forceinline__ void mask_tile(STile<D, NW, M>& s, int k0, int n, int qw0, int lane) {
    using T = PrefillTile<D, NW, M>;
    constexpr int R = M == 32 ? 16 : 4;  // registers per accumulator block
#pragma unroll
    for (int kb = 0; kb < T::KB; ++kb)
#pragma unroll
        for (int qb = 0; qb < T::QB; ++qb)
#pragma unroll
            for (int i = 0; i < R; ++i) {
                const int key = k0 + score_key<M>(kb, i, lane), qrow = qw0 + score_query<M>(qb, lane);
                if (key >= n || (CAUSAL && key > qrow)) s[kb][qb][i] = -INFINITY;
            }
}

// Softmax state of the rows a lane owns: the subtracted (scaled, base-2) row
// maximum m, starting at -inf, and the lane's share of the row sum l.
template <int QB>
struct RowState {
    float m[QB];
    float l[QB];
};

template <int D, int NW, int M>
__device__ __forceinline__ void move_max(RowState<PrefillTile<D, NW, M>::QB>& st, OAcc<D, NW, M>& o, int qb,
                                         float mnew) {
    using T = PrefillTile<D, NW, M>;
    const float alpha = exp2_fast(st.m[qb] - mnew);  // 0 on the first tile
    st.m[qb] = mnew;
    st.l[qb] *= alpha;
#pragma unroll
    for (int t = 0; t < T::DT; ++t) o[t][qb] *= alpha;
}

// Tile row maximum; moves the subtracted maximum (and rescales O and l) only
// when it grows by more than kRescaleSlack, which is rare after the first tile.
// Used on the diagonal (masked) tiles of causal D = 64 only.
template <int D, int NW, int M>
__device__ __forceinline__ void max_tile(const STile<D, NW, M>& s, OAcc<D, NW, M>& o,
                                         RowState<PrefillTile<D, NW, M>::QB>& st, float sl2) {
    using T = PrefillTile<D, NW, M>;
    constexpr int R = M == 32 ? 16 : 4;
    bool grow[T::QB], any = false;
    float mxs[T::QB];
#pragma unroll
    for (int qb = 0; qb < T::QB; ++qb) {
        float mx = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < T::KB; ++kb)
#pragma unroll
            for (int i = 0; i < R; ++i) mx = fmaxf(mx, s[kb][qb][i]);
        mxs[qb] = row_max<M>(mx) * sl2;                     // this tile's scaled row max (-inf if all masked)
        grow[qb] = mxs[qb] > st.m[qb] + kRescaleSlack;   // always true on the first tile
        any = any || grow[qb];
    }
    if (__builtin_amdgcn_ballot_w64(any)) {
#pragma unroll
        for (int qb = 0; qb < T::QB; ++qb)
            if (grow[qb]) move_max<D, NW, M>(st, o, qb, mxs[qb]);
    }
}

// P^T = 2^(S^T sl2 - m) as the fp16 B operand, for key steps [C0, C1) (see
// p_score).  The row sums are taken over the same fp16 values the MFMA
// consumes, two at a time by v_dot2_f32_f16 against (1, 1), in NCH chains per
// row.
template <int D, int NW, int M, int C0, int C1>
__device__ __forceinline__ void exp_part(const STile<D, NW, M>& s, PFrag<D, NW, M>& pf,
                                         const RowState<PrefillTile<D, NW, M>::QB>& st,
                                         float (&ps)[PrefillTile<D, NW, M>::QB][PrefillTile<D, NW, M>::NCH],
                                         float sl2) {
    using T = PrefillTile<D, NW, M>;
    const f16x2 ones = {(f16)1.f, (f16)1.f};
#pragma unroll
    for (int c = C0; c < C1; ++c)
#pragma unroll
        for (int qb = 0; qb < T::QB; ++qb) {
#pragma unroll
            for (int i = 0; i < 8; ++i)
                pf[c][qb][i] = (f16)exp2_fast(fmaf(p_score<D, NW, M>(s, c, qb, i), sl2, -st.m[qb]));
#pragma unroll
            for (int i = 0; i < 4; ++i)
                ps[qb][i % T::NCH] = __builtin_amdgcn_fdot2(f16x2{pf[c][qb][2 * i], pf[c][qb][2 * i + 1]}, ones,
                                                            ps[qb][i % T::NCH], false);
        }
}

// O^T += V^T P^T over key steps [C0, C1), key step outermost: the MFMAs of
// step c need only pf[c], so the exponentials of later steps can run under the
// MFMAs of earlier ones.
//   M = 32: in each 16-lane group, lane a points at row 16c + 8e + 4(l/32) +
//   a/4, head dims dbase + 4 sw(a%4) (sw swaps bits 0/1); lane i then
//   receives those 4 keys of head dim dbase + 4 sw(i/4) + i%4.
//   M = 16: in each 16-lane group g, lane a points at row 32c + 16e + 4g +
//   a/4, head dims 16t + 4(a%4) .. +3; lane i then receives keys 32c + 16e +
//   4g + 0..3 of head dim 16t + i.  Each V^T fragment feeds the two query
//   blocks back to back.
template <int D, int NW, int M, int C0, int C1>
__device__ __forceinline__ void pv_part(const f16* __restrict__ vs, const PFrag<D, NW, M>& pf, OAcc<D, NW, M>& o,
                                        int lane) {
    using T = PrefillTile<D, NW, M>;
    const int a = lane & 15;
#pragma unroll
    for (int c = C0; c < C1; ++c) {
#pragma unroll
        for (int t = 0; t < T::DT; ++t) {
            int dcol, r0;
            if constexpr (M == 32) {
                const int gd = (lane >> 4) & 1;
                dcol = t * 32 + 16 * gd + 4 * (((a & 1) << 1) | ((a >> 1) & 1));
                r0 = 16 * c + 4 * (lane >> 5) + (a >> 2);
            } else {
                dcol = t * 16 + 4 * (a & 3);
                r0 = 32 * c + 4 * (lane >> 4) + (a >> 2);
            }
            f16x4 lohi[2];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int r = r0 + e * (M == 32 ? 8 : 16);
                const f16* p = vs + r * D + v_chunk<D, M>(r, dcol >> 3) * 8 + (dcol & 7);
                lohi[e] = __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((AK_LDS s16x4*)p));
            }
            const f16x8 va = {lohi[0][0], lohi[0][1], lohi[0][2], lohi[0][3],
                              lohi[1][0], lohi[1][1], lohi[1][2], lohi[1][3]};
#pragma unroll
            for (int qb = 0; qb < T::QB; ++qb) {
                if constexpr (M == 32) o[t][qb] = mfma32x32x16(va, pf[c][qb], o[t][qb]);
                else o[t][qb] = mfma16x16x32(va, pf[c][qb], o[t][qb]);
            }
        }
    }
}

// Sum of a row's NCH dot2 chains: (c0 + c1) + (c2 + c3) for M = 32.
template <int NCH>
__device__ __forceinline__ float chain_sum(const float (&c)[NCH]) {
    if constexpr (NCH == 4) return (c[0] + c[1]) + (c[2] + c[3]);
    else return c[0] + c[1];
}

// Exponents checked after the fact instead of taking the tile maximum first:
// P = 2^(S sl2 - m) is computed against the current subtracted maximum m, and
// only if a lane's sum over key steps [C0, C1) reaches 2^14 (some P near the
// top of fp16) or is not finite (the first tile, against m = -inf) does the
// wave come here.  All lanes of each such row then move m to the maximum of
// those key steps, rescale O and l, and recompute P for them; rows that do not
// move recompute the same P.  D = 128 checks whole tiles; D = 64 checks each
// part of a tile before its P V MFMAs, and when the second part moves m the
// rescale also covers the first part's P V, already in O.  This saves the
// row-max pass (a max per score and a lane exchange per tile).
constexpr float kTileSumLimit = 16384.f;
template <int D, int NW, int M, int C0, int C1>
__device__ __forceinline__ void settle_part(const STile<D, NW, M>& s, PFrag<D, NW, M>& pf, OAcc<D, NW, M>& o,
                                            RowState<PrefillTile<D, NW, M>::QB>& st,
                                            float (&l_part)[PrefillTile<D, NW, M>::QB],
                                            const bool (&bad)[PrefillTile<D, NW, M>::QB], float sl2) {
    using T = PrefillTile<D, NW, M>;
#pragma unroll
    for (int qb = 0; qb < T::QB; ++qb) {
        float mx = -INFINITY;
#pragma unroll
        for (int c = C0; c < C1; ++c)
#pragma unroll
            for (int i = 0; i < 8; ++i) mx = fmaxf(mx, p_score<D, NW, M>(s, c, qb, i));
        const float mxs = row_max<M>(mx) * sl2;
        const bool move = row_max<M>(bad[qb] ? 1.f : 0.f) > 0.f && mxs > st.m[qb];
        if (move) move_max<D, NW, M>(st, o, qb, mxs);
    }
    float ps[T::QB][T::NCH] = {};
    exp_part<D, NW, M, C0, C1>(s, pf, st, ps, sl2);
#pragma unroll
    for (int qb = 0; qb < T::QB; ++qb) l_part[qb] = chain_sum<T::NCH>(ps[qb]);
}

// Instruction interleave of one pipelined tile (sched_group_barrier masks:
// 0x008 MFMA, 0x002 VALU, 0x400 transcendental, 0x100 LDS read).
//   M = 32: per MFMA of the next tile's S, 3 VALU ops and 2 exponentials of
//   this tile's P and the K read for a later MFMA.  At D = 64 each P V MFMA of
//   the tile's first half also takes 8 VALU ops and 4 exponentials of the
//   second half of P (max-first tiles: 4 and 2 over all P V MFMAs).
//   M = 16: each pair of QK^T MFMAs (one K fragment, two query blocks) takes an
//   equal share of this tile's P: two VALU ops (the FMA, half a conversion and
//   half a dot2) and one exponential per score.
// K reads run KPRE ahead, V reads VPRE (M = 16: 4 V^T fragments ahead, +3-4%
// against 2 at D = 128).
template <int D, int NW, int M>
struct PrefillSched {
    using T = PrefillTile<D, NW, M>;
    static constexpr int ceil_div(int a, int b) { return (a + b - 1) / b; }
    static constexpr int KPRE = 2;
    static constexpr int VPRE = M == 16 ? 8 : 4;
    static constexpr int NQK = T::KB * T::DC * T::QB;          // QK^T MFMAs per tile
    static constexpr int NPV = T::DT * T::PC * T::QB;          // P V MFMAs per tile
    static constexpr int VRD = M == 16 ? 1 : 2;                // transposed V reads per P V MFMA
    static constexpr int E1 = T::PC1 * T::QB * 8;              // scores exponentiated under QK^T
    static constexpr int QK_VALU = M == 16 ? ceil_div(4 * E1, NQK) : 3;   // per MFMA pair (16) / MFMA (32)
    static constexpr int QK_EXP = M == 16 ? ceil_div(2 * E1, NQK) : 2;
    static constexpr int E2 = (T::PC - T::PC1) * T::QB * 8;    // scores exponentiated under P V
    static constexpr int PV_VALU = M == 16 ? (E2 ? ceil_div(4 * E2, NPV) : 0) : 8;  // per first-half MFMA
    static constexpr int PV_EXP = M == 16 ? (E2 ? ceil_div(2 * E2, NPV) : 0) : 4;
    static constexpr int MF_VALU = M == 16 ? (E2 ? ceil_div(2 * E2, NPV) : 0) : 4;  // max-first, per MFMA
    static constexpr int MF_EXP = M == 16 ? (E2 ? ceil_div(E2, NPV) : 0) : 2;
};

// Software-pipelined key loop: iteration t multiplies the scores of tile t
// (computed one iteration earlier) into O while the matrix core computes the
// scores of tile t+1, so the exponentials of one tile overlap the QK^T MFMAs
// of the next inside every wave.  K runs two tiles ahead in a 2-buffer ring,
// V one tile ahead in another; one barrier per tile.
template <int D, bool CAUSAL, int NW, int M>
__device__ __forceinline__ void prefill_qtile(const f16* __restrict__ qsrc, const f16* __restrict__ kb,
                                              const f16* __restrict__ vb, f16* __restrict__ ob,
                                              f16* __restrict__ lds, int q0, int n, int qs, int ks, float sl2,
                                              uint32_t qflip) {
    using T = PrefillTile<D, NW, M>;
    using SC = PrefillSched<D, NW, M>;
    const int tid = threadIdx.x;
    const int lane = tid & 63, w = uniform(tid >> 6);
    const int qw0 = q0 + w * T::QW;
    f16* kbuf = lds;                 // 2 K tiles
    f16* vbuf = lds + 2 * T::TILE;   // 2 V tiles

    const int kend = CAUSAL ? min(n, q0 + T::BM) : n;
    const int nkt = (kend + T::BN - 1) / T::BN;
    // Tiles before kt_mask need no masking for any wave of the workgroup: all
    // their keys are < n and (causal) <= the workgroup's first query row.
    const int kt_mask = min(nkt, CAUSAL ? q0 / T::BN : n / T::BN);

    load_kv<D, false, NW, M>(kb, kbuf, 0, n, ks, w, lane);
    load_kv<D, true, NW, M>(vb, vbuf, 0, n, ks, w, lane);
    if (nkt > 1) load_kv<D, false, NW, M>(kb, kbuf + T::TILE, T::BN, n, ks, w, lane);

    // Q as the MFMA B operand: col = query, k = KK head dims per step.
    QFrag<D, NW, M> qf;
#pragma unroll
    for (int qb = 0; qb < T::QB; ++qb)
#pragma unroll
        for (int dc = 0; dc < T::DC; ++dc) {
            const int qrow = qw0 + score_query<M>(qb, lane);
            const int d0 = dc * T::KK + (M == 32 ? 8 * (lane >> 5) : 8 * (lane >> 4));
            // Rows past n are clamped to n-1: computed, never stored.
            f16x8 x = *reinterpret_cast<const f16x8*>(qsrc + (size_t)min(qrow, n - 1) * qs + d0);
            if (qflip) {  // negative scale: fold the sign into Q exactly
                x = __builtin_bit_cast(f16x8, __builtin_bit_cast(u32x4, x) ^ qflip);
            }
            qf[qb][dc] = x;
        }
    OAcc<D, NW, M> o;
#pragma unroll
    for (int t = 0; t < T::DT; ++t)
#pragma unroll
        for (int qb = 0; qb < T::QB; ++qb) o[t][qb] = typename T::Acc{};
    RowState<T::QB> st;
#pragma unroll
    for (int qb = 0; qb < T::QB; ++qb) {
        st.m[qb] = -INFINITY;  // the scaled row maxima subtracted so far
        st.l[qb] = 0.f;        // this lane's share of the row sums
    }

    wait_loads_and_sync();
    // S(t) alternates between sx and sy (loop unrolled by 2: no copies).
    STile<D, NW, M> sx, sy;
    qk_tile<D, NW, M>(kbuf, qf, sx, lane);

    // One tile: sc holds S(t); sn receives S(t+1), which the last tile skips.
    auto body = [&](int t, STile<D, NW, M>& sc, STile<D, NW, M>& sn, auto mask_tag, auto last_tag) {
        constexpr bool MASK = decltype(mask_tag)::value;
        constexpr bool LAST = decltype(last_tag)::value;  // the last tile: no next S to compute
        wait_loads_and_sync();  // K(t+1), V(t) landed; nobody reads K(t), V(t-1) any more
        if (t + 2 < nkt) load_kv<D, false, NW, M>(kb, kbuf + (t & 1) * T::TILE, (t + 2) * T::BN, n, ks, w, lane);
        // V(t+1) goes to the slot of V(t-1), last read before this barrier.  D = 64
        // issues it here; D = 128 after its QK^T phase, which spreads the CU's tile
        // loads over the tile (+1-2% at D = 128, -8-10% at D = 64).  Every body but
        // the last has a next tile (t + 1 < nkt), so the guard is compile-time: a
        // runtime branch after the QK^T phase let the compiler move the second
        // unrolled body's exponentials out of the QK^T interleave, below the branch.
        constexpr bool V_LATE = D == 128;
        if (!V_LATE && !LAST)
            load_kv<D, true, NW, M>(vb, vbuf + ((t + 1) & 1) * T::TILE, (t + 1) * T::BN, n, ks, w, lane);
        // Causal: a tile whose first key is after this wave's last row is skipped.
        const bool act = !MASK || !CAUSAL || t * T::BN <= qw0 + T::QW - 1;
        // The diagonal tiles of causal D = 64 take the tile's row maximum first; all
        // other tiles check the exponents after the fact (settle_part).
        // The split check on the masked tiles as well costs the causal D = 64 kernels
        // their register budget (spills at 8 waves, a third workgroup per CU at 4).
        constexpr bool MAX_FIRST = D == 64 && CAUSAL && MASK;
        if (act) {
            if constexpr (MASK) mask_tile<D, NW, M, CAUSAL>(sc, t * T::BN, n, qw0, lane);
            if constexpr (MAX_FIRST) max_tile<D, NW, M>(sc, o, st, sl2);
        }
        // The wave holds priority 1 while its QK^T MFMAs and exponentials run and
        // drops to 0 for P V and the max/barrier phase, so of the two waves on a
        // SIMD the one in the mixed MFMA+VALU phase issues first.  s_setprio ends
        // a scheduling region: each phase carries its own interleave.
        __builtin_amdgcn_s_setprio(1);
        if constexpr (!LAST) qk_tile<D, NW, M>(kbuf + ((t + 1) & 1) * T::TILE, qf, sn, lane);
        PFrag<D, NW, M> pf;
        float ps[T::QB][T::NCH] = {};
        if (act) {
            exp_part<D, NW, M, 0, T::PC1>(sc, pf, st, ps, sl2);
            if constexpr (!LAST) {
                __builtin_amdgcn_sched_group_barrier(0x100, SC::KPRE, 0);
                if constexpr (M == 32) {
#pragma unroll
                    for (int i = 0; i < SC::NQK; ++i) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA (S of the next tile)
                        __builtin_amdgcn_sched_group_barrier(0x002, SC::QK_VALU, 0);  // VALU (this tile's P)
                        __builtin_amdgcn_sched_group_barrier(0x400, SC::QK_EXP, 0);  // exp
                        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // next K fragment read
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < SC::NQK / 2; ++i) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA (S of the next tile)
                        __builtin_amdgcn_sched_group_barrier(0x002, SC::QK_VALU / 2, 0);  // VALU (this tile's P)
                        __builtin_amdgcn_sched_group_barrier(0x400, SC::QK_EXP / 2, 0);  // exp
                        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // next K fragment read
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA, same K fragment
                        __builtin_amdgcn_sched_group_barrier(0x002, SC::QK_VALU - SC::QK_VALU / 2, 0);
                        __builtin_amdgcn_sched_group_barrier(0x400, SC::QK_EXP - SC::QK_EXP / 2, 0);
                    }
                }
            }
        } else if constexpr (!LAST) {
            __builtin_amdgcn_sched_group_barrier(0x100, SC::KPRE, 0);
        }
        __builtin_amdgcn_s_setprio(0);
        if (V_LATE && !LAST)
            load_kv<D, true, NW, M>(vb, vbuf + ((t + 1) & 1) * T::TILE, (t + 1) * T::BN, n, ks, w, lane);
        if (act) {
            const f16* vt = vbuf + (t & 1) * T::TILE;
            if constexpr (MAX_FIRST) {
                exp_part<D, NW, M, T::PC1, T::PC>(sc, pf, st, ps, sl2);
#pragma unroll
                for (int qb = 0; qb < T::QB; ++qb) st.l[qb] += chain_sum<T::NCH>(ps[qb]);
                pv_part<D, NW, M, 0, T::PC>(vt, pf, o, lane);
                __builtin_amdgcn_sched_group_barrier(0x100, SC::VPRE, 0);
#pragma unroll
                for (int i = 0; i < SC::NPV; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA (O += V^T P^T)
                    __builtin_amdgcn_sched_group_barrier(0x100, SC::VRD, 0);  // transposed V reads
                    __builtin_amdgcn_sched_group_barrier(0x002, SC::MF_VALU, 0);  // second half of P
                    __builtin_amdgcn_sched_group_barrier(0x400, SC::MF_EXP, 0);
                }
            } else if constexpr (T::SPLIT) {
                // Each half of P is checked before its P V MFMAs: the first half was
                // formed under QK^T, the second is formed under the first half's P V.
                float l1[T::QB];
                bool bad1[T::QB], any1 = false;
#pragma unroll
                for (int qb = 0; qb < T::QB; ++qb) {
                    l1[qb] = chain_sum<T::NCH>(ps[qb]);
                    bad1[qb] = !(l1[qb] < kTileSumLimit);
                    any1 = any1 || bad1[qb];
                }
                if (__builtin_amdgcn_ballot_w64(any1)) settle_part<D, NW, M, 0, T::PC1>(sc, pf, o, st, l1, bad1, sl2);
#pragma unroll
                for (int qb = 0; qb < T::QB; ++qb) st.l[qb] += l1[qb];
                float ps2[T::QB][T::NCH] = {};
                exp_part<D, NW, M, T::PC1, T::PC>(sc, pf, st, ps2, sl2);
                pv_part<D, NW, M, 0, T::PC1>(vt, pf, o, lane);
                __builtin_amdgcn_sched_group_barrier(0x100, SC::VPRE, 0);
#pragma unroll
                for (int i = 0; i < SC::NPV / 2; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA (first half of P V)
                    __builtin_amdgcn_sched_group_barrier(0x100, SC::VRD, 0);  // transposed V reads
                    __builtin_amdgcn_sched_group_barrier(0x002, SC::PV_VALU, 0);  // second half of P
                    __builtin_amdgcn_sched_group_barrier(0x400, SC::PV_EXP, 0);
                }
                float l2[T::QB];
                bool bad2[T::QB], any2 = false;
#pragma unroll
                for (int qb = 0; qb < T::QB; ++qb) {
                    l2[qb] = chain_sum<T::NCH>(ps2[qb]);
                    bad2[qb] = !(l2[qb] < kTileSumLimit);
                    any2 = any2 || bad2[qb];
                }
                if (__builtin_amdgcn_ballot_w64(any2))
                    settle_part<D, NW, M, T::PC1, T::PC>(sc, pf, o, st, l2, bad2, sl2);
#pragma unroll
                for (int qb = 0; qb < T::QB; ++qb) st.l[qb] += l2[qb];
                pv_part<D, NW, M, T::PC1, T::PC>(vt, pf, o, lane);
                __builtin_amdgcn_sched_group_barrier(0x100, SC::VPRE, 0);
#pragma unroll
                for (int i = 0; i < SC::NPV / 2; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA (second half of P V)
                    __builtin_amdgcn_sched_group_barrier(0x100, SC::VRD, 0);  // transposed V reads
                }
            } else {
                float l_tile[T::QB];
                bool bad[T::QB], any = false;
#pragma unroll
                for (int qb = 0; qb < T::QB; ++qb) {
                    l_tile[qb] = chain_sum<T::NCH>(ps[qb]);
                    bad[qb] = !(l_tile[qb] < kTileSumLimit);
                    any = any || bad[qb];
                }
                if (__builtin_amdgcn_ballot_w64(any)) settle_part<D, NW, M, 0, T::PC>(sc, pf, o, st, l_tile, bad, sl2);
#pragma unroll
                for (int qb = 0; qb < T::QB; ++qb) st.l[qb] += l_tile[qb];
                pv_part<D, NW, M, 0, T::PC>(vt, pf, o, lane);
                __builtin_amdgcn_sched_group_barrier(0x100, SC::VPRE, 0);
#pragma unroll
                for (int i = 0; i < SC::NPV; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA (O += V^T P^T)
                    __builtin_amdgcn_sched_group_barrier(0x100, SC::VRD, 0);  // transposed V reads
                }
            }
        }
        __builtin_amdgcn_s_setprio(0);
    };
    // Tiles 0 .. nkt-2 compute the next tile's S; the last tile's body has no
    // QK^T (nkt >= 1: every query tile has a key).
    auto copy_s = [&]() {
#pragma unroll
        for (int kb2 = 0; kb2 < T::KB; ++kb2)
#pragma unroll
            for (int qb = 0; qb < T::QB; ++qb) sx[kb2][qb] = sy[kb2][qb];
    };
    const int um = min(kt_mask, nkt - 1);
    int t = 0;
    for (; t + 1 < um; t += 2) {
        body(t, sx, sy, std::false_type{}, std::false_type{});
        body(t + 1, sy, sx, std::false_type{}, std::false_type{});
    }
    if (t < um) {
        body(t, sx, sy, std::false_type{}, std::false_type{});
        copy_s();
        ++t;
    }
    for (; t < nkt - 1; ++t) {
        body(t, sx, sy, std::true_type{}, std::false_type{});
        copy_s();
    }
    if (t < kt_mask) body(t, sx, sy, std::false_type{}, std::true_type{});
    else body(t, sx, sy, std::true_type{}, std::true_type{});

    // O = O^T / l.
    //   M = 32: lane holds query l%32, head dims 32t + 16hh + 8(l/32) + i.
    //   M = 16: lane holds queries 16qb + l%16, head dims 16t + 4(l/16) + i.
#pragma unroll
    for (int qb = 0; qb < T::QB; ++qb) {
        const float l_tot = row_sum<M>(st.l[qb]);
        const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
        const int qrow = qw0 + score_query<M>(qb, lane);
        if (qrow < n) {
            if constexpr (M == 32) {
                f16* orow = ob + (size_t)qrow * qs + (lane >> 5) * 8;
#pragma unroll
                for (int t2 = 0; t2 < T::DT; ++t2)
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh) {
                        f16x8 v;
#pragma unroll
                        for (int i = 0; i < 8; ++i) v[i] = (f16)(o[t2][qb][hh * 8 + i] * inv);
                        *reinterpret_cast<f16x8*>(orow + t2 * 32 + hh * 16) = v;
                    }
            } else {
                f16* orow = ob + (size_t)qrow * qs + (lane >> 4) * 4;
#pragma unroll
                for (int t2 = 0; t2 < T::DT; ++t2) {
                    f16x4 v;
#pragma unroll
                    for (int i = 0; i < 4; ++i) v[i] = (f16)(o[t2][qb][i] * inv);
                    *reinterpret_cast<f16x4*>(orow + t2 * 16) = v;
                }
            }
        }
    }
}

// One workgroup per (sequence, query head, query-tile unit).  Query head h
// reads kv head h / group.  Dense layout: q/o [B, Hq, N, D], k/v [B, Hkv, N, D].
// Packed layout (VARLEN): q/o [total, Hq, D], k/v [total, Hkv, D], sequence b
// being rows cu[b] .. cu[b+1]-1; the grid is sized for the longest sequence and
// the units past a shorter one exit before touching memory.
template <int D, bool CAUSAL, bool VARLEN, int NW, int M>
__global__ void __launch_bounds__((PrefillTile<D, NW, M>::THREADS)) __attribute__((amdgpu_waves_per_eu(2)))
flash_prefill_kernel(const f16* __restrict__ Q, const f16* __restrict__ K, const f16* __restrict__ V,
                     f16* __restrict__ O, const int32_t* __restrict__ cu, int total_rows, int n_max,
                     int units_per_bh, int total_units, int hq, int group, float sl2, uint32_t qflip) {
    using T = PrefillTile<D, NW, M>;
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
        prefill_qtile<D, true, NW, M>(Qb, Kb, Vb, Ob, lds, heavy * T::BM, n, qs, ks, sl2, qflip);
        if (u != heavy) {
            __syncthreads();  // every wave is done with the buffers before they are refilled
            prefill_qtile<D, true, NW, M>(Qb, Kb, Vb, Ob, lds, u * T::BM, n, qs, ks, sl2, qflip);
        }
    } else {
        prefill_qtile<D, false, NW, M>(Qb, Kb, Vb, Ob, lds, u * T::BM, n, qs, ks, sl2, qflip);
    }
}

template <int D, bool CAUSAL, int NW, int M>
static hipError_t launch_prefill_nw(const PrefillArgs& a) {
    using T = PrefillTile<D, NW, M>;
    const int nqt = (int)((a.n + T::BM - 1) / T::BM);  // a.n: the (longest) sequence length
    const int units = CAUSAL ? (nqt + 1) / 2 : nqt;
    const long long total = (long long)units * a.bh;
    if (total <= 0) return hipSuccess;
    const int group = (int)(a.hq / a.hkv);
    if (a.cu)
        hipLaunchKernelGGL((flash_prefill_kernel<D, CAUSAL, true, NW, M>), dim3((unsigned)total), dim3(T::THREADS), 0,
                           (hipStream_t)a.stream, (const f16*)a.q, (const f16*)a.k, (const f16*)a.v, (f16*)a.o,
                           a.cu, (int)a.total_rows, (int)a.n, units, (int)total, (int)a.hq, group, a.sl2, a.qflip);
    else
        hipLaunchKernelGGL((flash_prefill_kernel<D, CAUSAL, false, NW, M>), dim3((unsigned)total), dim3(T::THREADS), 0,
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

// MFMA shape.  16x16x32 where the key loop is long enough for its lower energy
// per FLOP (a higher clock under the power limit) to outweigh its twice as
// many MFMA issues: D = 128, 8-wave workgroups, causal N >= 6144, non-causal
// N >= 3072.  Measured against 32x32x16 on one box at a time: causal N = 8192
// +0% to +4%, non-causal N = 4096 +4.5% to +6.7%, N = 3072 +1%, N = 2048 even;
// causal N = 3072-4096 -4% to -7%, the 4-wave kernels -6% to -9%, and D = 64
// -3% to -11% (its two exponentials per 32x32 MFMA leave no issue slots for
// the extra MFMA instructions).
static bool prefill_mfma16(int64_t n, int d, int nw, bool causal) {
    return d == 128 && nw == 8 && n >= (causal ? 6144 : 3072);
}

template <int D, bool CAUSAL>
static hipError_t launch_prefill(const PrefillArgs& a) {
    if (prefill_waves(a.n, CAUSAL, a.bh) == 4) return launch_prefill_nw<D, CAUSAL, 4, 32>(a);
    if constexpr (D == 128) {
        if (prefill_mfma16(a.n, D, 8, CAUSAL)) return launch_prefill_nw<D, CAUSAL, 8, 16>(a);
    }
    return launch_prefill_nw<D, CAUSAL, 8, 32>(a);
}

hipError_t prefill_launch(const PrefillArgs& a) {
    if (a.d == 64) return a.causal ? launch_prefill<64, true>(a) : launch_prefill<64, false>(a);
    return a.causal ? launch_prefill<128, true>(a) : launch_prefill<128, false>(a);
}

}  // namespace ak
