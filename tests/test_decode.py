"""Paged split-K decode parity on the GPU against the CPU oracle.

Mirrors the reference's suite (tests/test_decode.py:9-63: head groups x
contexts, ragged batch with 4 partitions, block sizes, long context, split
invariance, the gather+SDPA baseline) with the north-star tolerances, and adds
bit-exact page-gather checks and the full-size BASELINE decode configs.
"""
import numpy as np
import pytest
import torch

import attnkernels as ak
from attnkernels import reference as akref
import oracle
from conftest import TOL, max_err

pytestmark = pytest.mark.gpu


def cache(ctx, hkv, d, bs=16, extra=5, seed=0):
    kc, vc, bt, cl = oracle.make_paged_cache(ctx, hkv, d, block_size=bs, extra_blocks=extra, seed=seed)
    return kc, vc, bt, cl


def rand_q(b, hq, d, seed=1):
    return np.random.default_rng(seed).standard_normal((b, hq, d), dtype=np.float32).astype(np.float16)


def to_dev(*arrs):
    return [torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in arrs]


def run(ctx, hq, hkv, d, bs=16, partition=None, seed=0):
    kc, vc, bt, cl = cache(ctx, hkv, d, bs, seed=seed)
    q = rand_q(len(ctx), hq, d, seed + 1)
    qd, kcd, vcd, btd, cld = to_dev(q, kc, vc, bt, cl)
    out = ak.paged_decode(qd, kcd, vcd, btd, cld, max(ctx), partition_size=partition)
    torch.cuda.synchronize()
    ref = oracle.paged_decode_fp32(q, kc, vc, bt, cl)
    assert out.shape == qd.shape and out.dtype == torch.float16
    assert torch.isfinite(out).all()
    return max_err(out, ref)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("heads", [(8, 8), (8, 4), (32, 8), (16, 2)])
@pytest.mark.parametrize("ctx", [[1], [100], [256], [1000, 1000], [5000]])
def test_uniform(d, heads, ctx):
    assert run(ctx, heads[0], heads[1], d) < TOL[d]


RAGGED = [1, 17, 255, 256, 257, 999, 4097, 33]

# One long sequence among sequences of 0-17 tokens: at P = 256 its 36 splits
# go to the reduce kernel and all but the first of each short sequence's 36
# split workgroups are past its context, so they exit after loading its length
# (the page ids and q are loaded after that check); at P = 512 and 2048 the
# splits merge in the decode kernel.
SKEWED = [9000, 1, 3, 16, 1, 0, 2, 17, 1, 5]


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("heads", [(8, 8), (16, 8), (32, 8), (64, 8)])
@pytest.mark.parametrize("partition", [256, 512, 2048])
def test_skewed_batch_of_mostly_empty_splits(d, heads, partition):
    kc, vc, bt, cl = cache(SKEWED, heads[1], d, seed=41)
    q = rand_q(len(SKEWED), heads[0], d, 42)
    qd, kcd, vcd, btd, cld = to_dev(q, kc, vc, bt, cl)
    out = ak.paged_decode(qd, kcd, vcd, btd, cld, max(SKEWED), partition_size=partition)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    assert float(out[SKEWED.index(0)].abs().max()) == 0.0  # no context: a zero row
    live = [i for i, c in enumerate(SKEWED) if c > 0]
    ref = oracle.paged_decode_fp32(q[live], kc, vc, bt[live], cl[live])
    assert max_err(out[live], ref) < TOL[d]


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("partition", [None, 256, 1024, 1 << 20])
def test_ragged_batch(d, partition):
    """Different context lengths in one batch; partition 1<<20 means no split-K."""
    assert run(RAGGED, 32, 8, d, partition=partition) < TOL[d]


CHUNK_EDGES = [15, 16, 17, 31, 32, 33, 63, 65, 127, 129, 255, 257, 383, 385, 511, 513]


@pytest.mark.parametrize("d,hq,hkv", [(128, 16, 4), (128, 64, 8), (128, 8, 4), (64, 8, 4), (64, 32, 4),
                                      (64, 64, 8)])
@pytest.mark.parametrize("partition", [256, 512])
def test_chunk_edges_head_groups(d, hq, hkv, partition):
    """Context lengths one token either side of every chunk size the head-group
    kernel uses (16 tokens, one page, per wave; 64 per workgroup step) and of
    the splits; the whole-page loop hands the tail to the checked loop at each
    of them."""
    assert run(CHUNK_EDGES, hq, hkv, d, partition=partition) < TOL[d]


@pytest.mark.parametrize("bs", [8, 16, 32, 12])
@pytest.mark.parametrize("hq", [8, 16])
def test_block_sizes(bs, hq):
    """Four and eight query heads per kv head (the dot-product and the
    matrix-core kernels); pages of other than 16 tokens take the checked path."""
    assert run([300, 2000, 17], hq, 2, 128, bs=bs) < TOL[128]


def test_long_context_split():
    assert run([32768], 32, 8, 128) < TOL[128]


def test_split_choice_does_not_change_result():
    kc, vc, bt, cl = cache([6000, 3000], 4, 128, extra=0)
    q = rand_q(2, 16, 128)
    qd, kcd, vcd, btd, cld = to_dev(q, kc, vc, bt, cl)
    outs = [ak.paged_decode(qd, kcd, vcd, btd, cld, 6000, partition_size=p) for p in (256, 768, 2048, 6144)]
    for o in outs[1:]:
        assert max_err(o, outs[0]) < 2e-3


def test_torch_baseline_matches():
    """The gather + SDPA baseline kept in attnkernels.reference is itself correct
    (run in fp32 on the GPU, see the bf16/fp16 batched-GEMM caveat on this pool)."""
    ctx = [512, 512, 300]
    kc, vc, bt, cl = cache(ctx, 8, 128, extra=0)
    q = rand_q(3, 32, 128)
    qd, kcd, vcd, btd, cld = to_dev(q, kc, vc, bt, cl)
    out = akref.paged_decode_torch(qd.float(), kcd.float(), vcd.float(), btd, 32, context_lens=cld)
    assert max_err(out, oracle.paged_decode_fp32(q, kc, vc, bt, cl)) < TOL[128]


@pytest.mark.parametrize("d,hq,hkv", [(64, 4, 2), (128, 4, 4), (128, 16, 4), (64, 16, 2), (128, 16, 2)])
def test_scale_argument(d, hq, hkv):
    """Explicit scales on both kernels, including large ones (a nearly one-hot
    softmax: the per-wave reference maximum keeps moving) and negative ones."""
    kc, vc, bt, cl = cache([700, 40], hkv, d)
    q = rand_q(2, hq, d)
    qd, kcd, vcd, btd, cld = to_dev(q, kc, vc, bt, cl)
    for s in (0.5, -0.1, 0.0, 4.0, -30.0):
        out = ak.paged_decode(qd, kcd, vcd, btd, cld, 700, scale=s, partition_size=256)
        assert max_err(out, oracle.paged_decode_fp32(q, kc, vc, bt, cl, scale=s)) < TOL[d], s


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("hq", [4, 8, 16])
def test_rising_scores_move_the_reference_max(d, hq):
    """Scores shaped as a bump along the context (a triangle on one head dim,
    0 -> 24 -> 0 nats) move every wave's reference maximum several times on
    the way up, and one late key 6 nats above the peak moves it once more
    (it then carries about three quarters of the softmax, the bump the rest):
    each move rescales O and l of the heads in flight.  Two, four and eight
    query heads per kv head, split and unsplit."""
    lens, hkv = [3000, 777], 2
    kc, vc, bt, cl = cache(lens, hkv, d, seed=31)
    kc = kc.astype(np.float32)
    for b, n in enumerate(lens):
        t = np.arange(n)
        kc[bt[b, t // 16], :, t % 16, 0] = (6.0 * (1.0 - np.abs(2.0 * t / n - 1.0)))[:, None]
    kc[bt[0, 2900 // 16], :, 2900 % 16, 0] = 7.5
    kc = kc.astype(np.float16)
    q = (0.1 * np.random.default_rng(32).standard_normal((2, hq, d), dtype=np.float32)).astype(np.float16)
    q[..., 0] = 4.0
    qd, kcd, vcd, btd, cld = to_dev(q, kc, vc, bt, cl)
    ref = oracle.paged_decode_fp32(q, kc, vc, bt, cl, scale=1.0)
    for part in (256, 1 << 20):
        out = ak.paged_decode(qd, kcd, vcd, btd, cld, max(lens), scale=1.0, partition_size=part)
        assert max_err(out, ref) < TOL[d], part


def test_errors_match_reference():
    kc, vc, bt, cl = cache([300], 2, 128)
    qd, kcd, vcd, btd, cld = to_dev(rand_q(1, 6, 128), kc, vc, bt, cl)
    with pytest.raises(RuntimeError, match="multiple of num_kv_heads"):
        ak.load_extension().paged_decode(qd[:, :3].contiguous(), kcd, vcd, btd, cld, 300, 0.1, 256)
    with pytest.raises(RuntimeError, match="positive multiple of 256"):
        ak.load_extension().paged_decode(qd[:, :2].contiguous(), kcd, vcd, btd, cld, 300, 0.1, 100)
    with pytest.raises(RuntimeError, match=r"num_heads/num_kv_heads in \{1,2,4,8\}"):
        ak.load_extension().paged_decode(qd, kcd, vcd, btd, cld, 300, 0.1, 256)


# ------------------------------------------------ bit-exact page gathering --

@pytest.mark.parametrize("d,bs,group", [(128, 16, 1), (64, 8, 1), (128, 32, 1), (128, 16, 4), (128, 16, 2),
                                        (64, 16, 8), (128, 16, 8), (128, 32, 8)])
def test_gather_reads_exact_token(d, bs, group):
    """Each (sequence, kv head) attends to one chosen token only (its key gets a
    +64 score, every other key -64, scale 1): the output must be that token's V
    row, bit for bit, which proves the page/offset arithmetic for that token.
    With head groups (16-token pages) this runs the whole-page load path; every
    query head of a group must return its kv head's chosen row."""
    lens = [1, 16, 17, 255, 256, 513, 1000, 4095]
    hkv = 8
    kc, vc, bt, cl = cache(lens, hkv, d, bs, extra=7, seed=21)
    rng = np.random.default_rng(22)
    for trial in range(3):
        k2 = np.zeros_like(kc)
        k2[..., 0] = -8.0
        q = np.zeros((len(lens), hkv * group, d), np.float16)
        q[..., 0] = 8.0
        chosen = np.zeros((len(lens), hkv), np.int64)
        for b, c in enumerate(lens):
            for h in range(hkv):
                t = int(rng.integers(0, c)) if trial else [0, c - 1][h % 2]
                chosen[b, h] = t
                k2[bt[b, t // bs], h, t % bs, 0] = 8.0
        qd, kcd, vcd, btd, cld = to_dev(q, k2, vc, bt, cl)
        for part in (256, 1 << 20):
            out = ak.paged_decode(qd, kcd, vcd, btd, cld, max(lens), scale=1.0, partition_size=part)
            got = out.cpu().numpy()
            for b in range(len(lens)):
                for h in range(hkv * group):
                    t = chosen[b, h // group]
                    want = vc[bt[b, t // bs], h // group, t % bs]
                    assert np.array_equal(got[b, h], want), (trial, part, b, h, t)


def test_page_relabelling_is_bit_exact():
    """Moving pages to other physical slots and rewriting the table accordingly
    must give a bit-identical output: only the pages the table names are read."""
    lens = [1, 300, 2049, 77]
    kc, vc, bt, cl = cache(lens, 4, 128, extra=9, seed=31)
    q = rand_q(4, 8, 128, seed=32)
    perm = np.random.default_rng(33).permutation(kc.shape[0])
    inv = np.argsort(perm)
    kc2, vc2 = kc[perm], vc[perm]          # physical slot i now holds old page perm[i]
    bt2 = inv[bt].astype(np.int32)         # old page p lives at slot inv[p]
    for part in (256, 1024, 1 << 20):
        a = ak.paged_decode(*to_dev(q, kc, vc, bt, cl), max(lens), partition_size=part)
        b = ak.paged_decode(*to_dev(q, kc2, vc2, bt2, cl), max(lens), partition_size=part)
        assert torch.equal(a, b), part


@pytest.mark.parametrize("d,hq,hkv,ctx,bad,bad_id", [(64, 2, 2, 64, [1], 10 ** 6), (128, 8, 2, 600, [5, 21], 10 ** 6),
                                                      (64, 16, 2, 700, [0, 30], 10 ** 6), (128, 16, 2, 1000, [61], -3)])
def test_bad_page_ids_are_not_read(d, hq, hkv, ctx, bad, bad_id):
    """Out-of-range page ids (undefined in the reference; here past the pool or
    negative) are skipped, not read.  With head groups the bad pages sit inside
    whole-page chunks, which then hand over to the checked loads."""
    kc, vc, bt, cl = cache([ctx], hkv, d, extra=0, seed=41)
    bt_bad = bt.copy()
    bt_bad[0, bad] = bad_id
    q = rand_q(1, hq, d, seed=42)
    nblk = -(-ctx // 16)
    out = ak.paged_decode(*to_dev(q, kc, vc, bt_bad, cl), ctx, partition_size=256)
    keep = np.array([t for t in range(ctx) if t // 16 not in bad])
    kk = oracle.gather_kv(kc, bt, nblk)[0][:, keep]   # [Hkv, kept tokens, D]
    vv = oracle.gather_kv(vc, bt, nblk)[0][:, keep]
    g = hq // hkv
    ref = np.stack([oracle.attention_fp32(q[0, h][None], kk[h // g], vv[h // g])[0] for h in range(hq)])
    assert max_err(out[0], ref) < TOL[d]


def _ref_without_pages(q, kc, vc, bt, ctx, bad_pages, hq, hkv):
    """Oracle for one sequence whose tokens on ``bad_pages`` (table slots) are
    left out; a zero row when no token is left."""
    d = q.shape[-1]
    keep = np.array([t for t in range(ctx) if t // 16 not in bad_pages], dtype=np.int64)
    if keep.size == 0:
        return np.zeros((hq, d), np.float32)
    nblk = -(-ctx // 16)
    kk = oracle.gather_kv(kc, bt, nblk)[0][:, keep]
    vv = oracle.gather_kv(vc, bt, nblk)[0][:, keep]
    g = hq // hkv
    return np.stack([oracle.attention_fp32(q[h][None], kk[h // g], vv[h // g])[0] for h in range(hq)])


@pytest.mark.parametrize("d,hq,hkv", [(128, 8, 8), (128, 16, 4), (64, 8, 8), (64, 16, 2)])
@pytest.mark.parametrize("partition", [256, 1 << 20])
def test_bad_pages_cover_a_whole_split_or_sequence(d, hq, hkv, partition):
    """Every token of one 256-token split sits on out-of-range page ids
    (sequence 0, tokens 256..511), and every token of sequence 1: those tokens
    drop out of the softmax, the split with none left carries no weight in the
    merge, and the sequence with none left gets a zero row (no NaN)."""
    lens = [1000, 700, 300]
    kc, vc, bt, cl = cache(lens, hkv, d, extra=0, seed=43)
    bt_bad = bt.copy()
    bad0 = set(range(16, 32))
    bt_bad[0, sorted(bad0)] = 10 ** 6
    bt_bad[1, :] = -1
    q = rand_q(len(lens), hq, d, seed=44)
    out = ak.paged_decode(*to_dev(q, kc, vc, bt_bad, cl), max(lens), partition_size=partition)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    assert max_err(out[0], _ref_without_pages(q[0], kc, vc, bt[0:1], lens[0], bad0, hq, hkv)) < TOL[d]
    assert torch.count_nonzero(out[1]) == 0
    assert max_err(out[2:3], oracle.paged_decode_fp32(q[2:3], kc, vc, bt[2:3], cl[2:3])) < TOL[d]


# ---------------------------------------------------- BASELINE full sizes --

def baseline_cache(lens, hkv, d, bs, seed):
    """Pool = pages needed + 10% slack, pages by seeded permutation, fp16 N(0,1)
    caches generated on the device (seeded) and copied back for the oracle."""
    nblk = [-(-c // bs) for c in lens]
    total = sum(nblk)
    pool = -(-total * 11 // 10)
    rng = np.random.default_rng(seed)
    perm = rng.permutation(pool).astype(np.int32)
    bt = np.zeros((len(lens), max(nblk)), np.int32)
    pos = 0
    for b, nb in enumerate(nblk):
        bt[b, :nb] = perm[pos:pos + nb]
        pos += nb
    g = torch.Generator(device="cuda").manual_seed(seed)
    shape = (pool, hkv, bs, d)
    kcd = torch.randn(shape, generator=g, device="cuda", dtype=torch.float16)
    vcd = torch.randn(shape, generator=g, device="cuda", dtype=torch.float16)
    return kcd, vcd, bt, np.asarray(lens, np.int32)


def _check_rows(out, q, kcd, vcd, bt, cl, rows, d):
    for b in rows:
        pages = torch.from_numpy(bt[b]).long().cuda()
        kc_b = kcd[pages].cpu().numpy()   # the sequence's pages, in table order
        vc_b = vcd[pages].cpu().numpy()
        bt_b = np.arange(bt.shape[1], dtype=np.int32)[None]
        ref = oracle.paged_decode_fp32(q[b:b + 1], kc_b, vc_b, bt_b, cl[b:b + 1])
        assert max_err(out[b:b + 1], ref) < TOL[d], b


def _gpu_fp32_rows_err(out, qd, kcd, vcd, bt, cl, rows):
    """Max error of the given output rows against attention computed in float32
    on the GPU (pages gathered through the table, contiguous bmm operands):
    covers every row at full size, where the CPU oracle takes one sequence at a
    time; the oracle remains the checker on the sampled rows."""
    hkv, bs, d = kcd.shape[1], kcd.shape[2], kcd.shape[3]
    hq = qd.shape[1]
    worst = 0.0
    for b in rows:
        c = int(cl[b])
        nb = -(-c // bs)
        pages = torch.from_numpy(bt[b, :nb]).long().cuda()
        k = kcd[pages].permute(1, 0, 2, 3).reshape(hkv, nb * bs, d)[:, :c].float()
        v = vcd[pages].permute(1, 0, 2, 3).reshape(hkv, nb * bs, d)[:, :c].float().contiguous()
        q = qd[b].float().reshape(hkv, hq // hkv, d)
        s = torch.bmm(q, k.transpose(1, 2).contiguous()) * d ** -0.5
        ref = torch.bmm(torch.softmax(s, dim=-1), v).reshape(hq, d)
        worst = max(worst, (out[b].float() - ref).abs().max().item())
        del k, v, s
    return worst


def test_baseline_cfg4_ragged_64seqs():
    rng = np.random.default_rng(4)
    lens = rng.integers(1, 4097, size=64).tolist()
    kcd, vcd, bt, cl = baseline_cache(lens, 32, 128, 16, seed=4)
    q = rand_q(64, 32, 128, seed=5)
    qd, btd, cld = to_dev(q, bt, cl)
    out = ak.paged_decode(qd, kcd, vcd, btd, cld, max(lens), partition_size=512)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    _check_rows(out, q, kcd, vcd, bt, cl, list(range(0, 64, 4)) + [63], 128)
    assert _gpu_fp32_rows_err(out, qd, kcd, vcd, bt, cl, range(64)) < TOL[128]


@pytest.mark.parametrize("d", [128, 64])
def test_baseline_cfg5_long_context(d):
    lens = [32768] * 8
    kcd, vcd, bt, cl = baseline_cache(lens, 32, d, 16, seed=50 + d)
    q = rand_q(8, 32, d, seed=6)
    qd, btd, cld = to_dev(q, bt, cl)
    out = ak.paged_decode(qd, kcd, vcd, btd, cld, 32768, partition_size=256)
    torch.cuda.synchronize()
    _check_rows(out, q, kcd, vcd, bt, cl, [0, 7], d)
    assert _gpu_fp32_rows_err(out, qd, kcd, vcd, bt, cl, range(8)) < TOL[d]
    # every row: the 128-way split merge agrees with the unsplit kernel
    whole = ak.paged_decode(qd, kcd, vcd, btd, cld, 32768, partition_size=1 << 20)
    assert max_err(out, whole) < TOL[d]
    # every row: V = 1 gives exactly 1
    ones = torch.ones_like(vcd)
    o1 = ak.paged_decode(qd, kcd, ones, btd, cld, 32768, partition_size=256)
    assert (o1.float() - 1).abs().max().item() < 1e-3


@pytest.mark.parametrize("partition", [256, 4096])
def test_very_long_context_head_groups(partition):
    """256k and 100001 tokens, 4 query heads per kv head (the whole-page load
    path), 1024 / 64 splits into the reduce: kv heads 0 and 7 of both sequences
    against the oracle, gathered through the block table on the device."""
    lens, hq, hkv, d, bs = [262144, 100001], 32, 8, 128, 16
    kcd, vcd, bt, cl = baseline_cache(lens, hkv, d, bs, seed=51)
    q = rand_q(len(lens), hq, d, seed=52)
    qd, btd, cld = to_dev(q, bt, cl)
    out = ak.paged_decode(qd, kcd, vcd, btd, cld, max(lens), partition_size=partition)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    g = hq // hkv
    for b, c in enumerate(lens):
        pages = torch.from_numpy(bt[b, :-(-c // bs)]).long().cuda()
        for kvh in (0, hkv - 1):
            kk = kcd[pages, kvh].reshape(-1, d)[:c].cpu().numpy()
            vv = vcd[pages, kvh].reshape(-1, d)[:c].cpu().numpy()
            ref = oracle.attention_fp32(q[b, kvh * g:(kvh + 1) * g], kk, vv, False)
            assert max_err(out[b, kvh * g:(kvh + 1) * g], ref) < TOL[d], (b, kvh)


@pytest.mark.parametrize("partition", [256, 1 << 20])
def test_empty_context_gives_zero_rows(partition):
    """Context length 0 is outside the reference's contract (>= 1); here it
    yields a zero row with or without split-K, and the other sequences are
    unaffected."""
    lens = [0, 300, 0, 17]
    kc, vc, bt, cl = cache([max(c, 1) for c in lens], 2, 128, seed=61)
    cl = np.asarray(lens, np.int32)
    q = rand_q(4, 8, 128, seed=62)
    out = ak.paged_decode(*to_dev(q, kc, vc, bt, cl), 300, partition_size=partition)
    torch.cuda.synchronize()
    assert torch.count_nonzero(out[[0, 2]]) == 0
    for b in (1, 3):
        ref = oracle.paged_decode_fp32(q[b:b + 1], kc, vc, bt[b:b + 1], cl[b:b + 1])
        assert max_err(out[b:b + 1], ref) < TOL[128], b


@pytest.mark.parametrize("d,hq,hkv", [(128, 8, 4), (128, 32, 8), (128, 16, 2), (64, 32, 8), (64, 16, 2)])
def test_head_groups_repeatable_after_other_kernels(d, hq, hkv):
    """The grouped-query kernel exchanges values between lanes only through lane
    permutes; nothing it reads depends on what earlier kernels left in LDS or in
    the workspace.  Twelve calls, each after a prefill launch that fills LDS with
    other data, must give the same bits, all finite."""
    lens = [5000, 1, 700]
    kc, vc, bt, cl = cache(lens, hkv, d, seed=71)
    q = rand_q(len(lens), hq, d, seed=72)
    args = to_dev(q, kc, vc, bt, cl)
    g = torch.Generator(device="cuda").manual_seed(73)
    x = torch.randn(2, 8, 1024, d, generator=g, device="cuda", dtype=torch.float16) * 1e4
    first = None
    for i in range(12):
        ak.flash_attention(x, x, x, causal=bool(i % 2))
        out = ak.paged_decode(*args, max(lens), partition_size=256 if i % 3 else None)
        torch.cuda.synchronize()
        assert torch.isfinite(out).all(), i
        if first is None:
            first = out.clone()
            ref = oracle.paged_decode_fp32(q, kc, vc, bt, cl)
            assert max_err(out, ref) < TOL[d]
        elif i % 3:
            assert torch.equal(out, first) or max_err(out, ref) < TOL[d], i


@pytest.mark.parametrize("hq,d", [(32, 128), (64, 128), (32, 64)])
def test_grouped_query_layer_every_row(hq, d):
    """The bench's grouped-query decode layers (16 x 8192 tokens, 8 kv heads,
    4 or 8 query heads per kv head) at the default partition: every row against
    float32 attention on the GPU, sequence 0 against the oracle."""
    lens = [8192] * 16
    kcd, vcd, bt, cl = baseline_cache(lens, 8, d, 16, seed=81)
    q = rand_q(16, hq, d, seed=82)
    qd, btd, cld = to_dev(q, bt, cl)
    out = ak.paged_decode(qd, kcd, vcd, btd, cld, 8192)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    _check_rows(out, q, kcd, vcd, bt, cl, [0], d)
    assert _gpu_fp32_rows_err(out, qd, kcd, vcd, bt, cl, range(16)) < TOL[d]
