"""Pins of the CPU oracle (oracle/attention.py) -- runs without a GPU.

Each oracle function is checked against something that is not a retyping of
its own formula:
  * the float64 brute force written independently in C (oracle/attn_f64.c),
  * closed forms (N = 1, uniform scores, causal row 0),
  * torch's CPU attention routine in float64,
  * invariances (key permutation, split-K partition choice, page relabelling),
  * the decode_partition values recorded in the reference's own T4 run.
Planted mistakes (mutants of the oracle, built here on the CPU) must fail
those checks, so a dropped term, a wrong mask or index is caught.
"""
import json
import math
from pathlib import Path

import numpy as np
import pytest

import oracle
from oracle import f64

GOLDEN = Path(__file__).resolve().parent / "golden"
RNG = np.random.default_rng(1234)


def rand(*shape, scale=1.0, seed=None):
    r = RNG if seed is None else np.random.default_rng(seed)
    return (r.standard_normal(shape) * scale).astype(np.float16)


# ------------------------------------------------------------------ prefill --

@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("n,d", [(1, 64), (5, 64), (17, 128), (64, 64), (33, 128)])
@pytest.mark.parametrize("scale", [None, 0.3, -0.2, 0.0])
def test_attention_matches_f64_bruteforce(causal, n, d, scale):
    q, k, v = rand(2, 3, n, d), rand(2, 3, n, d), rand(2, 3, n, d)
    got = oracle.attention_fp32(q, k, v, causal, scale)
    want = f64.attention_f64(q, k, v, causal, scale)
    assert got.dtype == np.float32 and got.shape == q.shape
    assert np.abs(got - want).max() < 5e-6


def test_attention_single_token_is_v():
    q, k, v = rand(1, 2, 1, 64), rand(1, 2, 1, 64), rand(1, 2, 1, 64)
    for causal in (False, True):
        assert np.array_equal(oracle.attention_fp32(q, k, v, causal), v.astype(np.float32))


def test_attention_uniform_scores_give_means():
    n, d = 40, 64
    q = np.zeros((1, 1, n, d), np.float16)
    k, v = rand(1, 1, n, d), rand(1, 1, n, d)
    vf = v.astype(np.float64)[0, 0]
    full = oracle.attention_fp32(q, k, v, False)[0, 0]
    assert np.abs(full - vf.mean(axis=0)[None]).max() < 1e-6
    causal = oracle.attention_fp32(q, k, v, True)[0, 0]
    running = np.cumsum(vf, axis=0) / np.arange(1, n + 1)[:, None]
    assert np.abs(causal - running).max() < 1e-6


def test_causal_first_row_is_v0():
    q, k, v = rand(1, 1, 128, 64), rand(1, 1, 128, 64), rand(1, 1, 128, 64)
    out = oracle.attention_fp32(q, k, v, True)
    assert np.array_equal(out[0, 0, 0], v[0, 0, 0].astype(np.float32))


def test_attention_matches_torch_cpu_sdpa():
    torch = pytest.importorskip("torch")
    q, k, v = rand(2, 2, 70, 128), rand(2, 2, 70, 128), rand(2, 2, 70, 128)
    for causal in (False, True):
        t = [torch.from_numpy(x.astype(np.float64)) for x in (q, k, v)]
        want = torch.nn.functional.scaled_dot_product_attention(*t, is_causal=causal).numpy()
        assert np.abs(oracle.attention_fp32(q, k, v, causal) - want).max() < 5e-6


def test_noncausal_key_permutation_invariance():
    q, k, v = rand(1, 2, 50, 64), rand(1, 2, 50, 64), rand(1, 2, 50, 64)
    perm = np.random.default_rng(7).permutation(50)
    a = oracle.attention_fp32(q, k, v)
    b = oracle.attention_fp32(q, k[:, :, perm], v[:, :, perm])
    assert np.abs(a - b).max() < 1e-6


def _mutant_attention(kind):
    def fn(q, k, v, causal=False, scale=None):
        q, k, v = (x.astype(np.float32) for x in (q, k, v))
        n, d = q.shape[-2], q.shape[-1]
        scale = 1.0 / math.sqrt(d) if scale is None else scale
        s = q @ np.swapaxes(k, -1, -2)
        if kind != "no_scale":
            s = s * scale
        if causal:
            diag = 0 if kind == "mask_diagonal" else 1
            mask = np.triu(np.ones((n, n), bool), diag)
            if kind == "mask_transposed":
                mask = mask.T
            s = np.where(mask, -np.inf, s)
        axis = -2 if kind == "softmax_axis" else -1
        s = s - s.max(axis=axis, keepdims=True)
        p = np.exp(s)
        p = p / p.sum(axis=axis, keepdims=True)
        p = np.nan_to_num(p)
        return p @ v
    return fn


@pytest.mark.parametrize("kind", ["no_scale", "mask_diagonal", "mask_transposed", "softmax_axis"])
def test_planted_prefill_mistakes_are_caught(kind):
    q, k, v = rand(1, 2, 24, 64), rand(1, 2, 24, 64), rand(1, 2, 24, 64)
    want = f64.attention_f64(q, k, v, True)
    bad = _mutant_attention(kind)(q, k, v, True)
    assert np.abs(bad - want).max() > 1e-2


# ------------------------------------------------------------------- decode --

def _cache(lens, hkv, d, bs=16, extra=5, seed=0):
    return oracle.make_paged_cache(lens, hkv, d, block_size=bs, extra_blocks=extra, seed=seed)


@pytest.mark.parametrize("hq,hkv", [(8, 8), (8, 4), (32, 8), (16, 2)])
@pytest.mark.parametrize("bs", [8, 16, 32])
@pytest.mark.parametrize("d", [64, 128])
def test_paged_decode_matches_f64_bruteforce(hq, hkv, bs, d):
    lens = [1, 17, 255, 257, 40]
    kc, vc, bt, cl = _cache(lens, hkv, d, bs)
    q = rand(len(lens), hq, d)
    got = oracle.paged_decode_fp32(q, kc, vc, bt, cl)
    want = f64.paged_decode_f64(q, kc, vc, bt, cl)
    assert np.abs(got - want).max() < 5e-6


def test_paged_decode_equals_contiguous_attention():
    lens = [300, 77]
    kc, vc, bt, cl = _cache(lens, 2, 128, 16)
    q = rand(2, 8, 128)
    got = oracle.paged_decode_fp32(q, kc, vc, bt, cl)
    for b, c in enumerate(lens):
        nb = -(-c // 16)
        kk = oracle.gather_kv(kc, bt[b:b + 1], nb)[0, :, :c]
        vv = oracle.gather_kv(vc, bt[b:b + 1], nb)[0, :, :c]
        for h in range(8):
            ref = oracle.attention_fp32(q[b, h][None], kk[h // 4], vv[h // 4])[0]
            assert np.abs(got[b, h] - ref).max() < 1e-6


def test_gather_follows_page_table():
    """Token t of sequence b is cache[bt[b, t // bs], :, t % bs] -- checked on
    values that encode (page, offset), against explicit index arithmetic."""
    pool, hkv, bs, d = 12, 2, 8, 64
    cache = np.zeros((pool, hkv, bs, d), np.float32)
    cache[..., 0] = np.arange(pool)[:, None, None]
    cache[..., 1] = np.arange(bs)[None, None, :]
    cache[..., 2] = np.arange(hkv)[None, :, None]
    bt = np.array([[5, 0, 11], [3, 7, 2]], np.int32)
    g = oracle.gather_kv(cache, bt, 3)
    for b in range(2):
        for h in range(hkv):
            for t in range(24):
                assert tuple(g[b, h, t, :3]) == (bt[b, t // bs], t % bs, h)


@pytest.mark.parametrize("partition", [256, 768, 1024, 1 << 20])
def test_split_k_merge_equals_single_pass(partition):
    lens = [1, 255, 256, 257, 999, 2100]
    kc, vc, bt, cl = _cache(lens, 2, 64, 16)
    q = rand(len(lens), 8, 64)
    full = oracle.paged_decode_fp32(q, kc, vc, bt, cl)
    split = oracle.paged_decode_splitk(q, kc, vc, bt, cl, max(lens), partition)
    assert np.abs(full - split).max() < 2e-6


def test_partials_of_single_split_are_plain_softmax():
    lens = [100]
    kc, vc, bt, cl = _cache(lens, 1, 64, 16)
    q = rand(1, 1, 64)
    m, l, o = oracle.split_partials(q, kc, vc, bt, cl, 256, 1)
    kk = oracle.gather_kv(kc, bt, 7)[0, 0, :100].astype(np.float64)
    x = (q[0, 0].astype(np.float64) / 8.0 * oracle.LOG2E) @ kk.T
    assert abs(m[0, 0, 0] - x.max()) < 1e-5
    assert abs(l[0, 0, 0] - np.exp2(x - x.max()).sum()) < 1e-4


def _mutant_decode(kind):
    def fn(q, kc, vc, bt, cl):
        q = q.astype(np.float32)
        B, H, D = q.shape
        hkv, bs = kc.shape[1], kc.shape[2]
        g = H // hkv
        out = np.empty((B, H, D), np.float32)
        for b in range(B):
            c = int(cl[b])
            for h in range(H):
                kvh = h % hkv if kind == "head_modulo" else h // g
                toks = range(c)
                rows_k, rows_v = [], []
                for t in toks:
                    off = (bs - 1 - t % bs) if kind == "offset_reversed" else t % bs
                    rows_k.append(kc[bt[b, t // bs], kvh, off])
                    rows_v.append(vc[bt[b, t // bs], kvh, off])
                kk, vv = np.array(rows_k, np.float32), np.array(rows_v, np.float32)
                s = kk @ q[b, h] / math.sqrt(D)
                p = np.exp(s - s.max())
                out[b, h] = p @ vv / p.sum()
        return out
    return fn


@pytest.mark.parametrize("kind", ["head_modulo", "offset_reversed"])
def test_planted_decode_mistakes_are_caught(kind):
    lens = [37, 64]
    kc, vc, bt, cl = _cache(lens, 2, 64, 8)
    q = rand(2, 8, 64)
    want = f64.paged_decode_f64(q, kc, vc, bt, cl)
    assert np.abs(_mutant_decode("none")(q, kc, vc, bt, cl) - want).max() < 5e-6
    assert np.abs(_mutant_decode(kind)(q, kc, vc, bt, cl) - want).max() > 1e-2


def test_planted_merge_without_sums_is_caught():
    lens = [700, 1500]
    kc, vc, bt, cl = _cache(lens, 1, 64, 16)
    q = rand(2, 1, 64)
    m, l, o = oracle.split_partials(q, kc, vc, bt, cl, 256, 6)
    good = oracle.merge_partials(m, l, o, cl, 256)
    bad = oracle.merge_partials(m, np.ones_like(l), o, cl, 256)
    want = f64.paged_decode_f64(q, kc, vc, bt, cl)
    assert np.abs(good - want).max() < 5e-6
    assert np.abs(bad - want).max() > 1e-3


def test_make_paged_cache_structure():
    lens = [1, 16, 17, 100]
    kc, vc, bt, cl = oracle.make_paged_cache(lens, 2, 64, block_size=16, extra_blocks=3, seed=3)
    nblk = [1, 1, 2, 7]
    assert kc.shape == (sum(nblk) + 3, 2, 16, 64) and kc.dtype == np.float16
    used = np.concatenate([bt[b, :nb] for b, nb in enumerate(nblk)])
    assert len(set(used.tolist())) == len(used)            # each page handed out once
    assert all((bt[b, nb:] == 0).all() for b, nb in enumerate(nblk))  # unused slots: page 0
    assert bt.dtype == np.int32 and list(cl) == lens


# --------------------------------------------------------- decode_partition --

def test_decode_partition_matches_reference_t4_run():
    fx = json.loads((GOLDEN / "decode_partition_t4.json").read_text())
    assert len(fx["rows"]) == 23
    for r in fx["rows"]:
        p = oracle.decode_partition(r["batch"], r["num_kv_heads"], r["max_context_len"],
                                    fx["sm_count"])
        assert p == r["partition"], r
        assert -(-r["max_context_len"] // p) == r["splits"], r


def test_round_partition():
    assert [oracle.round_partition(p) for p in (1, 256, 257, 768, 1 << 20)] == \
        [256, 256, 512, 768, 1 << 20]


def test_workload_conventions():
    assert oracle.prefill_flops(2, 32, 8192, 128, True) == pytest.approx(1.0995e12, rel=1e-4)
    assert oracle.prefill_flops(4, 16, 2048, 64, False) == pytest.approx(6.872e10, rel=1e-3)
    assert oracle.decode_kv_bytes([32768] * 8, 32, 128) == 4294967296


# ------------------------------------------------------- paged cache writer --

def _write_loop(key, value, kc, vc, slots):
    """Element-by-element restatement: cache[slot // bs, h, slot % bs, d] = key[t, h, d]."""
    kc, vc = kc.copy(), vc.copy()
    nb, hkv, bs, d = kc.shape
    for t, s in enumerate(slots):
        if 0 <= s < nb * bs:
            for h in range(hkv):
                for j in range(d):
                    kc[s // bs, h, s % bs, j] = key[t, h, j]
                    vc[s // bs, h, s % bs, j] = value[t, h, j]
    return kc, vc


def test_append_slots_known_answers():
    bt = np.array([[7, 3, 9], [2, 5, 0]], np.int32)
    assert oracle.append_slots(bt, [0, 17], 16).tolist() == [7 * 16, 5 * 16 + 1]
    assert oracle.append_slots(bt, [47, -1], 16).tolist() == [9 * 16 + 15, -1]


@pytest.mark.parametrize("dtype", [np.float16, np.uint16])  # uint16 stands in for raw bf16 bits
def test_reshape_and_cache_equals_elementwise_loop(dtype):
    r = np.random.default_rng(3)
    kc = r.integers(0, 60000, (6, 2, 4, 8)).astype(np.uint16).view(dtype)
    vc = r.integers(0, 60000, (6, 2, 4, 8)).astype(np.uint16).view(dtype)
    key = r.integers(0, 60000, (5, 2, 8)).astype(np.uint16).view(dtype)
    value = r.integers(0, 60000, (5, 2, 8)).astype(np.uint16).view(dtype)
    slots = np.array([3, -1, 23, 24, 9], np.int64)  # 24 = past the pool of 6 * 4 slots
    got_k, got_v = oracle.reshape_and_cache(key, value, kc, vc, slots)
    want_k, want_v = _write_loop(key, value, kc, vc, slots)
    assert got_k.view(np.uint16).tolist() == want_k.view(np.uint16).tolist()
    assert got_v.view(np.uint16).tolist() == want_v.view(np.uint16).tolist()
    assert got_k.dtype == dtype


def test_reshape_and_cache_round_trip_through_gather():
    """Appending every token of every sequence through its block table, then
    gathering the pages, gives the tokens back in order (reference.py:47-51)."""
    lens = [37, 5, 16]
    kc0, vc0, bt, _ = oracle.make_paged_cache(lens, 3, 16, block_size=8, seed=4)
    r = np.random.default_rng(5)
    toks = [r.standard_normal((c, 3, 16)).astype(np.float16) for c in lens]
    kc, vc = np.zeros_like(kc0), np.zeros_like(vc0)
    for b, c in enumerate(lens):
        slots = oracle.append_slots(np.repeat(bt[b:b + 1], c, 0), np.arange(c), 8)
        kc, vc = oracle.reshape_and_cache(toks[b], -toks[b], kc, vc, slots)
    nb = bt.shape[1]
    for b, c in enumerate(lens):
        got = oracle.gather_kv(kc, bt[b:b + 1], nb)[0][:, :c]       # [Hkv, c, D]
        assert np.array_equal(got, toks[b].transpose(1, 0, 2))
        assert np.array_equal(oracle.gather_kv(vc, bt[b:b + 1], nb)[0][:, :c], -toks[b].transpose(1, 0, 2))


def test_planted_writer_mistake_is_caught():
    """Page and row swapped (slot % bs as the page): the round trip fails."""
    lens = [20]
    kc0, _, bt, _ = oracle.make_paged_cache(lens, 2, 8, block_size=4, seed=6)
    toks = np.random.default_rng(7).standard_normal((20, 2, 8)).astype(np.float16)
    slots = oracle.append_slots(np.repeat(bt, 20, 0), np.arange(20), 4)
    bad = np.zeros_like(kc0)
    nb_pool = bad.shape[0]
    for t, s in enumerate(slots):
        page, row = s % 4, (s // 4) % 4
        if page < nb_pool:
            bad[page, :, row, :] = toks[t]
    got = oracle.gather_kv(bad, bt, bt.shape[1])[0][:, :20]
    assert not np.array_equal(got, toks.transpose(1, 0, 2))


# ------------------------------------------------------- GQA / varlen prefill --

@pytest.mark.parametrize("h,hkv", [(4, 4), (8, 2), (6, 1)])
@pytest.mark.parametrize("causal", [False, True])
def test_gqa_matches_f64_per_head(h, hkv, causal):
    q, k, v = rand(2, h, 19, 64), rand(2, hkv, 19, 64), rand(2, hkv, 19, 64)
    got = oracle.attention_gqa(q, k, v, causal)
    for head in range(h):
        want = f64.attention_f64(q[:, head], k[:, head // (h // hkv)], v[:, head // (h // hkv)], causal, None)
        assert np.abs(got[:, head] - want).max() < 2e-5


def test_planted_gqa_head_map_is_caught():
    """kv head h % H_kv instead of h // G: different for G > 1."""
    q, k, v = rand(1, 8, 11, 64), rand(1, 2, 11, 64), rand(1, 2, 11, 64)
    bad = oracle.attention_fp32(q, k[:, [h % 2 for h in range(8)]], v[:, [h % 2 for h in range(8)]], False)
    assert np.abs(bad - oracle.attention_gqa(q, k, v, False)).max() > 1e-2


def test_varlen_single_sequence_equals_dense():
    q, k, v = rand(40, 4, 64), rand(40, 2, 64), rand(40, 2, 64)
    got = oracle.attention_varlen(q, k, v, [0, 40], True)
    dense = oracle.attention_gqa(q.transpose(1, 0, 2), k.transpose(1, 0, 2), v.transpose(1, 0, 2), True)
    assert np.array_equal(got, dense.transpose(1, 0, 2))


@pytest.mark.parametrize("causal", [False, True])
def test_varlen_matches_f64_per_sequence(causal):
    cu = [0, 1, 18, 18, 50]  # includes an empty sequence
    q, k, v = rand(50, 2, 128), rand(50, 2, 128), rand(50, 2, 128)
    got = oracle.attention_varlen(q, k, v, cu, causal)
    for b in range(4):
        s0, s1 = cu[b], cu[b + 1]
        if s1 > s0:
            want = f64.attention_f64(q[s0:s1].transpose(1, 0, 2), k[s0:s1].transpose(1, 0, 2),
                                     v[s0:s1].transpose(1, 0, 2), causal, None)
            assert np.abs(got[s0:s1] - want.transpose(1, 0, 2)).max() < 2e-5


def test_varlen_sequences_are_independent():
    cu = [0, 30, 70]
    q, k, v = rand(70, 2, 64), rand(70, 2, 64), rand(70, 2, 64)
    base = oracle.attention_varlen(q, k, v, cu, False)
    k2, v2 = k.copy(), v.copy()
    k2[30:], v2[30:] = rand(40, 2, 64), rand(40, 2, 64)
    other = oracle.attention_varlen(q, k2, v2, cu, False)
    assert np.array_equal(base[:30], other[:30]) and not np.array_equal(base[30:], other[30:])
