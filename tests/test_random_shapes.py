"""Seeded random shapes on the GPU against the CPU oracle.

The hand-picked grids of test_prefill.py and test_decode.py cover each edge
one at a time; this sweep draws combinations of them: odd batch x head
counts, lengths around the tile sizes, both head sizes, causal or not,
explicit scales, GQA ratios and variable lengths for prefill; head groups
1-8, page sizes 8/12/16/32, random partitions, ragged contexts and
out-of-range page ids for decode, plus a sweep that always takes eight query
heads per kv head (the matrix-core decode kernel; pages of 48 tokens as
well).  Sizes stay small enough for the oracle.
"""
import numpy as np
import pytest
import torch

import attnkernels as ak
import oracle
from conftest import TOL, max_err

pytestmark = pytest.mark.gpu

N_PREFILL, N_DECODE, N_DECODE_EIGHT = 24, 32, 12


def _prefill_case(i):
    rng = np.random.default_rng(1000 + i)
    d = int(rng.choice([64, 128]))
    causal = bool(i % 2)
    n = int(rng.choice([int(rng.integers(1, 40)), int(rng.integers(60, 300)), int(rng.integers(300, 1200))]))
    hkv = int(rng.choice([1, 2, 3]))
    g = int(rng.choice([1, 1, 2, 4]))
    b = int(rng.integers(1, 4))
    scale = None if rng.random() < 0.6 else float(rng.choice([0.02, 0.3, -0.1]))
    kind = rng.choice(["dense", "gqa", "varlen"])
    return dict(d=d, causal=causal, n=n, h=hkv * g, hkv=hkv, b=b, scale=scale, kind=str(kind), seed=2000 + i)


@pytest.mark.parametrize("i", range(N_PREFILL))
def test_prefill_random_shape(i):
    c = _prefill_case(i)
    print(c, flush=True)
    gen = torch.Generator().manual_seed(c["seed"])
    d, n, b, h, hkv = c["d"], c["n"], c["b"], c["h"], c["hkv"]
    sc = d ** -0.5 if c["scale"] is None else c["scale"]
    if c["kind"] == "varlen":
        lens = [int(x) for x in np.random.default_rng(c["seed"]).integers(1, n + 1, size=b)]
        tot = sum(lens)
        q = torch.randn(tot, h, d, generator=gen).half()
        k = torch.randn(tot, hkv, d, generator=gen).half()
        v = torch.randn(tot, hkv, d, generator=gen).half()
        cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
        out = ak.flash_attention_varlen(q.cuda(), k.cuda(), v.cuda(), cu, max(lens), causal=c["causal"],
                                        scale=c["scale"]).cpu()
        ref = oracle.attention_varlen(q.numpy(), k.numpy(), v.numpy(), cu.numpy(), c["causal"], sc)
    else:
        kh = hkv if c["kind"] == "gqa" else h
        q = torch.randn(b, h, n, d, generator=gen).half()
        k = torch.randn(b, kh, n, d, generator=gen).half()
        v = torch.randn(b, kh, n, d, generator=gen).half()
        if kh == h:
            out = ak.flash_attention(q.cuda(), k.cuda(), v.cuda(), causal=c["causal"], scale=c["scale"]).cpu()
            ref = oracle.attention_fp32(q.numpy(), k.numpy(), v.numpy(), c["causal"], sc)
        else:
            out = ak.flash_attention_gqa(q.cuda(), k.cuda(), v.cuda(), causal=c["causal"], scale=c["scale"]).cpu()
            ref = oracle.attention_gqa(q.numpy(), k.numpy(), v.numpy(), c["causal"], sc)
    assert torch.isfinite(out).all()
    assert max_err(out, ref) < TOL[d], c


def _decode_case(i, eight=False):
    """Seeded random decode shape; with eight=True always eight query heads per
    kv head (the matrix-core kernel) and more out-of-range pages."""
    rng = np.random.default_rng((5000 if eight else 3000) + i)
    d = int(rng.choice([64, 128]))
    hkv = int(rng.choice([1, 2, 4, 8]))
    g = 8 if eight else int(rng.choice([1, 2, 4, 8]))
    bs = int(rng.choice([16, 16, 8, 32, 12] + ([48] if eight else [])))
    b = int(rng.integers(1, 7))
    hi = int(rng.choice([40, 700, 3000]))
    lens = [int(x) for x in rng.integers(1, hi + 1, size=b)]
    part = None if rng.random() < 0.4 else 256 * int(rng.integers(1, 9))
    bad = rng.random() < (0.4 if eight else 0.25)
    return dict(d=d, hkv=hkv, hq=hkv * g, bs=bs, lens=lens, part=part, bad=bad, seed=(6000 if eight else 4000) + i)


@pytest.mark.parametrize("i", range(N_DECODE))
def test_decode_random_shape(i):
    _check_decode_case(_decode_case(i))


@pytest.mark.parametrize("i", range(N_DECODE_EIGHT))
def test_decode_random_shape_eight_heads(i):
    _check_decode_case(_decode_case(i, eight=True))


def _check_decode_case(c):
    print(c, flush=True)
    kc, vc, bt, cl = oracle.make_paged_cache(c["lens"], c["hkv"], c["d"], block_size=c["bs"], extra_blocks=3,
                                             seed=c["seed"])
    q = np.random.default_rng(c["seed"] + 1).standard_normal((len(c["lens"]), c["hq"], c["d"]),
                                                             dtype=np.float32).astype(np.float16)
    ref = oracle.paged_decode_fp32(q, kc, vc, bt, cl)
    bt_run = bt
    b = int(np.argmax(cl))
    pages = -(-int(cl[b]) // c["bs"])
    if c["bad"] and pages > 1:
        # one page of the longest sequence gets an out-of-range id: its tokens
        # drop out of the softmax; the reference is attention over the others
        bad = pages // 2
        bt_run = bt.copy()
        bt_run[b, bad] = kc.shape[0] + 5
        keep = np.array([t for t in range(int(cl[b])) if t // c["bs"] != bad])
        kk = oracle.gather_kv(kc, bt[b:b + 1], pages)[0][:, keep]
        vv = oracle.gather_kv(vc, bt[b:b + 1], pages)[0][:, keep]
        g = c["hq"] // c["hkv"]
        ref[b] = np.stack([oracle.attention_fp32(q[b, h][None], kk[h // g], vv[h // g])[0]
                           for h in range(c["hq"])])
    t = [torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in (q, kc, vc, bt_run, cl)]
    out = ak.paged_decode(*t, max(c["lens"]), partition_size=c["part"])
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    assert max_err(out, ref) < TOL[c["d"]], c
