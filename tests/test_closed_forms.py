"""Closed forms on the GPU, independent of the oracle's code.  With q = 0 every
score is equal, so softmax attention is a plain average of V: over every key
(non-causal prefill), over the keys up to the query (causal prefill: the
running mean), over the context (decode, whatever the split-K partition).
This pins the masking, the row sums and the LSE merge of the splits."""
import numpy as np
import pytest
import torch

import attnkernels as ak
import oracle
from conftest import TOL

pytestmark = pytest.mark.gpu


def _v(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape, dtype=np.float32).astype(np.float16)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("n", [1, 77, 1000, 4097])
def test_prefill_zero_queries_average_v(d, causal, n):
    b, h = 2, 3
    v = _v((b, h, n, d), seed=n + d)
    k = _v((b, h, n, d), seed=n + d + 1)
    q = np.zeros_like(v)
    out = ak.flash_attention(*(torch.from_numpy(x).cuda() for x in (q, k, v)), causal=causal)
    v64 = v.astype(np.float64)
    if causal:
        want = np.cumsum(v64, axis=2) / np.arange(1, n + 1)[None, None, :, None]
    else:
        want = np.broadcast_to(v64.mean(axis=2, keepdims=True), v64.shape)
    assert np.abs(out.float().cpu().numpy() - want).max() < TOL[d]


@pytest.mark.parametrize("d,hq,hkv", [(128, 8, 8), (128, 32, 8), (64, 16, 2), (128, 64, 8)])
@pytest.mark.parametrize("part", [256, 1024, 1 << 20])
def test_decode_zero_queries_average_context(d, hq, hkv, part):
    lens = [1, 255, 256, 257, 3000]
    kc, vc, bt, cl = oracle.make_paged_cache(lens, hkv, d, block_size=16, extra_blocks=4, seed=9)
    q = np.zeros((len(lens), hq, d), np.float16)
    out = ak.paged_decode(*(torch.from_numpy(np.ascontiguousarray(x)).cuda() for x in (q, kc, vc, bt, cl)),
                          max(lens), partition_size=part).float().cpu().numpy()
    g = hq // hkv
    for bi, c in enumerate(lens):
        pages = bt[bi, :-(-c // 16)]
        vseq = vc[pages].transpose(1, 0, 2, 3).reshape(hkv, -1, d)[:, :c].astype(np.float64)
        want = vseq.mean(axis=1)                      # [hkv, d]
        got = out[bi].reshape(hkv, g, d)
        assert np.abs(got - want[:, None, :]).max() < TOL[d], (bi, c)
