"""The entry points under HIP graph capture (torch.cuda.CUDAGraph), as a serving
loop runs decode: each graph is replayed several times with the program's own
eager work and synchronisations in between, and every replay must equal the
eager call bit for bit.  The captured paths record only kernel launches (no
memset nodes): outputs and split partials come from the caching allocator
uninitialised, and the kernels write every element they read back."""
import numpy as np
import pytest
import torch

import attnkernels as ak
import oracle

pytestmark = pytest.mark.gpu


def _capture(fn):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm the allocator off the capture
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    return g, out


def _replays_match(fn, replays=4):
    want = fn().clone()
    torch.cuda.synchronize()
    g, out = _capture(fn)
    for i in range(replays):
        out.fill_(float("nan"))  # a replay must rewrite every element
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), i
        junk = torch.randn(1 << 20, device="cuda").sum()  # eager work between replays
        torch.cuda.synchronize()
        del junk


@pytest.mark.parametrize("hq,hkv,part", [(32, 8, None), (16, 16, 256), (64, 8, 1024)])
def test_paged_decode_replays(hq, hkv, part):
    lens = [1, 700, 4096, 2500]
    kc, vc, bt, cl = oracle.make_paged_cache(lens, hkv, 128, block_size=16, extra_blocks=3, seed=3)
    q = np.random.default_rng(4).standard_normal((len(lens), hq, 128), dtype=np.float32).astype(np.float16)
    q, kc, vc, bt, cl = (torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in (q, kc, vc, bt, cl))
    _replays_match(lambda: ak.paged_decode(q, kc, vc, bt, cl, max(lens), partition_size=part))


@pytest.mark.parametrize("d,causal", [(64, False), (128, True)])
def test_flash_attention_replays(d, causal):
    g = torch.Generator(device="cuda").manual_seed(5)
    q, k, v = (torch.randn(2, 4, 1000, d, generator=g, device="cuda", dtype=torch.float16) for _ in range(3))
    _replays_match(lambda: ak.flash_attention(q, k, v, causal=causal))
