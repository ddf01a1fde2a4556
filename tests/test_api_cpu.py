"""Host logic of the attnkernels Python API that needs no GPU: validation
errors (reference attnkernels/__init__.py:53-61, 116-119), the split-size rule
(93-101) against the reference's recorded values, and the plain-PyTorch
baselines module against the CPU oracle."""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

import attnkernels as ak
from attnkernels import reference as akref
import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_public_surface_matches_reference():
    assert ak.__all__ == ["naive_attention", "flash_attention", "paged_decode", "decode_partition",
                          "reshape_and_cache", "flash_attention_gqa", "flash_attention_varlen", "load_extension"]
    assert ak.CHUNK == 256 and ak.WMMA_BLOCK_N == {64: 64, 128: 64}
    for name in ("attention_fp32", "make_paged_cache", "gather_kv", "paged_decode_fp32",
                 "paged_decode_torch"):
        assert callable(getattr(akref, name))


def test_prefill_rejects_cpu_tensors():
    q = torch.zeros(1, 1, 16, 64, dtype=torch.float16)
    for fn in (ak.naive_attention, ak.flash_attention):
        with pytest.raises(ValueError, match="fp16 CUDA tensors"):
            fn(q, q, q)


def test_paged_decode_validation():
    q = torch.zeros(2, 4, 64, dtype=torch.float16)
    kc = torch.zeros(3, 4, 16, 64, dtype=torch.float16)
    bt = torch.zeros(2, 3, dtype=torch.int32)
    lens = torch.ones(2, dtype=torch.int32)
    with pytest.raises(ValueError, match="fp16"):
        ak.paged_decode(q.float(), kc, kc, bt, lens, 1)
    with pytest.raises(ValueError, match="head_dim"):
        ak.paged_decode(q[..., :32], kc[..., :32], kc[..., :32], bt, lens, 1)
    with pytest.raises(ValueError, match="head_dim"):
        ak.paged_decode(q, kc[..., :32].contiguous(), kc[..., :32].contiguous(), bt, lens, 1)


def test_decode_partition_matches_reference_t4_run(monkeypatch):
    fx = json.loads((GOLDEN / "decode_partition_t4.json").read_text())
    monkeypatch.setattr(ak, "_sm_count", lambda dev: fx["sm_count"])
    for r in fx["rows"]:
        assert ak.decode_partition(r["batch"], r["num_kv_heads"], r["max_context_len"], 0,
                                   wg_per_cu=ak.REFERENCE_WG_PER_SM, min_chunks=1) == r["partition"], r


def test_decode_partition_on_256_cus(monkeypatch):
    monkeypatch.setattr(ak, "_sm_count", lambda dev: 256)
    for b, hkv, ctx in [(64, 32, 4096), (8, 32, 32768), (1, 8, 32768), (3, 8, 1), (64, 8, 1024)]:
        assert ak.decode_partition(b, hkv, ctx, 0, min_chunks=1) == \
            oracle.decode_partition(b, hkv, ctx, 256, wg_per_sm=ak.DECODE_WG_PER_CU)
        assert ak.decode_partition(b, hkv, ctx, 0, wg_per_cu=4, min_chunks=1) == oracle.decode_partition(b, hkv, ctx, 256)
    # The default floor of 2 chunks per split, where the reference's rule gives 256 tokens:
    # 512 splits wanted but 64 at most (128 chunks); 8 wanted, 2 at most (4 chunks);
    # a 1-token context keeps one 256-token split.
    assert ak.DECODE_MIN_CHUNKS == 2
    assert oracle.decode_partition(1, 8, 32768, 256, wg_per_sm=16) == 256
    assert ak.decode_partition(1, 8, 32768, 0) == 512
    assert oracle.decode_partition(64, 8, 1024, 256, wg_per_sm=16) == 256
    assert ak.decode_partition(64, 8, 1024, 0) == 512
    assert ak.decode_partition(3, 8, 1, 0) == 256
    assert ak.decode_partition(3, 8, 300, 0) == 512   # 2 chunks: one split
    assert ak.decode_partition(64, 32, 4096, 0) == 2048   # the floor does not bind


def test_decode_partition_default_is_near_the_measured_optimum(monkeypatch):
    """On 256 CUs the default rule picks a partition within 12% of the fastest
    one in every case of the MI355X split-K ablation, uniform and mixed context
    lengths (tests/golden/decode_partition_mi355x.json: bandwidth of every
    power-of-two partition per case); the reference's rule does not, nor does
    the default factor without the 2-chunk floor."""
    fx = json.loads((GOLDEN / "decode_partition_mi355x.json").read_text())
    monkeypatch.setattr(ak, "_sm_count", lambda dev: fx["cu_count"])
    assert fx["rows"] and any(r["mixed_lengths"] for r in fx["rows"])

    def worst(factor, min_chunks):
        fr = []
        for r in fx["rows"]:
            p = ak.decode_partition(r["batch"], r["num_kv_heads"], r["max_context_len"], 0, wg_per_cu=factor,
                                    min_chunks=min_chunks)
            fr.append(r["gbs"][str(p)] / max(r["gbs"].values()))
        return min(fr)

    best = worst(ak.DECODE_WG_PER_CU, ak.DECODE_MIN_CHUNKS)
    assert best >= 0.88
    assert worst(ak.REFERENCE_WG_PER_SM, 1) < best
    assert worst(ak.DECODE_WG_PER_CU, 1) < best


def test_reference_module_attention_matches_oracle():
    g = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn(2, 3, 45, 64, generator=g).half() for _ in range(3))
    for causal in (False, True):
        got = akref.attention_fp32(q, k, v, causal).numpy()
        want = oracle.attention_fp32(q.numpy(), k.numpy(), v.numpy(), causal)
        assert np.abs(got - want).max() < 1e-5


def test_reference_module_decode_matches_oracle():
    g = torch.Generator().manual_seed(6)
    kc, vc, bt, lens = akref.make_paged_cache([33, 300, 16], 2, 128, device="cpu",
                                              extra_blocks=4, generator=g)
    assert kc.shape == (3 + 19 + 1 + 4, 2, 16, 128) and bt.dtype == torch.int32
    q = torch.randn(3, 8, 128, generator=g).half()
    got = akref.paged_decode_fp32(q, kc, vc, bt, lens).numpy()
    want = oracle.paged_decode_fp32(q.numpy(), kc.numpy(), vc.numpy(), bt.numpy(), lens.numpy())
    assert np.abs(got - want).max() < 1e-5
    base = akref.paged_decode_torch(q.float(), kc.float(), vc.float(), bt, bt.shape[1],
                                    context_lens=lens).numpy()
    assert np.abs(base - want).max() < 1e-4
