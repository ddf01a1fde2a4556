"""GPU parity of the prefill layouts the reference does not have: grouped-query
attention (flash_attention_gqa) and packed variable-length sequences
(flash_attention_varlen), against the CPU oracle (oracle.attention_gqa /
oracle.attention_varlen) with the north-star tolerances, and bit-exact against
the dense kernel where the two compute the same thing."""
import ctypes

import numpy as np
import pytest
import torch

import attnkernels as ak
import oracle
from conftest import PKG_DIR, TOL, max_err

pytestmark = pytest.mark.gpu


def rand(*shape, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).half()


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("h,hkv,n", [(8, 2, 300), (32, 8, 77), (4, 1, 1000), (16, 2, 1)])
def test_gqa_matches_oracle(d, causal, h, hkv, n):
    q, k, v = rand(2, h, n, d, seed=1), rand(2, hkv, n, d, seed=2), rand(2, hkv, n, d, seed=3)
    out = ak.flash_attention_gqa(q.cuda(), k.cuda(), v.cuda(), causal=causal)
    torch.cuda.synchronize()
    assert max_err(out, oracle.attention_gqa(q.numpy(), k.numpy(), v.numpy(), causal)) < TOL[d]


def test_gqa_with_equal_heads_is_the_dense_kernel():
    q, k, v = (rand(1, 4, 513, 128, seed=s).cuda() for s in (4, 5, 6))
    a = ak.flash_attention_gqa(q, k, v, causal=True)
    b = ak.flash_attention(q, k, v, causal=True)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_gqa_equals_dense_on_repeated_heads():
    q, k, v = rand(1, 8, 260, 64, seed=7).cuda(), rand(1, 2, 260, 64, seed=8).cuda(), rand(1, 2, 260, 64, seed=9).cuda()
    a = ak.flash_attention_gqa(q, k, v, causal=False)
    b = ak.flash_attention(q, k.repeat_interleave(4, dim=1), v.repeat_interleave(4, dim=1), causal=False)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def packed(lens, h, hkv, d, seed=0):
    total = sum(lens)
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
    return rand(total, h, d, seed=seed), rand(total, hkv, d, seed=seed + 1), rand(total, hkv, d, seed=seed + 2), cu


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("lens,h,hkv", [([1, 255, 256, 257, 3], 4, 4), ([700, 40, 1300], 8, 2),
                                        ([129, 0, 511, 64], 6, 3)])
def test_varlen_matches_oracle(d, causal, lens, h, hkv):
    q, k, v, cu = packed(lens, h, hkv, d, seed=sum(lens))
    out = ak.flash_attention_varlen(q.cuda(), k.cuda(), v.cuda(), cu.cuda(), max(lens), causal=causal)
    torch.cuda.synchronize()
    want = oracle.attention_varlen(q.numpy(), k.numpy(), v.numpy(), cu.numpy(), causal)
    assert max_err(out, want) < TOL[d]


def test_varlen_on_equal_lengths_is_the_dense_kernel():
    """Same arithmetic per (sequence, head) on a row-strided layout: bit-identical."""
    b, h, n, d = 3, 4, 333, 128
    q, k, v = (rand(b, h, n, d, seed=s) for s in (10, 11, 12))
    dense = ak.flash_attention(q.cuda(), k.cuda(), v.cuda(), causal=True)
    pack = lambda t: t.transpose(1, 2).reshape(b * n, h, d).contiguous().cuda()  # noqa: E731
    cu = torch.arange(0, (b + 1) * n, n, dtype=torch.int32)
    out = ak.flash_attention_varlen(pack(q), pack(k), pack(v), cu, n, causal=True)
    torch.cuda.synchronize()
    assert torch.equal(out, pack(dense))


@pytest.mark.parametrize("d", [64, 128])
def test_varlen_gqa_workgroup_sizes_agree(d):
    """Long sequences over 64 query heads run on 8-wave workgroups; one GQA group
    alone (8 query heads, 1 kv head) is a small grid and runs on 4-wave ones.  At
    D = 128 the group's heads must come out bit-identical; at D = 64 the 4-wave
    workgroups take 64-key tiles instead of 128 and agree to rounding.  Both
    match the oracle."""
    lens, h, hkv = [2100, 2500], 64, 8
    q, k, v, cu = packed(lens, h, hkv, d, seed=d)
    big = ak.flash_attention_varlen(q.cuda(), k.cuda(), v.cuda(), cu.cuda(), max(lens), causal=True)
    g = h // hkv
    small = ak.flash_attention_varlen(q[:, :g].contiguous().cuda(), k[:, :1].contiguous().cuda(),
                                      v[:, :1].contiguous().cuda(), cu.cuda(), max(lens), causal=True)
    torch.cuda.synchronize()
    if d == 128:
        assert torch.equal(big[:, :g], small)
    else:
        assert max_err(big[:, :g], small) < TOL[d]
    want = oracle.attention_varlen(q[:, :g].numpy(), k[:, :1].numpy(), v[:, :1].numpy(), cu.numpy(), True)
    assert max_err(small, want) < TOL[d]
    assert max_err(big[:, :g], want) < TOL[d]


def test_varlen_host_offsets_and_larger_max_seqlen():
    q, k, v, cu = packed([90, 300], 4, 2, 64, seed=20)
    out = ak.flash_attention_varlen(q.cuda(), k.cuda(), v.cuda(), cu, 2048, causal=True)  # host cu, loose max
    torch.cuda.synchronize()
    assert max_err(out, oracle.attention_varlen(q.numpy(), k.numpy(), v.numpy(), cu.numpy(), True)) < TOL[64]


def test_varlen_offsets_are_clamped_to_the_tensors():
    """Device offsets past the packed rows: the last sequence is cut at the end
    of the tensors (computed over rows 100..299), nothing is read or written
    outside them."""
    q, k, v, _ = packed([300], 4, 4, 64, seed=30)
    cu = torch.tensor([0, 100, 400], dtype=torch.int32, device="cuda")
    out = ak.flash_attention_varlen(q.cuda(), k.cuda(), v.cuda(), cu, 300, causal=True)
    torch.cuda.synchronize()
    want = oracle.attention_varlen(q.numpy(), k.numpy(), v.numpy(), [0, 100, 300], True)
    assert max_err(out, want) < TOL[64]


def test_varlen_rejects_bad_input():
    q, k, v, cu = packed([10, 20], 4, 2, 64)
    with pytest.raises(ValueError, match="max_seqlen"):
        ak.flash_attention_varlen(q.cuda(), k.cuda(), v.cuda(), cu, 15)
    with pytest.raises(ValueError, match="non-decreasing"):
        ak.flash_attention_varlen(q.cuda(), k.cuda(), v.cuda(), torch.tensor([0, 20, 10], dtype=torch.int32), 20)
    with pytest.raises(ValueError, match="multiple of the kv heads"):
        ak.flash_attention_varlen(q.cuda(), k[:, :1].repeat(1, 3, 1).cuda(), v[:, :1].repeat(1, 3, 1).cuda(), cu, 20)
    with pytest.raises(ValueError, match="head_dim"):
        ak.flash_attention_gqa(*(t.cuda() for t in (rand(1, 2, 8, 32), rand(1, 1, 8, 32), rand(1, 1, 8, 32))))


def test_capi_prefill_varlen():
    lib = ctypes.CDLL(str(PKG_DIR / "attnkernels" / "libattnkernels.so"))
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    lib.ak_prefill_varlen.argtypes = [vp] * 5 + [i64] * 6 + [ctypes.c_int, ctypes.c_double, vp]
    lib.ak_last_error.restype = ctypes.c_char_p
    q, k, v, cu = packed([33, 400, 7], 8, 2, 128, seed=40)
    qd, kd, vd, cud = q.cuda(), k.cuda(), v.cuda(), cu.cuda()
    o = torch.empty_like(qd)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.ak_prefill_varlen(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), o.data_ptr(), cud.data_ptr(), 3, 440, 8, 2,
                               400, 128, 0, 128 ** -0.5, stream)
    assert rc == 0, lib.ak_last_error()
    torch.cuda.synchronize()
    assert max_err(o, oracle.attention_varlen(q.numpy(), k.numpy(), v.numpy(), cu.numpy(), False)) < TOL[128]
