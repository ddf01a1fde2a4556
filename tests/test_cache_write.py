"""GPU parity of the paged KV-cache writer (attnkernels.reshape_and_cache)
against the CPU oracle (oracle.reshape_and_cache): a bit copy, so the bar is
bit-exact, for fp16 and bf16."""
import ctypes

import numpy as np
import pytest
import torch

import attnkernels as ak
import oracle
from conftest import PKG_DIR

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.cpu().view(torch.int16).numpy()


def _case(T, hkv, d, nb, bs, dtype, seed=0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    key = torch.randn(T, hkv, d, generator=g, device="cuda").to(dtype)
    value = torch.randn(T, hkv, d, generator=g, device="cuda").to(dtype)
    kc = torch.randn(nb, hkv, bs, d, generator=g, device="cuda").to(dtype)
    vc = torch.randn(nb, hkv, bs, d, generator=g, device="cuda").to(dtype)
    perm = torch.randperm(nb * bs, generator=torch.Generator().manual_seed(seed))[:T]
    return key, value, kc, vc, perm.to(device="cuda", dtype=torch.int64)


def _check(key, value, kc0, vc0, kc, vc, slots):
    want_k, want_v = oracle.reshape_and_cache(_bits(key), _bits(value), _bits(kc0), _bits(vc0), slots.cpu().numpy())
    assert np.array_equal(_bits(kc), want_k)
    assert np.array_equal(_bits(vc), want_v)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("T,hkv,d,nb,bs", [(1, 8, 128, 4, 16), (37, 8, 128, 64, 16), (300, 32, 128, 40, 16),
                                           (129, 4, 64, 50, 16), (64, 2, 64, 30, 12), (17, 3, 40, 9, 5)])
def test_matches_oracle_bit_exact(dtype, T, hkv, d, nb, bs):
    key, value, kc, vc, slots = _case(T, hkv, d, nb, bs, dtype)
    kc0, vc0 = kc.clone(), vc.clone()
    ak.reshape_and_cache(key, value, kc, vc, slots)
    torch.cuda.synchronize()
    _check(key, value, kc0, vc0, kc, vc, slots)


def test_strided_rows_from_fused_projection():
    """key/value as slices of a [T, 3, Hkv, D] QKV output (token stride 3*Hkv*D)."""
    T, hkv, d = 50, 8, 128
    qkv = torch.randn(T, 3, hkv, d, device="cuda", dtype=torch.float16)
    key, value = qkv[:, 1], qkv[:, 2]
    assert key.stride(0) == 3 * hkv * d and not key.is_contiguous()
    kc = torch.zeros(8, hkv, 16, d, device="cuda", dtype=torch.float16)
    vc = torch.zeros_like(kc)
    slots = torch.arange(3, 3 + T, device="cuda", dtype=torch.int64)
    kc0, vc0 = kc.clone(), vc.clone()
    ak.reshape_and_cache(key, value, kc, vc, slots)
    torch.cuda.synchronize()
    _check(key, value, kc0, vc0, kc, vc, slots)


def test_padding_and_out_of_pool_slots_are_skipped():
    key, value, kc, vc, _ = _case(6, 8, 64, 4, 16, torch.float16, seed=3)
    slots = torch.tensor([5, -1, 63, 64, 1 << 40, 0], device="cuda", dtype=torch.int64)
    kc0, vc0 = kc.clone(), vc.clone()
    ak.reshape_and_cache(key, value, kc, vc, slots)
    torch.cuda.synchronize()
    _check(key, value, kc0, vc0, kc, vc, slots)
    untouched = torch.ones(4 * 16, dtype=torch.bool)
    untouched[[5, 63, 0]] = False
    flat = lambda c: c.permute(0, 2, 1, 3).reshape(64, -1)  # noqa: E731
    assert torch.equal(flat(kc).cpu()[untouched], flat(kc0).cpu()[untouched])


def test_int32_slots_and_empty_batch():
    key, value, kc, vc, slots = _case(10, 8, 128, 8, 16, torch.float16, seed=4)
    kc0, vc0 = kc.clone(), vc.clone()
    ak.reshape_and_cache(key, value, kc, vc, slots.to(torch.int32))
    torch.cuda.synchronize()
    _check(key, value, kc0, vc0, kc, vc, slots)
    before = kc.clone()
    ak.reshape_and_cache(key[:0], value[:0], kc, vc, slots[:0])
    torch.cuda.synchronize()
    assert torch.equal(kc, before)


def test_rejects_bad_input():
    key, value, kc, vc, slots = _case(4, 8, 128, 4, 16, torch.float16)
    with pytest.raises(ValueError, match="fp16 or all bf16"):
        ak.reshape_and_cache(key.float(), value.float(), kc, vc, slots)
    with pytest.raises(ValueError, match="matching key"):
        ak.reshape_and_cache(key[:, :4].contiguous(), value[:, :4].contiguous(), kc, vc, slots)
    with pytest.raises(ValueError, match="num_tokens"):
        ak.reshape_and_cache(key, value, kc, vc, slots[:3])


def test_decode_reads_what_was_written():
    """Append the last token of every sequence through its block table, then
    decode: the result is bit-identical to decoding a cache that held that
    token from the start."""
    lens = [70, 1, 33, 256, 17]
    hkv, d, bs = 8, 128, 16
    kc_full, vc_full, bt, cl = (torch.from_numpy(x) for x in oracle.make_paged_cache(lens, hkv, d, bs, seed=9))
    kc_full, vc_full, bt, cl = kc_full.cuda(), vc_full.cuda(), bt.cuda(), cl.cuda()
    pos = np.asarray(lens) - 1
    slots = torch.from_numpy(oracle.append_slots(bt.cpu().numpy(), pos, bs)).cuda()
    page, row = slots // bs, slots % bs
    new_k = kc_full[page, :, row].clone()   # [B, Hkv, D]
    new_v = vc_full[page, :, row].clone()
    kc, vc = kc_full.clone(), vc_full.clone()
    kc[page, :, row] = 0
    vc[page, :, row] = 0
    ak.reshape_and_cache(new_k, new_v, kc, vc, slots)
    q = torch.randn(len(lens), 4 * hkv, d, device="cuda", dtype=torch.float16)
    a = ak.paged_decode(q, kc, vc, bt, cl, max(lens))
    b = ak.paged_decode(q, kc_full, vc_full, bt, cl, max(lens))
    torch.cuda.synchronize()
    assert torch.equal(kc, kc_full) and torch.equal(a, b)


def test_capi_reshape_and_cache():
    lib = ctypes.CDLL(str(PKG_DIR / "attnkernels" / "libattnkernels.so"))
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    lib.ak_reshape_and_cache.argtypes = [vp] * 5 + [i64] * 7 + [vp]
    lib.ak_last_error.restype = ctypes.c_char_p
    key, value, kc, vc, slots = _case(33, 8, 128, 16, 16, torch.bfloat16, seed=7)
    kc0, vc0 = kc.clone(), vc.clone()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.ak_reshape_and_cache(key.data_ptr(), value.data_ptr(), kc.data_ptr(), vc.data_ptr(), slots.data_ptr(),
                                  33, 8, 128, 16, 16, 8 * 128, 8 * 128, stream)
    assert rc == 0, lib.ak_last_error()
    torch.cuda.synchronize()
    _check(key, value, kc0, vc0, kc, vc, slots)
