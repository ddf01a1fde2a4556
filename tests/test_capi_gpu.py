"""Parity through the C-ABI itself (include/attnkernels.h via ctypes), with
device buffers from torch and the oracle as the checker."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from conftest import PKG_DIR, TOL, max_err

pytestmark = pytest.mark.gpu

LIB = PKG_DIR / "attnkernels" / "libattnkernels.so"


@pytest.fixture(scope="module")
def lib():
    L = ctypes.CDLL(str(LIB))
    vp, i64, f64 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_double
    L.ak_last_error.restype = ctypes.c_char_p
    L.ak_flash_wmma.argtypes = [vp] * 4 + [i64] * 4 + [ctypes.c_int, f64, i64, vp]
    L.ak_naive_attention.argtypes = [vp] * 4 + [i64] * 4 + [ctypes.c_int, f64, vp]
    L.ak_paged_decode_workspace_size.argtypes = [i64] * 5
    L.ak_paged_decode_workspace_size.restype = ctypes.c_size_t
    L.ak_paged_decode.argtypes = [vp] * 6 + [i64] * 8 + [f64, i64, vp, ctypes.c_size_t, vp]
    return L


def ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


@pytest.mark.parametrize("d,causal,n", [(64, False, 200), (128, True, 333), (128, False, 64)])
def test_capi_prefill(lib, d, causal, n):
    g = torch.Generator().manual_seed(d + n)
    q, k, v = (torch.randn(2, 3, n, d, generator=g).half() for _ in range(3))
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    o = torch.empty_like(qd)
    rc = lib.ak_flash_wmma(ptr(qd), ptr(kd), ptr(vd), ptr(o), 2, 3, n, d, int(causal), d ** -0.5, 64,
                           stream())
    assert rc == 0, lib.ak_last_error()
    torch.cuda.synchronize()
    assert max_err(o, oracle.attention_fp32(q.numpy(), k.numpy(), v.numpy(), causal)) < TOL[d]
    o2 = torch.empty_like(qd)
    assert lib.ak_naive_attention(ptr(qd), ptr(kd), ptr(vd), ptr(o2), 2, 3, n, d, int(causal),
                                  d ** -0.5, stream()) == 0
    torch.cuda.synchronize()
    assert torch.equal(o, o2)


def test_capi_paged_decode_with_workspace(lib):
    lens = [1, 700, 2500]
    kc, vc, bt, cl = oracle.make_paged_cache(lens, 4, 128, block_size=16, extra_blocks=3, seed=9)
    q = np.random.default_rng(10).standard_normal((3, 16, 128), dtype=np.float32).astype(np.float16)
    qd, kcd, vcd, btd, cld = (torch.from_numpy(a).cuda() for a in (q, kc, vc, bt, cl))
    out = torch.empty_like(qd)
    need = lib.ak_paged_decode_workspace_size(3, 16, 128, 2500, 256)
    assert need > 0
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    args = [ptr(qd), ptr(kcd), ptr(vcd), ptr(btd), ptr(cld), ptr(out), 3, 16, 4, 128, kc.shape[0], 16,
            bt.shape[1], 2500, 128 ** -0.5, 256]
    assert lib.ak_paged_decode(*args, None, 0, stream()) == 3          # workspace missing
    assert lib.ak_paged_decode(*args, ptr(ws), need, stream()) == 0, lib.ak_last_error()
    torch.cuda.synchronize()
    assert max_err(out, oracle.paged_decode_fp32(q, kc, vc, bt, cl)) < TOL[128]


@pytest.mark.parametrize("hq,hkv", [(16, 4), (4, 4)])
def test_capi_context_beyond_table_capacity(lib, hq, hkv):
    """context_lens larger than the table row (32 pages x 16 = 512 tokens) with
    max_context_len 1000 and 256-token splits: splits 2 and 3 start past the
    table and write no partial; the reduce must not read them.  The workspace
    is pre-filled with NaN, so reading one would show."""
    lens = [512, 300]
    kc, vc, bt, _ = oracle.make_paged_cache(lens, hkv, 128, block_size=16, extra_blocks=3, seed=12)
    cl = np.asarray([1000, 300], np.int32)
    q = np.random.default_rng(13).standard_normal((2, hq, 128), dtype=np.float32).astype(np.float16)
    qd, kcd, vcd, btd, cld = (torch.from_numpy(a).cuda() for a in (q, kc, vc, bt, cl))
    out = torch.empty_like(qd)
    need = lib.ak_paged_decode_workspace_size(2, hq, 128, 1000, 256)
    ws = torch.full((need // 4,), float("nan"), dtype=torch.float32, device="cuda")
    rc = lib.ak_paged_decode(ptr(qd), ptr(kcd), ptr(vcd), ptr(btd), ptr(cld), ptr(out), 2, hq, hkv, 128,
                             kc.shape[0], 16, bt.shape[1], 1000, 128 ** -0.5, 256, ptr(ws), need, stream())
    assert rc == 0, lib.ak_last_error()
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    ref = oracle.paged_decode_fp32(q, kc, vc, bt, np.asarray([512, 300], np.int32))
    assert max_err(out, ref) < TOL[128]


@pytest.mark.parametrize("nbytes", [16, 48, (1 << 20) + 16 * 37, 300 << 20])
def test_stream_checksum_is_the_xor_of_all_words(lib, nbytes):
    """ak_stream_checksum (the bench's read ceiling) reads every 16-byte word
    once: its result is the XOR of all words, for buffers inside one grid
    stride, across the unrolled loop, and with a ragged tail."""
    lib.ak_stream_checksum.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p]
    print(f"stream checksum bytes={nbytes}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(nbytes % 1009)
    src = torch.randint(-2 ** 31, 2 ** 31 - 1, (nbytes // 4,), generator=g, device="cuda", dtype=torch.int32)
    out = torch.zeros(4, dtype=torch.int32, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.ak_stream_checksum(ptr(src), nbytes, ptr(out), stream) == 0, lib.ak_last_error()
    torch.cuda.synchronize()
    want = np.bitwise_xor.reduce(src.cpu().numpy().view(np.uint32).reshape(-1, 4), axis=0)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want)


def test_stream_checksum_extension_accumulates(ext):
    """The torch entry point: a fresh result, and XOR-accumulation into a
    caller's int32[4] (the same buffer read twice leaves it at zero)."""
    x = torch.randint(-2 ** 31, 2 ** 31 - 1, ((5 << 20) // 4 + 12,), device="cuda", dtype=torch.int32)
    one = ext.stream_checksum(x)
    acc = torch.zeros(4, dtype=torch.int32, device="cuda")
    ext.stream_checksum(x, acc)
    assert torch.equal(one, acc)
    ext.stream_checksum(x, acc)
    assert int(acc.count_nonzero()) == 0
    with pytest.raises(RuntimeError):
        ext.stream_checksum(x, torch.zeros(3, dtype=torch.int32, device="cuda"))
