"""ak_paged_decode_noalloc (static per-GPU split partials, no workspace argument)
against ak_paged_decode with a caller workspace, through the C-ABI: the same
kernels, so the outputs must be bit-identical, and both must match the oracle.
Two calls in a row, the second with a smaller input, show that the shared
static array carries nothing from one call into the next."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from conftest import PKG_DIR, TOL, max_err

pytestmark = pytest.mark.gpu

LIB = PKG_DIR / "attnkernels" / "libattnkernels.so"
MAX_BYTES = 32 << 20  # AK_PAGED_DECODE_NOALLOC_MAX_BYTES


@pytest.fixture(scope="module")
def lib():
    L = ctypes.CDLL(str(LIB))
    vp, i64, f64 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_double
    L.ak_last_error.restype = ctypes.c_char_p
    L.ak_paged_decode_workspace_size.argtypes = [i64] * 5
    L.ak_paged_decode_workspace_size.restype = ctypes.c_size_t
    L.ak_paged_decode.argtypes = [vp] * 6 + [i64] * 8 + [f64, i64, vp, ctypes.c_size_t, vp]
    L.ak_paged_decode_noalloc.argtypes = [vp] * 6 + [i64] * 8 + [f64, i64, vp]
    return L


def ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def one_case(lib, lens, hq, hkv, d, partition, seed):
    print(f"noalloc case lens={lens} hq={hq} hkv={hkv} d={d} P={partition}", flush=True)
    kc, vc, bt, cl = oracle.make_paged_cache(lens, hkv, d, block_size=16, extra_blocks=3, seed=seed)
    q = np.random.default_rng(seed + 1).standard_normal((len(lens), hq, d), dtype=np.float32).astype(np.float16)
    qd, kcd, vcd, btd, cld = (torch.from_numpy(a).cuda() for a in (q, kc, vc, bt, cl))
    max_ctx = max(lens)
    sizes = [len(lens), hq, hkv, d, kc.shape[0], 16, bt.shape[1], max_ctx]
    need = lib.ak_paged_decode_workspace_size(len(lens), hq, d, max_ctx, partition)
    assert 0 < need <= MAX_BYTES
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    want = torch.empty_like(qd)
    rc = lib.ak_paged_decode(ptr(qd), ptr(kcd), ptr(vcd), ptr(btd), ptr(cld), ptr(want), *sizes, d ** -0.5,
                             partition, ptr(ws), need, stream())
    assert rc == 0, lib.ak_last_error()
    got = torch.full_like(qd, float("nan"))
    rc = lib.ak_paged_decode_noalloc(ptr(qd), ptr(kcd), ptr(vcd), ptr(btd), ptr(cld), ptr(got), *sizes,
                                     d ** -0.5, partition, stream())
    assert rc == 0, lib.ak_last_error()
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert max_err(got, oracle.paged_decode_fp32(q, kc, vc, bt, cl)) < TOL[d]


def test_noalloc_matches_workspace_entry_point_twice(lib):
    # 3 sequences x 16 heads x 12 splits of 256 tokens, then a smaller batch
    # with fewer heads, splits and a different head size: the second call
    # reads only what it wrote itself.
    one_case(lib, [3000, 700, 1], 16, 4, 128, 256, seed=71)
    one_case(lib, [600, 20], 8, 8, 64, 256, seed=73)


def test_noalloc_rejects_partials_beyond_the_static_array(lib):
    vp = ctypes.c_void_p(4096)  # never dereferenced: the size check fails first
    # 64 x 32 heads x 4096 splits x (128 + 2) floats = 4.4 GB of partials
    rc = lib.ak_paged_decode_noalloc(vp, vp, vp, vp, vp, vp, 64, 32, 8, 128, 100, 16, 65536, 1 << 20,
                                     0.1, 256, None)
    assert rc == 3
    assert b"static scratch" in lib.ak_last_error()
