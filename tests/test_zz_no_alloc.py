"""ak_paged_decode_noalloc (static per-GPU split partials and split counters,
no workspace argument) against ak_paged_decode_fused with a caller workspace
and counter array, through the C-ABI: the same kernels, so the outputs must be
bit-identical; both must match the oracle and the two-kernel ak_paged_decode.
Two calls in a row, the second with a smaller input, show that the shared
static arrays carry nothing from one call into the next.  A call allocates no
device memory, and one captured in a HIP graph replays bit-identically."""
import ctypes
import json
import subprocess
import sys

import numpy as np
import pytest
import torch

import oracle
from conftest import PKG_DIR, ROOT, TOL, max_err

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
    L.ak_paged_decode_fused.argtypes = [vp] * 6 + [i64] * 8 + [f64, i64, vp, ctypes.c_size_t, vp, i64, vp]
    L.ak_paged_decode_noalloc.argtypes = [vp] * 6 + [i64] * 8 + [f64, i64, vp]
    return L


def ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def make_case(lens, hq, hkv, d, seed):
    kc, vc, bt, cl = oracle.make_paged_cache(lens, hkv, d, block_size=16, extra_blocks=3, seed=seed)
    q = np.random.default_rng(seed + 1).standard_normal((len(lens), hq, d), dtype=np.float32).astype(np.float16)
    dev = [torch.from_numpy(a).cuda() for a in (q, kc, vc, bt, cl)]
    sizes = [len(lens), hq, hkv, d, kc.shape[0], 16, bt.shape[1], max(lens)]
    return (q, kc, vc, bt, cl), dev, sizes


def noalloc(lib, dev, sizes, out, partition):
    qd, kcd, vcd, btd, cld = dev
    return lib.ak_paged_decode_noalloc(ptr(qd), ptr(kcd), ptr(vcd), ptr(btd), ptr(cld), ptr(out), *sizes,
                                       sizes[3] ** -0.5, partition, stream())


def one_case(lib, lens, hq, hkv, d, partition, seed):
    print(f"noalloc case lens={lens} hq={hq} hkv={hkv} d={d} P={partition}", flush=True)
    (q, kc, vc, bt, cl), dev, sizes = make_case(lens, hq, hkv, d, seed)
    qd, kcd, vcd, btd, cld = dev
    max_ctx = max(lens)
    need = lib.ak_paged_decode_workspace_size(len(lens), hq, d, max_ctx, partition)
    assert 0 < need <= MAX_BYTES
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    counters = torch.zeros(len(lens) * hkv, dtype=torch.int32, device="cuda")
    want = torch.empty_like(qd)
    rc = lib.ak_paged_decode_fused(ptr(qd), ptr(kcd), ptr(vcd), ptr(btd), ptr(cld), ptr(want), *sizes,
                                   d ** -0.5, partition, ptr(ws), need, ptr(counters), counters.numel(), stream())
    assert rc == 0, lib.ak_last_error()
    plain = torch.empty_like(qd)
    rc = lib.ak_paged_decode(ptr(qd), ptr(kcd), ptr(vcd), ptr(btd), ptr(cld), ptr(plain), *sizes, d ** -0.5,
                             partition, ptr(ws), need, stream())
    assert rc == 0, lib.ak_last_error()
    got = torch.full_like(qd, float("nan"))
    assert noalloc(lib, dev, sizes, got, partition) == 0, lib.ak_last_error()
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    ref = oracle.paged_decode_fp32(q, kc, vc, bt, cl)
    assert max_err(got, ref) < TOL[d]
    assert max_err(plain, ref) < TOL[d]


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


def test_noalloc_allocates_no_device_memory(lib):
    """Free device memory (hipMemGetInfo) is the same before and after a call;
    a first call loads the module and its static arrays, so it runs first."""
    _, dev, sizes = make_case([2000, 500], 16, 4, 128, seed=81)
    out = torch.empty_like(dev[0])
    assert noalloc(lib, dev, sizes, out, 256) == 0, lib.ak_last_error()
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    for _ in range(3):
        assert noalloc(lib, dev, sizes, out, 256) == 0, lib.ak_last_error()
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert free1 == free0


def test_noalloc_under_graph_capture_replays_bit_identically(lib):
    """A noalloc call captured in a HIP graph (stream capture through torch):
    each replay, with eager noalloc calls of another shape between them, gives
    the eager result bit for bit."""
    (q, kc, vc, bt, cl), dev, sizes = make_case([3000, 1200, 40], 32, 8, 128, seed=91)
    eager = torch.empty_like(dev[0])
    assert noalloc(lib, dev, sizes, eager, 256) == 0, lib.ak_last_error()
    torch.cuda.synchronize()
    assert max_err(eager, oracle.paged_decode_fp32(q, kc, vc, bt, cl)) < TOL[128]
    out = torch.full_like(dev[0], float("nan"))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        rc = noalloc(lib, dev, sizes, out, 256)
    assert rc == 0, lib.ak_last_error()
    _, other_dev, other_sizes = make_case([700, 700], 16, 16, 64, seed=93)
    other = torch.empty_like(other_dev[0])
    for _ in range(3):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        assert noalloc(lib, other_dev, other_sizes, other, 256) == 0, lib.ak_last_error()
        torch.cuda.synchronize()


@pytest.mark.parametrize("hq", [32, 64])
def test_noalloc_first_call_on_the_device_inside_a_graph_capture(hq):
    """In a fresh process, the library's first call on the device is a
    noalloc call inside a graph capture (the symbol lookup, the module load and
    the grouped-query kernel's occupancy query happen under capture); replays
    equal the fused entry point bit for bit and, after the graph's first
    launch, leave free device memory unchanged.  Four and eight query heads
    per kv head (the dot-product and the matrix-core kernel)."""
    helper = ROOT / "tests" / "noalloc_capture_first.py"
    print(f"fresh process, hq={hq}", flush=True)
    r = subprocess.run([sys.executable, str(helper), str(hq)], capture_output=True, text=True, timeout=100)
    print(r.stdout, r.stderr[-2000:], flush=True)
    assert r.returncode == 0
    res = json.loads(r.stdout.strip().splitlines()[-1])
    assert res["capture_rc"] == 0, res["error"]
    assert res["fused_rc"] == 0 and res["finite"]
    assert res["replays_equal"] == [True] * 4
    assert res["free_unchanged"]
