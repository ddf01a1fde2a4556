"""Run as a child process by test_zz_no_alloc.py: the first call of this
library on the device is an ak_paged_decode_noalloc call made inside a HIP
graph capture (torch.cuda.graph, global capture mode).  No kernel of the
library runs before it; the inputs are made with torch.  The replays must
equal ak_paged_decode_fused (the same kernels with a caller workspace) bit for
bit, and free device memory must not change across the replays after the
first.  argv[1]: query heads (32: four per kv head, the dot-product kernel;
64: eight, the matrix-core kernel).  Prints one JSON line."""
import ctypes
import json
import sys
from pathlib import Path

import torch

LIB = Path(__file__).resolve().parents[1] / "flash-attention-from-scratch_amd" / "attnkernels" / "libattnkernels.so"


def main():
    lib = ctypes.CDLL(str(LIB))
    vp, i64, f64 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_double
    lib.ak_last_error.restype = ctypes.c_char_p
    lib.ak_paged_decode_workspace_size.argtypes = [i64] * 5
    lib.ak_paged_decode_workspace_size.restype = ctypes.c_size_t
    lib.ak_paged_decode_fused.argtypes = [vp] * 6 + [i64] * 8 + [f64, i64, vp, ctypes.c_size_t, vp, i64, vp]
    lib.ak_paged_decode_noalloc.argtypes = [vp] * 6 + [i64] * 8 + [f64, i64, vp]
    hq = int(sys.argv[1]) if len(sys.argv) > 1 else 32
    lens, hkv, d, bs, part = [3000, 1200, 40], 8, 128, 16, 256
    nblk = [-(-n // bs) for n in lens]
    pool = sum(nblk) + 3
    g = torch.Generator(device="cuda").manual_seed(5)
    perm = torch.randperm(pool, generator=torch.Generator().manual_seed(5)).to(torch.int32)
    tables = torch.zeros(len(lens), max(nblk), dtype=torch.int32)
    pos = 0
    for b, nb in enumerate(nblk):
        tables[b, :nb] = perm[pos:pos + nb]
        pos += nb
    kc, vc = (torch.randn(pool, hkv, bs, d, generator=g, device="cuda", dtype=torch.float16) for _ in range(2))
    q = torch.randn(len(lens), hq, d, generator=g, device="cuda", dtype=torch.float16)
    bt, cl = tables.cuda(), torch.tensor(lens, dtype=torch.int32, device="cuda")
    sizes = [len(lens), hq, hkv, d, pool, bs, bt.shape[1], max(lens)]
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    out = torch.full_like(q, float("nan"))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        rc = lib.ak_paged_decode_noalloc(p(q), p(kc), p(vc), p(bt), p(cl), p(out), *sizes, d ** -0.5, part,
                                         ctypes.c_void_p(side.cuda_stream))
    res = dict(capture_rc=rc, error=(lib.ak_last_error() or b"").decode() if rc else "")
    if rc == 0:
        need = lib.ak_paged_decode_workspace_size(len(lens), hq, d, max(lens), part)
        ws = torch.empty(need, dtype=torch.uint8, device="cuda")
        counters = torch.zeros(len(lens) * hkv, dtype=torch.int32, device="cuda")
        want = torch.empty_like(q)
        rc2 = lib.ak_paged_decode_fused(p(q), p(kc), p(vc), p(bt), p(cl), p(want), *sizes, d ** -0.5, part,
                                        p(ws), need, p(counters), counters.numel(),
                                        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        # the first launch of a graph executable may set up the runtime's own
        # state for it: free memory is compared over the replays after it
        equal, free = [], [torch.cuda.mem_get_info()[0]]
        for _ in range(4):
            out.fill_(float("nan"))
            graph.replay()
            torch.cuda.synchronize()
            equal.append(bool(torch.equal(out, want)))
            free.append(torch.cuda.mem_get_info()[0])
        res.update(fused_rc=rc2, replays_equal=equal, first_replay_free_delta=free[1] - free[0],
                   free_unchanged=len(set(free[1:])) == 1, finite=bool(torch.isfinite(want).all()))
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
