"""ak_paged_decode_fused (the split merge in the decode kernel: the last split
of each (sequence, kv head) to finish merges the partials) through the C-ABI,
against the two-kernel ak_paged_decode and the oracle on the same inputs.

The merge is an LSE rule over partials written with agent-coherent stores and
counted by an agent-scope atomic; these tests check what that protocol must
guarantee: every output row matches the oracle, the counters are back at zero
after every call, and calls that reuse one workspace and one counter array
with new data never see the previous call's partials."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from conftest import PKG_DIR, TOL, max_err

pytestmark = pytest.mark.gpu

LIB = PKG_DIR / "attnkernels" / "libattnkernels.so"
FUSED_MAX_SPLITS = 32  # more splits go to the reduce kernel (kFusedMaxSplits)


@pytest.fixture(scope="module")
def lib():
    L = ctypes.CDLL(str(LIB))
    vp, i64, f64 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_double
    L.ak_last_error.restype = ctypes.c_char_p
    L.ak_paged_decode_workspace_size.argtypes = [i64] * 5
    L.ak_paged_decode_workspace_size.restype = ctypes.c_size_t
    L.ak_paged_decode.argtypes = [vp] * 6 + [i64] * 8 + [f64, i64, vp, ctypes.c_size_t, vp]
    L.ak_paged_decode_fused.argtypes = [vp] * 6 + [i64] * 8 + [f64, i64, vp, ctypes.c_size_t, vp, i64, vp]
    return L


def ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


class Case:
    """One paged cache on the device plus its oracle output."""

    def __init__(self, lens, hq, hkv, d, seed, bad_pages=()):
        kc, vc, bt, cl = oracle.make_paged_cache(lens, hkv, d, block_size=16, extra_blocks=3, seed=seed)
        for b, j in bad_pages:  # page ids outside the pool: their tokens drop out
            bt[b, j] = kc.shape[0] + 5
        q = np.random.default_rng(seed + 1).standard_normal((len(lens), hq, d), dtype=np.float32)
        self.q = q.astype(np.float16)
        self.kc, self.vc, self.bt, self.cl = kc, vc, bt, cl
        self.dev = [torch.from_numpy(a).cuda() for a in (self.q, kc, vc, bt, cl)]
        self.lens, self.hq, self.hkv, self.d = lens, hq, hkv, d

    def oracle(self):
        bt = self.bt.copy()
        bad = (bt < 0) | (bt >= self.kc.shape[0])
        if not bad.any():
            return oracle.paged_decode_fp32(self.q, self.kc, self.vc, bt, self.cl)
        # tokens on out-of-range pages drop out of the softmax: the oracle on the
        # remaining tokens, one sequence and page at a time
        out = np.zeros(self.q.shape, np.float32)
        for b, n in enumerate(self.lens):
            keep = [t for t in range(n) if not bad[b, t // 16]]
            if not keep:
                continue
            k = np.stack([self.kc[bt[b, t // 16], :, t % 16] for t in keep], 1).astype(np.float32)
            v = np.stack([self.vc[bt[b, t // 16], :, t % 16] for t in keep], 1).astype(np.float32)
            g = self.hq // self.hkv
            k, v = np.repeat(k, g, 0), np.repeat(v, g, 0)
            s = np.einsum("hd,htd->ht", self.q[b].astype(np.float32), k) / np.sqrt(self.d)
            p = np.exp(s - s.max(1, keepdims=True))
            out[b] = np.einsum("ht,htd->hd", p / p.sum(1, keepdims=True), v)
        return out

    def run(self, lib, partition, fused, ws, counters):
        qd, kcd, vcd, btd, cld = self.dev
        out = torch.full_like(qd, float("nan"))
        sizes = [len(self.lens), self.hq, self.hkv, self.d, self.kc.shape[0], 16, self.bt.shape[1],
                 max(max(self.lens), 1)]
        need = lib.ak_paged_decode_workspace_size(len(self.lens), self.hq, self.d, sizes[-1], partition)
        args = [ptr(qd), ptr(kcd), ptr(vcd), ptr(btd), ptr(cld), ptr(out), *sizes, self.d ** -0.5, partition,
                ptr(ws) if need else None, need]
        if fused:
            rc = lib.ak_paged_decode_fused(*args, ptr(counters), counters.numel(), stream())
        else:
            rc = lib.ak_paged_decode(*args, stream())
        assert rc == 0, lib.ak_last_error()
        return out


def buffers(lib, case, partition, n_counters=4096):
    need = lib.ak_paged_decode_workspace_size(len(case.lens), case.hq, case.d, max(max(case.lens), 1), partition)
    ws = torch.full((max(need, 4) // 4,), float("nan"), dtype=torch.float32, device="cuda")
    return ws, torch.zeros(n_counters, dtype=torch.int32, device="cuda")


@pytest.mark.parametrize("lens,hq,hkv,d,partition", [
    ([700, 300, 1], 8, 8, 128, 256),          # 3 splits, G = 1
    ([3000, 20, 1500], 16, 4, 128, 256),      # 12 splits, G = 4
    ([4096], 64, 8, 128, 256),                # 16 splits, G = 8
    ([2000, 2000], 16, 8, 64, 256),           # 8 splits, G = 2, D = 64
    ([8192], 32, 8, 128, 256),                # 32 splits (the most merged in the kernel)
    ([8448], 32, 8, 128, 256),                # 33 splits: the reduce kernel
    ([8192, 3000], 64, 8, 128, 256),          # 32 splits, G = 8
    ([8000, 100], 8, 8, 64, 256),             # 32 splits, G = 1, D = 64
])
def test_fused_matches_reduce_and_oracle(lib, lens, hq, hkv, d, partition):
    print(f"fused case lens={lens} hq={hq} hkv={hkv} d={d} P={partition}", flush=True)
    c = Case(lens, hq, hkv, d, seed=sum(lens) % 997)
    ws, counters = buffers(lib, c, partition)
    fused = c.run(lib, partition, True, ws, counters)
    torch.cuda.synchronize()
    assert int(torch.count_nonzero(counters)) == 0  # every call leaves its counters at zero
    plain = c.run(lib, partition, False, ws, None)
    torch.cuda.synchronize()
    ref = c.oracle()
    assert max_err(fused, ref) < TOL[d]
    assert max_err(plain, ref) < TOL[d]
    assert max_err(fused, plain) < 1e-3
    if -(-max(lens) // partition) > FUSED_MAX_SPLITS:
        assert torch.equal(fused, plain)  # the same reduce kernel


def test_fused_reuse_never_reads_an_earlier_call(lib):
    """Five calls with new q and caches but the same workspace (pre-filled with
    NaN) and counters, alternating shapes and split counts: a partial left by
    an earlier call would put wrong (or NaN) rows in a later output."""
    ws = torch.full((8 << 20,), float("nan"), dtype=torch.float32, device="cuda")
    counters = torch.zeros(4096, dtype=torch.int32, device="cuda")
    shapes = [([2500, 2500, 900], 32, 8, 128, 256), ([600, 601], 16, 4, 64, 256),
              ([2500, 2500, 900], 32, 8, 128, 512), ([5000], 64, 8, 128, 256), ([300, 4000, 17], 8, 8, 128, 256)]
    for i, (lens, hq, hkv, d, p) in enumerate(shapes):
        print(f"reuse call {i}: lens={lens} hq={hq} hkv={hkv} d={d} P={p}", flush=True)
        c = Case(lens, hq, hkv, d, seed=100 + i)
        out = c.run(lib, p, True, ws, counters)
        torch.cuda.synchronize()
        assert torch.isfinite(out).all()
        assert max_err(out, c.oracle()) < TOL[d]
        assert int(torch.count_nonzero(counters)) == 0


def test_fused_empty_sequences_and_bad_pages(lib):
    """A sequence with no context gets a zero row; a split whose pages are all
    out of range has no weight; a sequence whose every page is out of range
    gets a zero row (as the reduce gives them)."""
    lens = [1000, 0, 1200, 600]
    bad = [(0, j) for j in range(16, 32)] + [(3, j) for j in range(38)]  # split 1 of seq 0; all of seq 3
    c = Case(lens, 16, 4, 128, seed=31, bad_pages=bad)
    ws, counters = buffers(lib, c, 256)
    out = c.run(lib, 256, True, ws, counters)
    torch.cuda.synchronize()
    assert int(torch.count_nonzero(counters)) == 0
    assert torch.isfinite(out).all()
    assert float(out[1].abs().max()) == 0.0 and float(out[3].abs().max()) == 0.0
    assert max_err(out, c.oracle()) < TOL[128]


def test_fused_rejects_short_counter_array(lib):
    c = Case([1000, 1000], 16, 8, 128, seed=5)
    ws, _ = buffers(lib, c, 256)
    qd, kcd, vcd, btd, cld = c.dev
    out = torch.empty_like(qd)
    counters = torch.zeros(15, dtype=torch.int32, device="cuda")  # needs batch * num_kv_heads = 16
    rc = lib.ak_paged_decode_fused(ptr(qd), ptr(kcd), ptr(vcd), ptr(btd), ptr(cld), ptr(out), 2, 16, 8, 128,
                                   c.kc.shape[0], 16, c.bt.shape[1], 1000, 128 ** -0.5, 256, ptr(ws),
                                   ws.numel() * 4, ptr(counters), 15, stream())
    assert rc == 1
    assert b"counters" in lib.ak_last_error()


def test_extension_decode_steps_on_one_stream(ext):
    """The torch entry point keeps one counter array per stream: many decode
    calls of different shapes in a row on the current stream, then on a second
    stream, all against the oracle."""
    import attnkernels as ak
    side = torch.cuda.Stream()
    for i, (lens, hq, hkv, d) in enumerate([([3000, 1000], 32, 8, 128), ([200] * 9, 16, 16, 64),
                                            ([8000], 64, 8, 128), ([3000, 1000], 32, 8, 128)]):
        c = Case(lens, hq, hkv, d, seed=200 + i)
        qd, kcd, vcd, btd, cld = c.dev
        torch.cuda.synchronize()  # the inputs were copied on the current stream
        for s in (torch.cuda.current_stream(), side):
            with torch.cuda.stream(s):
                out = ak.paged_decode(qd, kcd, vcd, btd, cld, max(lens), partition_size=256)
            s.synchronize()
            assert max_err(out, c.oracle()) < TOL[d]


@pytest.mark.parametrize("hq,d", [(32, 128), (64, 128), (16, 64)])
def test_small_and_large_grid_wave_counts_agree(lib, hq, d):
    """One sequence of 16384 tokens, 8 kv heads: partition 512 gives 256
    workgroups (the grouped-query kernel's 8-wave workgroups, merged in the
    kernel), partition 256 gives 512 (4-wave workgroups, merged by the reduce
    kernel).  Both against the oracle and each other."""
    print(f"wave counts hq={hq} d={d}", flush=True)
    c = Case([16384], hq, 8, d, seed=hq + d)
    ref = c.oracle()
    outs = []
    for p in (512, 256):
        ws, counters = buffers(lib, c, p)
        outs.append(c.run(lib, p, True, ws, counters))
        torch.cuda.synchronize()
        assert int(torch.count_nonzero(counters)) == 0
        assert max_err(outs[-1], ref) < TOL[d]
    assert max_err(outs[0], outs[1]) < 1e-3
