"""Benchmark of the attention hot path on one MI355X; prints ONE JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--cpu-seconds S] [--settle-seconds T]

Headline (``value``): causal flash prefill, B=2, H=32, N=8192, D=128 fp16
(where the north-star target is stated), in TFLOP/s with
the reference's FLOP convention 4*B*H*N^2*D/2 (bench/bench.py:153).  A step is
one prefill call over that batch with inputs already resident in HBM.  Each
workload first runs untimed for --settle-seconds (the GPU's clock leaves its
idle state), then W untimed warmup steps, then the K timed steps.

The same line carries, under ``workloads``, the other BASELINE configs measured
the same way: non-causal prefill, the N=8191 variant, the two
paged split-K decode configs in KV GB/s with the reference's byte convention
sum(ctx)*Hkv*D*2*2 (bench/bench.py:199-200), two grouped-query decode layers (4
and 8 query heads per kv head) at the library's default partition, the paged
cache writer (K/V rows read + written, GB/s), and a packed variable-length GQA
prefill.

``roofline`` is the headline kernel's algorithmic FLOP per launch divided by its
mean launch duration (HIP events on the launch stream, inside the timed
region), against the 2.5 PFLOP/s dense fp16 MFMA peak.  Every workload is
also timed a second way, ``flushed``: K more steps, each after 512 MiB of
device memory is overwritten (outside the step's start/end events), median
reported, as the reference times every rep after an L2 flush.
``measured_ceilings`` times hipBLASLt's 8192^3 fp16 GEMM, a 2 GiB device copy
and a 2 GiB read-only stream in the same run, the same way; each roofline also
carries its rate as a fraction of the matching one (``frac_of_measured_ceiling``:
prefill against the GEMM, decode against the read stream, the cache writer
against the copy).  ``cpu_baseline`` times
the numpy oracle (oracle/attention.py) on a bounded sample of the same
workload on this host's cores.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "flash-attention-from-scratch_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_FP16_TFLOPS = 2500.0   # MI355X dense fp16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
# HBM bytes per launch of each workload's dominant kernel, from the committed
# rocprofv3 FETCH_SIZE/WRITE_SIZE passes (scaled by a 1 GiB copy; see profiles/).
TRAFFIC_FILE = ROOT / "profiles" / "traffic.json"


def measured_traffic(name):
    try:
        return json.loads(TRAFFIC_FILE.read_text()).get(name)
    except (OSError, ValueError):
        return None


def prefill_flops(b, h, n, d, causal):
    """The reference's prefill FLOP convention (bench/bench.py:153): 4*B*H*N^2*D, halved if causal."""
    return 4.0 * b * h * n * n * d * (0.5 if causal else 1.0)


def decode_kv_bytes(lens, hkv, d):
    """The reference's decode byte convention (bench/bench.py:199-200): K and V,
    fp16, sum(ctx) * Hkv * D * 2 * 2."""
    return float(sum(int(c) for c in lens)) * hkv * d * 2 * 2


def torch_attention_fp32(q, k, v, causal, scale):
    """softmax(scale q k^T, keys after the query masked if causal) v in float32 on
    the GPU, for one [n, D] slice: the accuracy column of the GPU workloads
    (the numpy oracle is reserved for the tests and the CPU baseline)."""
    import torch

    q, k, v = (t.float().contiguous() for t in (q, k, v))
    s = (q @ k.t().contiguous()) * scale
    if causal:
        mask = torch.ones(s.shape, dtype=torch.bool, device=s.device).triu(1)
        s = s.masked_fill(mask, float("-inf"))
    return torch.softmax(s, dim=-1) @ v


def log(msg):
    print(msg, file=sys.stderr, flush=True)


# Seconds of untimed calls before each workload's W warmup steps (--settle-seconds).
# On MI355X a kernel stream started from idle runs about 6% slower for its first
# ~50 ms (causal prefill, same box: 990 TFLOP/s after 5 warmup steps, 1051 after
# 50, 1056 in a long-running loop), so a few steps of warmup measure the ramp,
# not the steady state a serving or training loop runs in.
SETTLE_S = 0.25


def timed_steps(fn, steps, warmup):
    """The driver's protocol (attnkernels.timing.steady_steps): settle, W warmup
    steps, the K timed back-to-back steps between a start and an end event,
    K more steps with an event at each boundary (per-step median), then K
    flushed steps (512 MiB overwritten before each, outside its events)."""
    from attnkernels import timing

    return timing.steady_steps(fn, steps, warmup, settle_s=SETTLE_S)


def timing_fields(t, steps, work, unit):
    """The per-workload timing columns: `value` from the K timed back-to-back
    steps (wall clock), `kernel_ms_mean` from the two events around them,
    `kernel_ms_median` from the marked steps, `flushed` from the K flushed
    steps; `work` is FLOP (unit TFLOP/s) or bytes (GB/s) per step."""
    from attnkernels.timing import FLUSH_BYTES

    scale, peak = (1e12, PEAK_FP16_TFLOPS) if unit == "TFLOP/s" else (1e9, PEAK_HBM_GBS)

    def rate(ms):
        return work / (ms * 1e-3) / scale

    ms = t["total_ms"] / steps
    key = "kernel_tflops" if unit == "TFLOP/s" else "kernel_gbs"
    return {"value": round(rate(ms), 2), "unit": unit, "ms_per_step": round(ms, 4),
            "kernel_ms_mean": round(t["mean_ms"], 4), "kernel_ms_median": round(t["median_ms"], 4),
            key: round(rate(t["mean_ms"]), 2), "frac_of_peak": round(rate(t["mean_ms"]) / peak, 4),
            "flushed": {"flush_bytes": FLUSH_BYTES, "steps": steps, "kernel_ms_mean": round(t["flushed_mean_ms"], 4),
                        "kernel_ms_median": round(t["flushed_median_ms"], 4),
                        "value": round(rate(t["flushed_median_ms"]), 2), "unit": unit,
                        "frac_of_peak": round(rate(t["flushed_median_ms"]) / peak, 4)},
            "calls_before_timed": t["calls_before_timed"]}


def measured_ceilings(steps, warmup):
    """What this GPU sustains in the same run, timed like the workloads: an
    8192^3 fp16 GEMM (hipBLASLt through torch.mm) on normal random inputs, a
    2 GiB device-to-device copy (read + write bytes), and 2 GiB read once by
    the library's streaming checksum.  The reference's bench reports its
    kernels against a GEMM and a copy (bench/bench.py:119-131); decode only
    reads, and reads faster than a copy moves, so its rates are reported
    against the read stream."""
    import torch

    import attnkernels as ak

    n = 8192
    g = torch.Generator(device="cuda").manual_seed(0)
    a, b = (torch.randn(n, n, generator=g, device="cuda", dtype=torch.float16) for _ in range(2))
    c = torch.empty_like(a)
    t = timed_steps(lambda: torch.mm(a, b, out=c), steps, warmup)
    gemm = 2.0 * n ** 3 / (t["mean_ms"] * 1e-3) / 1e12
    del a, b, c
    nbytes = 2 << 30
    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    t = timed_steps(lambda: dst.copy_(src), steps, warmup)
    copy = 2.0 * nbytes / (t["mean_ms"] * 1e-3) / 1e9
    del dst
    ext = ak.load_extension()
    acc = torch.zeros(4, dtype=torch.int32, device="cuda")
    t = timed_steps(lambda: ext.stream_checksum(src, acc), steps, warmup)
    read = nbytes / (t["mean_ms"] * 1e-3) / 1e9
    del src
    torch.cuda.empty_cache()
    return {"fp16_gemm": {"value": round(gemm, 1), "unit": "TFLOP/s", "what": "torch.mm 8192^3 fp16, N(0,1) inputs"},
            "device_copy": {"value": round(copy, 1), "unit": "GB/s", "what": "2 GiB device-to-device copy, read + write"},
            "read_stream": {"value": round(read, 1), "unit": "GB/s",
                            "what": "2 GiB read once (ak_stream_checksum: a contiguous chunk per CU, 16-byte "
                                    "non-temporal loads, 16 in flight per lane); the ceiling of the decode kernels, which only read their K/V"}}


# Values of the dense prefill inputs (--inputs): the benchmark's are normal
# random; the others switch fewer bits in the matrix core and exist for the
# power-limit diagnostic (the same sweep as benchsuite's input_activity).
INPUTS = "randn"


def prefill_case(b, h, n, d, causal, steps, warmup, seed=0):
    import numpy as np
    import torch

    import attnkernels as ak
    from attnkernels.benchsuite import activity_tensor

    g = torch.Generator(device="cuda").manual_seed(seed)
    q, k, v = (activity_tensor(INPUTS, (b, h, n, d), g) for _ in range(3))
    fn = lambda: ak.flash_attention(q, k, v, causal=causal)  # noqa: E731
    out = fn()
    torch.cuda.synchronize()
    ref = torch_attention_fp32(q[0, 0], k[0, 0], v[0, 0], causal, d ** -0.5)
    err = float((out[0, 0].float() - ref).abs().max())
    del out, ref
    t = timed_steps(fn, steps, warmup)
    flops = prefill_flops(b, h, n, d, causal)
    res = dict(workload=f"prefill B={b} H={h} N={n} D={d} {'causal' if causal else 'non-causal'}"
                        + ("" if INPUTS == "randn" else f" [{INPUTS} inputs]"),
               **timing_fields(t, steps, flops, "TFLOP/s"), flop_per_launch=flops, max_abs_err=float(f"{err:.3g}"))
    del q, k, v
    torch.cuda.empty_cache()
    return res


def decode_case(lens, hkv, d, bs, partition, steps, warmup, seed=0, hq=None):
    import numpy as np
    import torch

    import attnkernels as ak

    hq = hkv if hq is None else hq
    if partition is None:  # the library's default split rule
        partition = ak.decode_partition(len(lens), hkv, max(lens))
    nblk = [-(-c // bs) for c in lens]
    pool = -(-sum(nblk) * 11 // 10)
    rng = np.random.default_rng(seed)
    perm = rng.permutation(pool).astype(np.int32)
    bt = np.zeros((len(lens), max(nblk)), np.int32)
    pos = 0
    for i, nb in enumerate(nblk):
        bt[i, :nb] = perm[pos:pos + nb]
        pos += nb
    g = torch.Generator(device="cuda").manual_seed(seed)
    shape = (pool, hkv, bs, d)
    kc = torch.randn(shape, generator=g, device="cuda", dtype=torch.float16)
    vc = torch.randn(shape, generator=g, device="cuda", dtype=torch.float16)
    q = torch.randn(len(lens), hq, d, generator=g, device="cuda", dtype=torch.float16)
    btd = torch.from_numpy(bt).cuda()
    cld = torch.tensor(lens, dtype=torch.int32, device="cuda")
    max_ctx = max(lens)
    fn = lambda: ak.paged_decode(q, kc, vc, btd, cld, max_ctx, partition_size=partition)  # noqa: E731
    out = fn()
    torch.cuda.synchronize()
    # Sequence 0 gathered through its block table, every query head against kv head h // G.
    pages = torch.from_numpy(bt[0, :nblk[0]]).long().cuda()
    kseq = kc[pages].permute(1, 0, 2, 3).reshape(hkv, -1, d)[:, :lens[0]]
    vseq = vc[pages].permute(1, 0, 2, 3).reshape(hkv, -1, d)[:, :lens[0]]
    grp = hq // hkv
    err = 0.0
    for kvh in range(hkv):
        ref = torch_attention_fp32(q[0, kvh * grp:(kvh + 1) * grp], kseq[kvh], vseq[kvh], False, d ** -0.5)
        err = max(err, float((out[0, kvh * grp:(kvh + 1) * grp].float() - ref).abs().max()))
    del out, kseq, vseq
    t = timed_steps(fn, steps, warmup)
    nbytes = decode_kv_bytes(lens, hkv, d)
    res = dict(workload=f"paged decode B={len(lens)} Hq={hq} Hkv={hkv} D={d} bs={bs} P={partition} "
                        f"sum_ctx={sum(lens)} max_ctx={max_ctx}",
               **timing_fields(t, steps, nbytes, "GB/s"), bytes_per_step=nbytes, splits=-(-max_ctx // partition),
               max_abs_err=float(f"{err:.3g}"))
    del kc, vc, q
    torch.cuda.empty_cache()
    return res


def varlen_case(lens, h, hkv, d, causal, steps, warmup, seed=0):
    """Packed variable-length causal prefill with GQA (no padding): FLOP is the
    sum over sequences of the reference convention 4*H*n^2*D(/2 if causal)."""
    import numpy as np
    import torch

    import attnkernels as ak

    total = sum(lens)
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn(total, h, d, generator=g, device="cuda", dtype=torch.float16)
    k = torch.randn(total, hkv, d, generator=g, device="cuda", dtype=torch.float16)
    v = torch.randn(total, hkv, d, generator=g, device="cuda", dtype=torch.float16)
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32, device="cuda")
    fn = lambda: ak.flash_attention_varlen(q, k, v, cu, max(lens), causal=causal)  # noqa: E731
    out = fn()
    torch.cuda.synchronize()
    n0 = lens[0]  # first sequence, first 2 query heads (both read kv head 0)
    err = max(float((out[:n0, hh].float() - torch_attention_fp32(q[:n0, hh], k[:n0, 0], v[:n0, 0], causal,
                                                                d ** -0.5)).abs().max()) for hh in range(2))
    del out
    t = timed_steps(fn, steps, warmup)
    flops = sum(prefill_flops(1, h, n, d, causal) for n in lens)
    res = dict(workload=f"varlen prefill {len(lens)} seqs total={total} max={max(lens)} H={h} Hkv={hkv} D={d} "
                        f"{'causal' if causal else 'non-causal'}",
               **timing_fields(t, steps, flops, "TFLOP/s"), flop_per_launch=flops, max_abs_err=float(f"{err:.3g}"))
    del q, k, v
    torch.cuda.empty_cache()
    return res


def cache_write_case(tokens, hkv, d, bs, steps, warmup, seed=0):
    """Paged KV-cache writer: ``tokens`` new K/V rows (a batch of prompts)
    scattered into a shuffled page pool; bytes = K+V read + written."""
    import numpy as np
    import torch

    import attnkernels as ak

    g = torch.Generator(device="cuda").manual_seed(seed)
    key = torch.randn(tokens, hkv, d, generator=g, device="cuda", dtype=torch.float16)
    value = torch.randn(tokens, hkv, d, generator=g, device="cuda", dtype=torch.float16)
    pool = -(-tokens // bs) * 11 // 10 + 1
    kc = torch.zeros(pool, hkv, bs, d, device="cuda", dtype=torch.float16)
    vc = torch.zeros_like(kc)
    pages = np.random.default_rng(seed).permutation(pool)[: -(-tokens // bs)]
    slots_np = (pages[np.arange(tokens) // bs] * bs + np.arange(tokens) % bs).astype(np.int64)
    slots = torch.from_numpy(slots_np).cuda()
    fn = lambda: ak.reshape_and_cache(key, value, kc, vc, slots)  # noqa: E731
    fn()
    torch.cuda.synchronize()
    # Bit-exact: token i's rows sit at page slot // bs, row slot % bs of each cache,
    # and the pages no token maps to are still zero.
    page_of, row_of = slots // bs, slots % bs
    mism = int((kc[page_of, :, row_of, :] != key).sum()) + int((vc[page_of, :, row_of, :] != value).sum())
    unused = torch.ones(pool, dtype=torch.bool, device="cuda")
    unused[torch.from_numpy(pages).cuda()] = False
    mism += int(kc[unused].count_nonzero()) + int(vc[unused].count_nonzero())
    t = timed_steps(fn, steps, warmup)
    nbytes = 2 * tokens * hkv * d * 2 * 2 + tokens * 8
    res = dict(workload=f"paged cache write T={tokens} Hkv={hkv} D={d} bs={bs} fp16 (shuffled pages)",
               **timing_fields(t, steps, nbytes, "GB/s"), bytes_per_step=nbytes, mismatched_elements=mism)
    del key, value, kc, vc
    torch.cuda.empty_cache()
    return res


def cpu_baseline(seconds):
    """The numpy fp32 oracle on (batch, head) slices of the headline workload,
    on this host's cores, for about ``seconds`` of CPU work."""
    import numpy as np

    import oracle

    import torch

    try:
        from threadpoolctl import threadpool_info
        threads = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:  # noqa: BLE001
        threads = os.cpu_count() or 1
    n, d = 8192, 128
    rng = np.random.default_rng(0)
    q, k, v = (rng.standard_normal((n, d), dtype=np.float32).astype(np.float16) for _ in range(3))
    oracle.attention_fp32(q[:512], k[:512], v[:512], True)  # warm the BLAS threads
    done, t0 = 0, time.perf_counter()
    while True:
        oracle.attention_fp32(q, k, v, True)
        done += 1
        if time.perf_counter() - t0 >= seconds:
            break
    el = time.perf_counter() - t0
    log(f"cpu oracle: {done} slices of causal N={n} D={d} in {el:.1f} s")
    flops = oracle.prefill_flops(1, done, n, d, True)
    return dict(value=round(flops / el / 1e12, 5), unit="TFLOP/s", cores=int(threads), kind="port",
                sample=f"{done} (batch, head) slices of causal N=8192 D=128 through the numpy fp32 "
                       f"oracle, {el:.1f} s, os.cpu_count()={os.cpu_count()}",
                os_cpu_count=os.cpu_count(), torch_num_threads=torch.get_num_threads(), blas_threads=int(threads),
                configs=cpu_configs())


def cpu_configs():
    """The same oracle on the other reference configurations (wall time,
    time.perf_counter; nothing extrapolated): prefill B=1 H=4 N=256 D=64 and
    B=4 H=16 N=2048 D=64 (non-causal, scale 1/8) whole; the ragged paged
    decode of configs[3] whole (the bench's 64 seeded lengths, Hq=Hkv=32,
    D=128, pages of 16); and one whole sequence of the long decode of
    configs[4] at D=128 and D=64 (32768 tokens, 32 heads; the batch holds 8
    such sequences).  A configuration runs once, and twice more (the median
    is reported) when one run takes under 3 s."""
    import statistics

    import numpy as np
    import torch

    import oracle

    def median_s(fn):
        ts = []
        while len(ts) < (1 if ts and ts[0] >= 3.0 else 3):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts), len(ts)

    def paged_cache(lens, h, d, bs, seed):
        # the caches are drawn on the GPU and copied to host memory: drawing
        # 10^8-10^9 normals on the host takes longer than the oracle itself
        nblk = [-(-n // bs) for n in lens]
        total = sum(nblk) + len(lens)
        perm = torch.randperm(total, generator=torch.Generator().manual_seed(seed)).to(torch.int32).numpy()
        tables = np.zeros((len(lens), max(nblk)), np.int32)
        pos = 0
        for b, nb in enumerate(nblk):
            tables[b, :nb] = perm[pos:pos + nb]
            pos += nb
        g = torch.Generator(device="cuda").manual_seed(seed)
        kc, vc = (torch.randn((total, h, bs, d), generator=g, device="cuda", dtype=torch.float16).cpu().numpy()
                  for _ in range(2))
        return kc, vc, tables, np.asarray(lens, np.int32)

    rng = np.random.default_rng(1)
    rows = []
    for (b, h, n, d) in ((1, 4, 256, 64), (4, 16, 2048, 64)):
        q, k, v = (rng.standard_normal((b, h, n, d), dtype=np.float32).astype(np.float16) for _ in range(3))
        sec, runs = median_s(lambda: oracle.attention_fp32(q, k, v, False, 0.125))
        log(f"cpu oracle: prefill B={b} H={h} N={n} D={d} {sec:.2f} s ({runs} runs)")
        rows.append(dict(config=f"prefill B={b} H={h} N={n} D={d} non-causal",
                         value=round(oracle.prefill_flops(b, h, n, d, False) / sec / 1e12, 5), unit="TFLOP/s",
                         seconds=round(sec, 4), runs=runs, stat="median" if runs > 1 else "single run"))
    lens4 = torch.randint(1, 4097, (64,), generator=torch.Generator().manual_seed(4)).tolist()
    for lens, d, what in ((lens4, 128, "configs[3] paged decode, all 64 ragged sequences"),
                          ([32768], 128, "configs[4] paged decode D=128, one whole 32768-token sequence"),
                          ([32768], 64, "configs[4] paged decode D=64, one whole 32768-token sequence")):
        kc, vc, bt, cl = paged_cache(lens, 32, d, 16, seed=4)
        qd = rng.standard_normal((len(lens), 32, d), dtype=np.float32).astype(np.float16)
        sec, runs = median_s(lambda: oracle.paged_decode_fp32(qd, kc, vc, bt, cl))
        log(f"cpu oracle: {what} {sec:.2f} s ({runs} runs)")
        rows.append(dict(config=f"{what} (sum_ctx={sum(lens)}) Hq=Hkv=32 D={d} bs=16",
                         value=round(oracle.decode_kv_bytes(lens, 32, d) / sec / 1e9, 3), unit="GB/s",
                         seconds=round(sec, 4), runs=runs, stat="median" if runs > 1 else "single run"))
        del kc, vc
    return rows


def main():
    global SETTLE_S, INPUTS
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--settle-seconds", type=float, default=SETTLE_S,
                    help="untimed calls of each workload before its warmup steps (clock settle)")
    ap.add_argument("--only", default="all",
                    help="all | headline | prefill | decode | comma list of workload names")
    ap.add_argument("--inputs", choices=("randn", "signs", "ones", "zeros"), default="randn",
                    help="values of the dense prefill inputs; the benchmark's are randn, the others are "
                         "a diagnostic of the power-limited clock (fewer bits switching in the matrix core)")
    ap.add_argument("--calib-copy", action="store_true",
                    help="first run one plain 1 GiB device-to-device copy: the known-size kernel "
                         "that scales rocprofv3 FETCH_SIZE/WRITE_SIZE readings to bytes")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path; run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    import torch

    import attnkernels as ak

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    ak.load_extension()
    torch.manual_seed(0)
    if args.calib_copy:
        src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        torch.cuda.empty_cache()
    K, W = args.steps, args.warmup
    SETTLE_S = max(0.0, args.settle_seconds)
    INPUTS = args.inputs
    lens4 = torch.randint(1, 4097, (64,), generator=torch.Generator().manual_seed(4)).tolist()
    lensv = torch.randint(512, 8193, (16,), generator=torch.Generator().manual_seed(5)).tolist()
    cases = {  # BASELINE.json configs[1..4]
        "prefill_d128_n8192_causal": lambda: prefill_case(2, 32, 8192, 128, True, K, W),
        "prefill_d64_n2048": lambda: prefill_case(4, 16, 2048, 64, False, K, W),
        "prefill_d128_n8191_causal": lambda: prefill_case(2, 32, 8191, 128, True, K, W),
        "decode_ragged64_d128": lambda: decode_case(lens4, 32, 128, 16, 512, K, W),
        "decode_long8_d128": lambda: decode_case([32768] * 8, 32, 128, 16, 256, K, W),
        "decode_long8_d64": lambda: decode_case([32768] * 8, 32, 64, 16, 256, K, W),
        # a Llama-3-8B-like decode layer: 4 query heads per kv head, the default partition
        "decode_gqa16_d128": lambda: decode_case([8192] * 16, 8, 128, 16, None, K, W, hq=32),
        # 8 query heads per kv head (the heaviest head group the kernels take), default partition
        "decode_g8_d128": lambda: decode_case([8192] * 8, 8, 128, 16, None, K, W, hq=64),
        # packed prompts of mixed lengths, 4 query heads per kv head, no padding
        "prefill_varlen_gqa": lambda: varlen_case(lensv, 32, 8, 128, True, K, W),
        # the step before decode reads the cache: append a batch of prompts' K/V to it
        "cache_write_t16k": lambda: cache_write_case(16384, 32, 128, 16, K, W),
    }
    groups = {"all": list(cases), "headline": ["prefill_d128_n8192_causal"],
              "prefill": [c for c in cases if c.startswith("prefill")],
              "layouts": ["prefill_d128_n8192_causal", "prefill_varlen_gqa", "cache_write_t16k"],
              "decode": ["prefill_d128_n8192_causal"] + [c for c in cases if c.startswith("decode")],
              "cache": ["prefill_d128_n8192_causal", "cache_write_t16k"]}
    selected = groups.get(args.only, [c for c in args.only.split(",") if c in cases])
    if not selected:
        raise SystemExit(f"--only: choose from {sorted(groups)} or a comma list of {sorted(cases)}")
    results = {}
    for name in selected:
        results[name] = cases[name]()
        log(json.dumps(results[name]))
    headline = results.get("prefill_d128_n8192_causal")
    # Measured after the workloads, on the same GPU, when the headline runs (not
    # in profiling runs of other workloads, whose traces it would lengthen).
    ceil = measured_ceilings(K, W) if headline is not None else None
    if ceil:
        log(json.dumps({"measured_ceilings": ceil}))

    def of_ceiling(ach, hbm, decode=False):
        if not ceil:
            return None
        return round(ach / ceil[("read_stream" if decode else "device_copy") if hbm else "fp16_gemm"]["value"], 4)

    workloads = []
    for k, v in results.items():
        if k == "prefill_d128_n8192_causal":
            continue
        t = measured_traffic(k)
        hbm = v["unit"] == "GB/s"
        ach = v["kernel_gbs"] if hbm else v["kernel_tflops"]
        peak = PEAK_HBM_GBS if hbm else PEAK_FP16_TFLOPS
        workloads.append(dict(name=k, **v, roofline={
            "bound": "hbm" if hbm else "mfma", "achieved": ach, "peak": peak, "unit": v["unit"],
            "frac": round(ach / peak, 4), "traffic": t["traffic_bytes"] if t else None,
            "frac_of_measured_ceiling": of_ceiling(ach, hbm, k.startswith("decode"))}))
    cpu = cpu_baseline(args.cpu_seconds) if args.cpu_seconds > 0 else None
    from attnkernels import build as akbuild
    digest = akbuild.sources_digest()  # names the kernel sources measured (profiles cite it)
    if headline is None:  # a profiling run of other workloads: report them only
        print(json.dumps({"workloads": workloads, "steps": K, "warmup": W, "sources_sha256": digest,
                          "cpu_baseline": cpu}), flush=True)
        return
    ach = headline["kernel_tflops"]
    line = {
        "metric": "prefill TFLOP/s (% MFMA peak); paged decode KV GB/s (% HBM peak)",
        "value": headline["value"], "unit": "TFLOP/s", "n_gpus": 1, "steps": K, "warmup": W, "settle_s": SETTLE_S,
        "ms_per_step": headline["ms_per_step"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic" if INPUTS == "randn" else f"synthetic, prefill inputs all {INPUTS} (diagnostic, not the benchmark)",
        "config": {"workload": headline["workload"] + " (BASELINE configs[2])", "global_batch": 2,
                   "seq_len": 8192, "heads": 32, "head_dim": 128, "causal": True, "parallelism": "none"},
        "max_abs_err": headline["max_abs_err"],
        # the same workload with 512 MiB written before each step (outside the
        # step's event pair), as the reference times every rep
        "flushed": headline["flushed"],
        "kernel_ms_mean": headline["kernel_ms_mean"], "kernel_ms_median": headline["kernel_ms_median"],
        "flop_per_launch": headline["flop_per_launch"], "calls_before_timed": headline["calls_before_timed"],
        "sources_sha256": digest,
        "roofline": {"bound": "mfma", "achieved": ach, "peak": PEAK_FP16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(ach / PEAK_FP16_TFLOPS, 4),
                     "traffic": (measured_traffic("prefill_d128_n8192_causal") or {}).get("traffic_bytes"),
                     "traffic_source": "profiles/traffic.json (rocprofv3 FETCH_SIZE+WRITE_SIZE, copy-scaled)",
                     "kernel": (measured_traffic("prefill_d128_n8192_causal") or {}).get("kernel",
                                                                                       "flash_prefill_kernel"),
                     "kernel_ms_mean": headline["kernel_ms_mean"],
                     # against the GEMM timed in this run (measured_ceilings)
                     "frac_of_measured_ceiling": of_ceiling(ach, False)},
        "measured_ceilings": ceil,
        "cpu_baseline": cpu,
        "workloads": workloads,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
