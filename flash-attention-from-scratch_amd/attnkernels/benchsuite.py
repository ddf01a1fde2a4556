"""Comparison benchmark of the attention kernels on one MI355X; writes a JSON file.

The counterpart of the reference's comparison harness (bench/bench.py:142-332),
with the same sections:

* ``prefill``: this build's flash prefill against PyTorch's SDPA backends over a
  sweep of sequence lengths at a constant token count, D in {64, 128}, causal
  and not (bench/bench.py:142-189);
* ``decode``: paged split-K decode (and the same kernel with one split) against
  "gather the pages, then SDPA" and SDPA on an already contiguous cache, for a
  Llama-3-8B-like layer, Hq=32, Hkv=8, D=128, page size 16
  (bench/bench.py:194-268);
* ``split_ablation``: decode bandwidth for every power-of-two partition, to
  check the ``decode_partition`` rule on 256 CUs (bench/bench.py:271-278);
* ``ragged``: a batch with mixed context lengths (bench/bench.py:281-287);
* ``roofs``: practical ceilings of this GPU, a large device copy and an
  8192^3 fp16 GEMM (bench/bench.py:111-124).

Timing: hipEvents around each call after a warm-up, median over 3..50 calls
(about 0.3 s per case).  Before every timed call a 512 MiB buffer is cleared,
outside the timed region, so the 256 MB Infinity Cache does not serve data
from the previous call.

SDPA is always pinned to its flash / memory-efficient backends: its math
backend (batched matmuls on transposed views) is never run.

    python -m attnkernels.benchsuite --out results/mi355x.json [--quick]
    python -m attnkernels.report results/mi355x.json > results/mi355x.md
"""
from __future__ import annotations

import argparse
import datetime as dt
import json
import platform
import statistics
import sys
import time
from pathlib import Path

import torch
import torch.nn.functional as F

import attnkernels as ak
from attnkernels import reference as akref

try:
    from torch.nn.attention import SDPBackend, sdpa_kernel
except ImportError:  # older torch
    SDPBackend = sdpa_kernel = None

FLUSH_BYTES = 512 << 20
_flush_buf = None


def flush_caches():
    """Clear a 512 MiB buffer: evicts L2 and the Infinity Cache."""
    global _flush_buf
    if _flush_buf is None:
        _flush_buf = torch.empty(FLUSH_BYTES, dtype=torch.uint8, device="cuda")
    _flush_buf.zero_()


def median_ms(fn, warmup=1, budget_ms=300.0, lo=3, hi=50):
    """Median hipEvent time of fn() over lo..hi calls, each after a cache flush."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    samples, reps = [], hi
    while len(samples) < reps:
        flush_caches()
        t0.record()
        fn()
        t1.record()
        t1.synchronize()
        samples.append(t0.elapsed_time(t1))
        if len(samples) == 1:
            reps = int(min(hi, max(lo, budget_ms / max(samples[0], 1e-3))))
    return statistics.median(samples)


def extra_peak_mb(fn):
    """Peak device memory one call allocates on top of what is live (output included)."""
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    before = torch.cuda.memory_allocated()
    out = fn()
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated() - before
    del out
    return round(peak / 2**20, 1)


def sdpa_pinned(*backends):
    """SDPA restricted to the given backends (never the math path)."""
    def run(q, k, v, causal=False, attn_mask=None):
        with sdpa_kernel(list(backends)):
            return F.scaled_dot_product_attention(q, k, v, attn_mask=attn_mask, is_causal=causal)
    return run


def probe_sdpa_backends():
    """Which fused SDPA backends accept fp16 [B, H, N, 128] here."""
    found = {}
    if sdpa_kernel is None:
        return found
    q = torch.randn(1, 2, 256, 128, device="cuda", dtype=torch.float16)
    for name in ("FLASH_ATTENTION", "EFFICIENT_ATTENTION", "CUDNN_ATTENTION"):
        backend = getattr(SDPBackend, name, None)
        if backend is None:
            continue
        try:
            sdpa_pinned(backend)(q, q, q, True)
            torch.cuda.synchronize()
            found[name] = "ok"
        except Exception as e:  # noqa: BLE001
            found[name] = "unavailable: " + str(e).splitlines()[0][:200]
    found["MATH"] = "not run (batched matmuls on transposed views are avoided on this GPU pool)"
    return found


def fused_backends(found):
    return [getattr(SDPBackend, n) for n in ("FLASH_ATTENTION", "EFFICIENT_ATTENTION") if found.get(n) == "ok"]


def roofs():
    """Practical ceilings: 2 GiB device-to-device copy, 8192^3 fp16 GEMM."""
    src = torch.empty(2 << 30, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    ms = median_ms(lambda: dst.copy_(src))
    copy_gbs = 2 * src.numel() / (ms * 1e-3) / 1e9
    del src, dst
    a = torch.randn(8192, 8192, device="cuda", dtype=torch.float16)
    b = torch.randn(8192, 8192, device="cuda", dtype=torch.float16)
    ms = median_ms(lambda: torch.mm(a, b))
    gemm = 2 * 8192**3 / (ms * 1e-3) / 1e12
    del a, b
    torch.cuda.empty_cache()
    return dict(copy_gbs=round(copy_gbs, 1), fp16_gemm_tflops=round(gemm, 1))


def err_vs_fp32(out, q, k, v, causal):
    """Max abs error against fp32 attention on batch 0, heads 0-1."""
    ref = akref.attention_fp32(q[:1, :2], k[:1, :2], v[:1, :2], causal)
    return (out[:1, :2].float() - ref).abs().max().item()


def section_prefill(rows, quick, found):
    heads, tokens = 16, (4096 if quick else 16384)
    seqs = (512, 1024) if quick else (512, 1024, 2048, 4096, 8192)
    pinned = fused_backends(found)
    for d in (64, 128):
        for causal in (False, True):
            for n in seqs:
                b = max(1, tokens // n)
                g = torch.Generator(device="cuda").manual_seed(n + d)
                q, k, v = (torch.randn(b, heads, n, d, generator=g, device="cuda", dtype=torch.float16)
                           for _ in range(3))
                flops = 4.0 * b * heads * n * n * d * (0.5 if causal else 1.0)
                impls = {"flash_attention": lambda: ak.flash_attention(q, k, v, causal=causal)}
                if pinned:
                    impls["sdpa_fused"] = lambda: sdpa_pinned(*pinned)(q, k, v, causal)
                for name in ("FLASH_ATTENTION", "EFFICIENT_ATTENTION"):
                    if found.get(name) == "ok":
                        be = getattr(SDPBackend, name)
                        impls["sdpa_" + name.split("_")[0].lower()] = (
                            lambda be=be: sdpa_pinned(be)(q, k, v, causal))
                case = []
                for name, fn in impls.items():
                    try:
                        out = fn()
                        err = err_vs_fp32(out, q, k, v, causal)
                        del out
                        ms = median_ms(fn)
                        mem = extra_peak_mb(fn)
                    except Exception as e:  # noqa: BLE001  e.g. unsupported shape
                        print(f"prefill {name} d={d} N={n}: {e!r}"[:300], flush=True)
                        torch.cuda.empty_cache()
                        continue
                    case.append(dict(section="prefill", impl=name, batch=b, heads=heads, seq=n, head_dim=d,
                                     causal=causal, ms=round(ms, 4), tflops=round(flops / (ms * 1e-3) / 1e12, 2),
                                     peak_mem_mb=mem, max_abs_err=float(f"{err:.3g}")))
                base = next((r["ms"] for r in case if r["impl"] == "sdpa_fused"), None)
                for r in case:
                    r["speedup_vs_sdpa"] = round(base / r["ms"], 3) if base else None
                    rows.append(r)
                    print(f"prefill d={d} causal={int(causal)} B={b:2d} N={n:5d} {r['impl']:16s} "
                          f"{r['ms']:8.3f} ms {r['tflops']:8.1f} TFLOP/s err {r['max_abs_err']:.1e} "
                          f"x{r['speedup_vs_sdpa']}", flush=True)
                del q, k, v
                torch.cuda.empty_cache()


HQ, HKV, D, BS = 32, 8, 128, 16  # Llama-3-8B-like attention layer


def kv_bytes(lens, hkv=HKV, d=D):
    return sum(lens) * hkv * d * 2 * 2


def decode_case(rows, section, lens, wanted, found, partition=None, extra=None, seed=0):
    B = len(lens)
    gen = torch.Generator().manual_seed(seed)
    kc, vc, tables, clens = akref.make_paged_cache(lens, HKV, D, block_size=BS, generator=gen)
    q = torch.randn(B, HQ, D, device="cuda", dtype=torch.float16)
    max_ctx = max(lens)
    nblk = -(-max_ctx // BS)
    uniform = len(set(lens)) == 1
    pinned = fused_backends(found)
    impls = {}
    if "paged_split" in wanted:
        impls["paged_split"] = lambda: ak.paged_decode(q, kc, vc, tables, clens, max_ctx, partition_size=partition)
    if "paged_nosplit" in wanted:
        impls["paged_nosplit"] = lambda: ak.paged_decode(q, kc, vc, tables, clens, max_ctx,
                                                          partition_size=-(-max_ctx // ak.CHUNK) * ak.CHUNK)
    if "torch_gather_sdpa" in wanted and pinned:
        def gather_sdpa():
            with sdpa_kernel(pinned):
                return akref.paged_decode_torch(q, kc, vc, tables, nblk, context_lens=None if uniform else clens)
        impls["torch_gather_sdpa"] = gather_sdpa
    kg = vg = None
    if "torch_sdpa_contiguous" in wanted and uniform and pinned:
        kg, vg = akref.gather_kv(kc, tables, nblk), akref.gather_kv(vc, tables, nblk)
        qg = q.view(B, HKV, HQ // HKV, D)
        impls["torch_sdpa_contiguous"] = lambda: sdpa_pinned(*pinned)(qg, kg, vg)
    expect = akref.paged_decode_fp32(q[:1], kc, vc, tables[:1], clens[:1])
    nbytes = kv_bytes(lens)
    part = partition if partition is not None else ak.decode_partition(B, HKV, max_ctx)
    case = []
    for name, fn in impls.items():
        try:
            out = fn()
            err = (out[:1].float().reshape(expect.shape) - expect).abs().max().item()
            del out
            ms = median_ms(fn)
        except Exception as e:  # noqa: BLE001
            print(f"{section} {name} B={B} ctx={max_ctx}: {e!r}"[:300], flush=True)
            torch.cuda.empty_cache()
            continue
        r = dict(section=section, impl=name, batch=B, ctx=max_ctx, ctx_mean=round(sum(lens) / B, 1), heads=HQ,
                 kv_heads=HKV, head_dim=D, block_size=BS, ms=round(ms, 4),
                 gbs=round(nbytes / (ms * 1e-3) / 1e9, 1), max_abs_err=float(f"{err:.3g}"))
        if name == "paged_split":
            r["partition"] = part
            r["splits"] = -(-max_ctx // part)
        if extra:
            r.update(extra)
        case.append(r)
    base = next((r["ms"] for r in case if r["impl"] == "torch_gather_sdpa"), None)
    for r in case:
        r["speedup_vs_torch_gather"] = round(base / r["ms"], 3) if base else None
        rows.append(r)
        print(f"{section} B={B:3d} ctx={max_ctx:6d} {r['impl']:22s} {r['ms']:8.4f} ms {r['gbs']:8.1f} GB/s "
              f"err {r['max_abs_err']:.1e}{'  P=' + str(r['partition']) if 'partition' in r else ''}", flush=True)
    del kc, vc, kg, vg, q
    torch.cuda.empty_cache()


def section_decode(rows, quick, found):
    batches = (1, 16) if quick else (1, 4, 16, 64)
    ctxs = (1024, 4096) if quick else (1024, 2048, 4096, 8192, 16384, 32768)
    wanted = ("paged_split", "paged_nosplit", "torch_gather_sdpa", "torch_sdpa_contiguous")
    for B in batches:
        for c in ctxs:
            if kv_bytes([c] * B) <= 2.2e9:
                decode_case(rows, "decode", [c] * B, wanted, found)


def section_split_ablation(rows, quick, found):
    uniform = ((1, 8192),) if quick else ((1, 32768), (4, 8192), (16, 4096), (64, 4096), (64, 1024))
    for B, c in uniform:
        p = ak.CHUNK
        while p <= c:
            decode_case(rows, "split_ablation", [c] * B, ("paged_split",), found, partition=p)
            p *= 2
    # Mixed lengths: the partition is chosen from max_ctx alone, so check it here too.
    g = torch.Generator().manual_seed(1)
    ragged = [(8, 512, 8192)] if quick else [(4, 512, 32768), (16, 512, 32768), (64, 1, 4096)]
    for B, lo, hi in ragged:
        lens = torch.randint(lo, hi + 1, (B,), generator=g).tolist()
        p = ak.CHUNK
        while p < max(lens) * 2:
            decode_case(rows, "split_ablation_ragged", lens, ("paged_split",), found, partition=p,
                        extra=dict(ctx_lens=lens))
            p *= 2


def section_ragged(rows, quick, found):
    g = torch.Generator().manual_seed(0)
    B, hi = (8, 8192) if quick else (16, 32768)
    lens = torch.randint(512, hi + 1, (B,), generator=g).tolist()
    decode_case(rows, "ragged", lens, ("paged_split", "paged_nosplit", "torch_gather_sdpa"), found,
                extra=dict(ctx_lens=lens))


SECTIONS = {"prefill": section_prefill, "decode": section_decode, "split_ablation": section_split_ablation,
            "ragged": section_ragged}


def device_meta():
    p = torch.cuda.get_device_properties(0)
    return dict(gpu=p.name, arch=getattr(p, "gcnArchName", ""), cu_count=p.multi_processor_count,
                memory_gb=round(p.total_memory / 2**30, 1), torch=torch.__version__,
                hip=getattr(torch.version, "hip", None), python=platform.python_version(),
                date=dt.datetime.now(dt.timezone.utc).strftime("%Y-%m-%d %H:%M UTC"))


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--out", default="results/mi355x.json")
    ap.add_argument("--quick", action="store_true", help="small sizes (a smoke run)")
    ap.add_argument("--only", nargs="*", default=list(SECTIONS), choices=list(SECTIONS))
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        raise SystemExit("benchsuite needs a GPU")
    torch.manual_seed(0)
    ak.load_extension()
    meta = device_meta()
    meta["sdpa_backends"] = probe_sdpa_backends()
    meta["roofs"] = roofs()
    meta["timing"] = "hipEvent median of 3..50 calls, 512 MiB cache flush before each call"
    print(json.dumps(meta, indent=1), flush=True)
    rows = []
    out = Path(args.out)
    for name in args.only:
        t = time.perf_counter()
        try:
            SECTIONS[name](rows, args.quick, meta["sdpa_backends"])
        except Exception as e:  # noqa: BLE001  keep the other sections
            print(f"section {name} failed: {e!r}", flush=True)
            meta.setdefault("failed_sections", {})[name] = repr(e)[:500]
        meta.setdefault("section_seconds", {})[name] = round(time.perf_counter() - t, 1)
        out.parent.mkdir(parents=True, exist_ok=True)
        out.write_text(json.dumps(dict(meta=meta, results=rows), indent=1))
    print("wrote", out, flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
