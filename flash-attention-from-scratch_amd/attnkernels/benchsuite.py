"""Comparison suite on one MI355X: this build's kernels against PyTorch's own
attention, and the split-K partition sweeps behind ``decode_partition``.
Writes a JSON file that ``attnkernels.report`` renders as markdown.

    python -m attnkernels.benchsuite --out results/mi355x.json [--quick] [--sections ...]
    python -m attnkernels.report results/mi355x.json > results/mi355x.md

Structure.  A section is a list of case builders.  A builder allocates one
case's inputs on the device and returns a ``Case``: the row's shape columns,
the work of one call (FLOP, or K/V bytes), the implementations to compare
(zero-argument callables), and an error function against an fp32 reference.
One runner, ``run_case``, times every implementation with the flushed
protocol of ``attnkernels.timing`` (512 MiB overwritten before each call,
median of 5-40 calls within a quarter second), measures its extra peak
memory, and emits one row per implementation.  The JSON file is rewritten
after every case, so an interrupted run keeps what it measured.

Sections (the row schema ``attnkernels.report`` reads):
  prefill                flash_attention vs SDPA (flash, memory-efficient, both),
                         at a constant token count per shape, D in {64, 128},
                         causal and not: the shapes of the reference's T4
                         tables (its bench/bench.py prefill sweep), so the two
                         can be read side by side
  decode                 paged_decode (default partition, and one split) vs
                         gathering the pages then SDPA, and SDPA on a cache
                         that is already contiguous: Llama-3-8B's attention
                         layer (32 query heads, 8 kv heads, D=128, 16-token pages)
  decode_heads           paged_decode over head-group sizes 1-8 and D 64/128
  split_ablation         every power-of-two partition from 256 tokens to one
                         split, uniform batches
  split_ablation_ragged  the same over batches of mixed context lengths
  ragged                 one mixed-length batch, all decode implementations
  input_activity         the headline prefill shapes and an 8192^3 fp16 GEMM on
                         random, random-sign, all-ones and all-zero inputs

SDPA is pinned to its fused backends; its math backend (batched products on
transposed views, which have faulted GPUs on this pool) never runs.
"""
from __future__ import annotations

import argparse
import datetime as dt
import json
import os
import platform
import sys
import time
from dataclasses import dataclass, field
from pathlib import Path
from typing import Callable, Dict, Iterator, Optional

import torch
import torch.nn.functional as F

import attnkernels as ak
from attnkernels import reference as akref
from attnkernels import timing

try:
    from torch.nn.attention import SDPBackend, sdpa_kernel
except ImportError:  # older torch
    SDPBackend = sdpa_kernel = None

PEAK = {"TFLOP/s": 2500.0, "GB/s": 8000.0}   # MI355X: dense fp16 MFMA, HBM3E


@dataclass
class Case:
    section: str
    fields: dict                                   # the row's shape columns
    work: float                                    # FLOP or bytes of one call
    unit: str                                      # "TFLOP/s" or "GB/s"
    impls: Dict[str, Callable[[], torch.Tensor]]
    error: Callable[[torch.Tensor], float]         # output -> max abs error vs fp32
    baseline: Optional[str] = None                 # implementation the speed-ups divide by
    speedup_key: Optional[str] = None
    per_impl: Dict[str, dict] = field(default_factory=dict)  # extra columns of one implementation


# ---------------------------------------------------------------- SDPA -----

def sdpa_on(backends):
    """SDPA restricted to ``backends`` (never the math path)."""
    def run(q, k, v, causal=False):
        with sdpa_kernel(list(backends)):
            return F.scaled_dot_product_attention(q, k, v, is_causal=causal)
    return run


def available_sdpa():
    """{backend name: "ok" | reason} for the fused SDPA backends on this GPU (fp16, D=128)."""
    status = {}
    if sdpa_kernel is None:
        return status
    x = torch.randn(1, 2, 128, 128, device="cuda", dtype=torch.float16)
    for name in ("FLASH_ATTENTION", "EFFICIENT_ATTENTION", "CUDNN_ATTENTION"):
        be = getattr(SDPBackend, name, None)
        if be is None:
            continue
        try:
            sdpa_on([be])(x, x, x, True)
            torch.cuda.synchronize()
            status[name] = "ok"
        except Exception as e:  # noqa: BLE001
            status[name] = "unavailable: " + str(e).splitlines()[0][:160]
    status["MATH"] = "not run (batched products on transposed views are avoided on this GPU pool)"
    return status


def usable(status):
    return [getattr(SDPBackend, n) for n, s in status.items() if s == "ok"]


# ------------------------------------------------------------- ceilings ----

def ceilings():
    """What this GPU sustains in practice: a 2 GiB device copy (GB/s of reads +
    writes) and an 8192^3 fp16 GEMM (hipBLASLt through torch.mm)."""
    n = 2 << 30
    src = torch.ones(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    copy_ms = min(timing.flushed_samples(lambda: dst.copy_(src), min_calls=5, max_calls=10))
    del src, dst
    a, b = (torch.randn(8192, 8192, device="cuda", dtype=torch.float16) for _ in range(2))
    gemm_ms = min(timing.flushed_samples(lambda: torch.mm(a, b), min_calls=5, max_calls=20))
    del a, b
    torch.cuda.empty_cache()
    return dict(copy_gbs=round(2 * n / (copy_ms * 1e-3) / 1e9, 1),
                fp16_gemm_tflops=round(2 * 8192 ** 3 / (gemm_ms * 1e-3) / 1e12, 1))


# ---------------------------------------------------------------- cases ----

def prefill_builders(quick, status, max_kv_gb=None) -> Iterator[Callable[[], Case]]:
    heads = 16
    tokens = 4096 if quick else 16384          # batch x sequence length per shape
    seqs = (512, 1024) if quick else (512, 1024, 2048, 4096, 8192)
    fused = usable(status)
    for d in (64, 128):
        for causal in (False, True):
            for n in seqs:
                def build(d=d, causal=causal, n=n):
                    b = max(1, tokens // n)
                    g = torch.Generator(device="cuda").manual_seed(1000 * d + n)
                    q, k, v = (torch.randn(b, heads, n, d, generator=g, device="cuda", dtype=torch.float16)
                               for _ in range(3))
                    impls = {"flash_attention": lambda: ak.flash_attention(q, k, v, causal=causal)}
                    if fused:
                        impls["sdpa_fused"] = lambda: sdpa_on(fused)(q, k, v, causal)
                    for be in fused:
                        impls["sdpa_" + be.name.split("_")[0].lower()] = lambda be=be: sdpa_on([be])(q, k, v, causal)

                    def error(out):
                        # the first and the last (batch, head) slice against fp32 attention
                        worst = 0.0
                        for bi, hi in ((0, 0), (b - 1, heads - 1)):
                            ref = akref.attention_fp32(q[bi:bi + 1, hi:hi + 1], k[bi:bi + 1, hi:hi + 1],
                                                       v[bi:bi + 1, hi:hi + 1], causal)
                            worst = max(worst, (out[bi:bi + 1, hi:hi + 1].float() - ref).abs().max().item())
                        return worst
                    return Case("prefill", dict(batch=b, heads=heads, seq=n, head_dim=d, causal=causal),
                                4.0 * b * heads * n * n * d * (0.5 if causal else 1.0), "TFLOP/s", impls, error,
                                baseline="sdpa_fused", speedup_key="speedup_vs_sdpa")
                yield build


# Llama-3-8B's attention layer: 32 query heads over 8 kv heads, head_dim 128;
# 16-token pages.
LAYER = dict(hq=32, hkv=8, d=128, bs=16)


def decode_case(section, lens, impl_names, status, partition=None, hq=LAYER["hq"], hkv=LAYER["hkv"], d=LAYER["d"],
                seed=0, extra=None):
    """A paged cache holding ``lens`` tokens per sequence (pages scattered by a
    seeded permutation), the query of each sequence, and the implementations
    in impl_names."""
    bs, B, max_ctx = LAYER["bs"], len(lens), max(lens)
    gen = torch.Generator().manual_seed(seed)
    kc, vc, tables, clens = akref.make_paged_cache(lens, hkv, d, block_size=bs, generator=gen)
    q = torch.randn(B, hq, d, device="cuda", dtype=torch.float16, generator=torch.Generator(device="cuda")
                    .manual_seed(seed + 1))
    nblk = -(-max_ctx // bs)
    fused = usable(status)
    part = ak.decode_partition(B, hkv, max_ctx) if partition is None else partition
    impls, per_impl = {}, {}
    if "paged_split" in impl_names:
        impls["paged_split"] = lambda: ak.paged_decode(q, kc, vc, tables, clens, max_ctx, partition_size=part)
        per_impl["paged_split"] = dict(partition=part, splits=-(-max_ctx // part))
    if "paged_nosplit" in impl_names:
        one = -(-max_ctx // ak.CHUNK) * ak.CHUNK
        impls["paged_nosplit"] = lambda: ak.paged_decode(q, kc, vc, tables, clens, max_ctx, partition_size=one)
    uniform = len(set(lens)) == 1
    if "torch_gather_sdpa" in impl_names and fused:
        def gather_then_sdpa():
            with sdpa_kernel(fused):
                return akref.paged_decode_torch(q, kc, vc, tables, nblk, context_lens=None if uniform else clens)
        impls["torch_gather_sdpa"] = gather_then_sdpa
    if "torch_sdpa_contiguous" in impl_names and uniform and fused:
        kg, vg = akref.gather_kv(kc, tables, nblk), akref.gather_kv(vc, tables, nblk)
        qg = q.view(B, hkv, hq // hkv, d)
        impls["torch_sdpa_contiguous"] = lambda: sdpa_on(fused)(qg, kg, vg)
    check = [0, B - 1] if B > 1 else [0]
    refs = {b: akref.paged_decode_fp32(q[b:b + 1], kc, vc, tables[b:b + 1], clens[b:b + 1]) for b in check}

    def error(out):
        out = out.reshape(B, hq, d)
        return max((out[b:b + 1].float() - refs[b].reshape(1, hq, d)).abs().max().item() for b in check)
    if "paged_split" in impl_names and hq > hkv:
        # The grouped-query kernels round P to fp16; the one-head kernel keeps
        # it in fp32.  The same queries through the one-head kernel, on caches
        # whose kv heads are repeated once per query head, give the error of
        # the fp32-P path on identical data (checked once, not timed).
        g = hq // hkv
        kr, vr = (c.repeat_interleave(g, dim=1) for c in (kc, vc))
        out1 = ak.paged_decode(q, kr, vr, tables, clens, max_ctx, partition_size=part)
        per_impl["paged_split"]["max_abs_err_one_head_path"] = float(f"{error(out1):.3g}")
        del kr, vr, out1
    fields = dict(batch=B, ctx=max_ctx, ctx_mean=round(sum(lens) / B, 1), heads=hq, kv_heads=hkv, head_dim=d,
                  block_size=bs, **(extra or {}))
    return Case(section, fields, float(sum(lens)) * hkv * d * 2 * 2, "GB/s", impls, error,
                baseline="torch_gather_sdpa", speedup_key="speedup_vs_torch_gather", per_impl=per_impl)


def kv_gb(lens, hkv=LAYER["hkv"], d=LAYER["d"]):
    return sum(lens) * hkv * d * 4 / 1e9


def decode_builders(quick, status, max_kv_gb):
    grid = [(B, c) for B in ((1, 16) if quick else (1, 4, 16, 64, 256))
            for c in ((1024, 4096) if quick else (1024, 2048, 4096, 8192, 16384, 32768))]
    names = ("paged_split", "paged_nosplit", "torch_gather_sdpa", "torch_sdpa_contiguous")
    for B, c in grid:
        if kv_gb([c] * B) <= max_kv_gb:
            yield lambda B=B, c=c: decode_case("decode", [c] * B, names, status)


def decode_head_builders(quick, status, max_kv_gb):
    B, c = (4, 4096) if quick else (16, 8192)
    for d in (64, 128):
        for g in (1, 2, 4, 8):
            hkv = 8
            yield lambda d=d, g=g, hkv=hkv: decode_case("decode_heads", [c] * B, ("paged_split",), status, hq=g * hkv,
                                                        hkv=hkv, d=d, extra=dict(group=g))


def partitions_up_to(max_ctx):
    """256, 512, ... up to the first partition that leaves one split."""
    out, p = [], ak.CHUNK
    while True:
        out.append(p)
        if p >= max_ctx:
            return out
        p *= 2


def mixed_lengths(batch, lo, hi, seed):
    return torch.randint(lo, hi + 1, (batch,), generator=torch.Generator().manual_seed(seed)).tolist()


# Head shapes of the split-K ablation: (query heads, kv heads).  The layer above
# (4 query heads per kv head), one query head per kv head (the BASELINE decode
# configs) and 8 per kv head: each runs a different decode kernel.
ABLATION_HEADS = ((32, 8), (32, 32), (64, 8))


def ablation_builders(quick, status, max_kv_gb):
    # the last of each head shape: B * Hkv >= 2 per CU with more than 8192 tokens
    uniform = {(32, 8): ((1, 4096), (1, 16384), (1, 32768), (2, 4096), (4, 8192), (16, 4096), (16, 8192), (64, 1024),
                         (64, 4096), (64, 16384)),
               (32, 32): ((8, 32768), (16, 8192), (64, 4096), (16, 16384)),
               (64, 8): ((1, 32768), (8, 8192), (16, 8192), (64, 4096), (64, 16384))}
    mixed = {(32, 8): ((4, 512, 32768, 1), (16, 512, 32768, 2), (64, 1, 4096, 3), (64, 512, 32768, 9)),
             (32, 32): ((64, 1, 4096, 4),),
             (64, 8): ((16, 512, 32768, 5),)}
    # one long sequence among many short ones, with B * Hkv >= 2 per CU
    skewed = {(32, 8): ((64, 32768, 2048, 6), (64, 16384, 2048, 10)), (32, 32): ((32, 32768, 2048, 7),),
              (64, 8): ((64, 32768, 2048, 8), (64, 16384, 2048, 11))}
    if quick:
        uniform, mixed, skewed = {(32, 8): ((1, 8192),)}, {(32, 8): ((8, 512, 8192, 3),)}, {}
    for (hq, hkv), shapes in uniform.items():
        for B, c in shapes:
            if kv_gb([c] * B, hkv) > max_kv_gb:
                continue
            for p in partitions_up_to(c):
                yield lambda B=B, c=c, p=p, hq=hq, hkv=hkv: decode_case("split_ablation", [c] * B, ("paged_split",),
                                                                        status, partition=p, hq=hq, hkv=hkv)
    for (hq, hkv), shapes in mixed.items():
        for B, lo, hi, seed in shapes:
            lens = mixed_lengths(B, lo, hi, seed)
            if kv_gb(lens, hkv) > max_kv_gb:
                continue
            for p in partitions_up_to(max(lens)):
                yield lambda lens=lens, p=p, hq=hq, hkv=hkv: decode_case(
                    "split_ablation_ragged", lens, ("paged_split",), status, partition=p, hq=hq, hkv=hkv,
                    extra=dict(ctx_lens=lens))
    for (hq, hkv), shapes in skewed.items():
        for B, long, short_hi, seed in shapes:
            lens = [long] + mixed_lengths(B - 1, 1, short_hi, seed)
            for p in partitions_up_to(long):
                yield lambda lens=lens, p=p, hq=hq, hkv=hkv: decode_case(
                    "split_ablation_ragged", lens, ("paged_split",), status, partition=p, hq=hq, hkv=hkv,
                    extra=dict(ctx_lens=lens))


def ragged_builders(quick, status, max_kv_gb):
    # The reference's ragged batch (16 sequences of 512-32768 tokens, torch's CPU
    # generator seeded 0: mean 14722, max 31683), regenerated identically so that
    # its T4 row and this one describe the same batch.
    B, hi = (8, 8192) if quick else (16, 32768)
    lens = mixed_lengths(B, 512, hi, 0)
    names = ("paged_split", "paged_nosplit", "torch_gather_sdpa")
    yield lambda: decode_case("ragged", lens, names, status, extra=dict(ctx_lens=lens))


# Input patterns ordered by how many bits they switch in the matrix core:
# normal random values, random signs of one magnitude, all ones, all zeros.
ACTIVITY = ("randn", "signs", "ones", "zeros")


def activity_tensor(pattern, shape, gen):
    x = torch.randn(*shape, generator=gen, device="cuda", dtype=torch.float16)
    if pattern == "randn":
        return x
    if pattern == "signs":
        return torch.where(x > 0, 1.0, -1.0).to(torch.float16)
    return torch.ones_like(x) if pattern == "ones" else torch.zeros_like(x)


def activity_builders(quick, status, max_kv_gb=None):
    """The prefill kernel and hipBLASLt's fp16 GEMM on the same shapes with
    inputs of decreasing bit activity.  The instruction stream and control flow
    hardly depend on the values (every tile is computed, and for all four
    patterns the running maximum moves almost only on the first tile), so a
    rate that rises as the inputs switch fewer bits shows a power-limited
    clock, not an instruction-bound schedule."""
    shapes = ([(1, 8, 2048, 128, True), (2, 8, 1024, 64, False)] if quick else
              [(2, 32, 8192, 128, True), (2, 32, 8192, 128, False), (4, 16, 2048, 64, False)])
    gemm_n = 2048 if quick else 8192
    for pattern in ACTIVITY:
        for (b, h, n, d, causal) in shapes:
            def build(pattern=pattern, b=b, h=h, n=n, d=d, causal=causal):
                g = torch.Generator(device="cuda").manual_seed(7)
                q, k, v = (activity_tensor(pattern, (b, h, n, d), g) for _ in range(3))

                def error(out):
                    ref = akref.attention_fp32(q[:1, :1], k[:1, :1], v[:1, :1], causal)
                    return (out[:1, :1].float() - ref).abs().max().item()
                name = f"prefill {'causal ' if causal else ''}B={b} H={h} N={n} D={d}"
                return Case("input_activity", dict(workload=name, data=pattern, batch=b, heads=h, seq=n, head_dim=d,
                                                   causal=causal),
                            4.0 * b * h * n * n * d * (0.5 if causal else 1.0), "TFLOP/s",
                            {"flash_attention": lambda: ak.flash_attention(q, k, v, causal=causal)}, error)
            yield build

        def build_gemm(pattern=pattern, n=gemm_n):
            g = torch.Generator(device="cuda").manual_seed(8)
            a, b = (activity_tensor(pattern, (n, n), g) for _ in range(2))

            def error(out):
                ref = a[:64].float() @ b[:, :64].float()
                return (out[:64, :64].float() - ref).abs().max().item()
            return Case("input_activity", dict(workload=f"fp16 GEMM {n}^3", data=pattern), 2.0 * n ** 3, "TFLOP/s",
                        {"hipblaslt_gemm": lambda: torch.mm(a, b)}, error)
        yield build_gemm


SECTIONS = {"prefill": prefill_builders, "decode": decode_builders, "decode_heads": decode_head_builders,
            "split_ablation": ablation_builders, "ragged": ragged_builders, "input_activity": activity_builders}


# --------------------------------------------------------------- runner ----

def run_case(case: Case):
    """One row per implementation: flushed median time, rate, fraction of the
    MI355X peak, extra peak memory, max abs error; speed-ups against the
    case's baseline when it ran."""
    rate_key = "tflops" if case.unit == "TFLOP/s" else "gbs"
    scale = 1e12 if case.unit == "TFLOP/s" else 1e9
    rows = []
    for name, fn in case.impls.items():
        try:
            out = fn()
            err = case.error(out)
            del out
            ms = sorted(timing.flushed_samples(fn))
            med = ms[len(ms) // 2] if len(ms) % 2 else 0.5 * (ms[len(ms) // 2 - 1] + ms[len(ms) // 2])
            mem = timing.extra_peak_bytes(fn) / 2 ** 20
        except Exception as e:  # noqa: BLE001  an implementation that rejects the shape
            print(f"  {case.section} {name} {case.fields}: {e!r}"[:300], flush=True)
            torch.cuda.empty_cache()
            continue
        rate = case.work / (med * 1e-3) / scale
        rows.append(dict(section=case.section, impl=name, **case.fields, ms=round(med, 4), calls=len(ms),
                         **{rate_key: round(rate, 2 if case.unit == "TFLOP/s" else 1)},
                         frac_of_peak=round(rate / PEAK[case.unit], 4), peak_mem_mb=round(mem, 1),
                         max_abs_err=float(f"{err:.3g}"), **case.per_impl.get(name, {})))
    base = next((r["ms"] for r in rows if r["impl"] == case.baseline), None)
    if case.speedup_key:
        for r in rows:
            r[case.speedup_key] = round(base / r["ms"], 3) if base else None
    return rows


def device_meta():
    from attnkernels import build as akbuild

    p = torch.cuda.get_device_properties(0)
    return dict(gpu=p.name, arch=getattr(p, "gcnArchName", ""), cu_count=p.multi_processor_count,
                memory_gb=round(p.total_memory / 2 ** 30, 1), torch=torch.__version__,
                hip=getattr(torch.version, "hip", None), python=platform.python_version(),
                host_cpus=os.cpu_count(), date=dt.datetime.now(dt.timezone.utc).strftime("%Y-%m-%d %H:%M UTC"),
                # the kernel sources measured (the same digest bench.py and profiles/ cite)
                sources_sha256=akbuild.sources_digest())


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--out", default="results/mi355x.json")
    ap.add_argument("--quick", action="store_true", help="small sizes (a smoke run)")
    ap.add_argument("--sections", nargs="*", default=list(SECTIONS), choices=list(SECTIONS))
    ap.add_argument("--max-kv-gb", type=float, default=4.5,
                    help="skip decode cases whose K/V exceed this (the BASELINE decode configs hold up to 4.3 GB)")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        raise SystemExit("benchsuite needs a GPU")
    ak.load_extension()
    meta = device_meta()
    meta["sdpa_backends"] = available_sdpa()
    meta["roofs"] = ceilings()
    meta["timing"] = (f"hipEvent median of 5-40 calls (0.25 s budget), {timing.FLUSH_BYTES >> 20} MiB overwritten "
                      "before each call")
    print(json.dumps(meta), flush=True)
    out, rows = Path(args.out), []
    out.parent.mkdir(parents=True, exist_ok=True)
    for name in args.sections:
        t0, n = time.perf_counter(), 0
        for build in SECTIONS[name](args.quick, meta["sdpa_backends"], args.max_kv_gb):
            try:
                case = build()
                new = run_case(case)
                del case
            except Exception as e:  # noqa: BLE001  keep the other cases
                print(f"{name}: case failed: {e!r}"[:300], flush=True)
                meta.setdefault("failed_cases", []).append(f"{name}: {e!r}"[:300])
                new = []
            torch.cuda.empty_cache()
            for r in new:
                rate = r.get("tflops", r.get("gbs"))
                print(f"{name:22s} {r['impl']:22s} {json.dumps({k: r[k] for k in r if k in ('batch', 'seq', 'ctx', 'head_dim', 'causal', 'partition', 'group')})} "
                      f"{r['ms']:.4f} ms {rate} err {r['max_abs_err']:.1e}", flush=True)
            rows += new
            n += 1
            tmp = out.with_suffix(".tmp")
            tmp.write_text(json.dumps(dict(meta=meta, results=rows), indent=1))
            os.replace(tmp, out)
        meta.setdefault("section_seconds", {})[name] = round(time.perf_counter() - t0, 1)
        meta.setdefault("section_cases", {})[name] = n
    out.write_text(json.dumps(dict(meta=meta, results=rows), indent=1))
    print("wrote", out, flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
