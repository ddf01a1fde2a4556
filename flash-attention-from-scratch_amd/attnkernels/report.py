"""Markdown report of a ``benchsuite`` JSON file (the counterpart of the
reference's bench/report.py:36-98): device and ceilings, then one table per
section, with this build's kernels as fractions of the MI355X peaks.

    python -m attnkernels.report results/mi355x.json > results/mi355x.md
"""
from __future__ import annotations

import json
import sys
from collections import defaultdict

PEAK_TFLOPS = 2500.0  # dense fp16 MFMA
PEAK_GBS = 8000.0     # HBM3E


def _table(header, rows):
    out = ["| " + " | ".join(header) + " |", "|" + "---|" * len(header)]
    out += ["| " + " | ".join(str(c) for c in r) + " |" for r in rows]
    return "\n".join(out)


def prefill_tables(rows):
    impls = []
    for r in rows:
        if r["impl"] not in impls:
            impls.append(r["impl"])
    parts = []
    for d in (64, 128):
        for causal in (False, True):
            sel = [r for r in rows if r["head_dim"] == d and r["causal"] == causal]
            if not sel:
                continue
            by_n = defaultdict(dict)
            for r in sel:
                by_n[(r["batch"], r["seq"])][r["impl"]] = r
            body = []
            for (b, n), rs in sorted(by_n.items(), key=lambda kv: kv[0][1]):
                cells = [f"{b}x{n}"]
                for i in impls:
                    r = rs.get(i)
                    cells.append(f"{r['tflops']:.1f}" if r else "-")
                ours = rs.get("flash_attention")
                cells.append(f"{100 * ours['tflops'] / PEAK_TFLOPS:.1f}%" if ours else "-")
                cells.append(f"{ours['speedup_vs_sdpa']}x" if ours and ours.get("speedup_vs_sdpa") else "-")
                cells.append(f"{ours['max_abs_err']:.1e}" if ours else "-")
                body.append(cells)
            parts.append(f"**D={d}, {'causal' if causal else 'non-causal'}** (TFLOP/s; H=16)\n\n" +
                         _table(["B x N"] + impls + ["flash % peak", "vs SDPA", "max err"], body))
    return "\n\n".join(parts)


def _impls(rows):
    out = []
    for r in rows:
        if r["impl"] not in out:
            out.append(r["impl"])
    return out


def prefill_memory_tables(rows):
    """Extra device memory one call allocates at its peak (output included), per
    head dim, non-causal: the flash kernels hold O(N) state, the naive
    formulation O(N^2)."""
    parts = []
    for d in sorted({r["head_dim"] for r in rows}):
        sel = [r for r in rows if r["head_dim"] == d and not r["causal"] and "peak_mem_mb" in r]
        if not sel:
            continue
        impls, by = _impls(sel), defaultdict(dict)
        for r in sel:
            by[(r["batch"], r["seq"])][r["impl"]] = r["peak_mem_mb"]
        body = [[f"{b}x{n}"] + [f"{by[(b, n)][i]:.0f}" if i in by[(b, n)] else "-" for i in impls]
                for (b, n) in sorted(by, key=lambda k: k[1])]
        parts.append(f"**D={d}, non-causal** (MB above what is live; output included)\n\n" +
                     _table(["B x N"] + impls, body))
    return "\n\n".join(parts)


def worst_error_table(rows):
    """Worst max-abs error against fp32 of each implementation, over every shape
    of the prefill sections and of the decode sections."""
    body = []
    for title, secs in (("prefill", ("prefill",)),
                        ("decode", ("decode", "decode_heads", "ragged", "split_ablation", "split_ablation_ragged"))):
        sel = [r for r in rows if r["section"] in secs and "max_abs_err" in r]
        for i in _impls(sel):
            errs = [r["max_abs_err"] for r in sel if r["impl"] == i]
            body.append([title, i, len(errs), f"{max(errs):.2e}"])
    return _table(["path", "impl", "shapes", "worst max abs error"], body) if body else ""


def head_group_error_table(rows):
    """Max-abs error against fp32 per head group: the grouped-query kernels
    (fp16 P) and the one-head kernel (fp32 P) on the same queries and K/V."""
    sel = sorted((r for r in rows if r["section"] == "decode_heads" and "max_abs_err" in r),
                 key=lambda r: (r["head_dim"], r.get("group", 1)))
    body = [[r["head_dim"], r.get("group", 1), f"{r['batch']} x {r['ctx']}", f"{r['max_abs_err']:.2e}",
             f"{r['max_abs_err_one_head_path']:.2e}" if "max_abs_err_one_head_path" in r else "(the same kernel)"]
            for r in sel]
    return _table(["D", "G", "B x ctx", "max abs error (G-head kernel)", "one-head kernel, same data"],
                  body) if body else ""


def decode_time_table(rows, section="decode"):
    sel = [r for r in rows if r["section"] == section]
    if not sel:
        return ""
    impls, by = _impls(sel), defaultdict(dict)
    for r in sel:
        by[(r["batch"], r["ctx"])][r["impl"]] = r["ms"]
    body = [[b, c] + [f"{by[(b, c)][i]:.4f}" if i in by[(b, c)] else "-" for i in impls] for (b, c) in sorted(by)]
    return _table(["B", "max ctx"] + [f"{i} ms" for i in impls], body)


def head_group_table(rows):
    sel = [r for r in rows if r["section"] == "decode_heads"]
    if not sel:
        return ""
    body = [[r["head_dim"], r["group"], r["heads"], r["kv_heads"], r["batch"], r["ctx"], r.get("partition", "-"),
             f"{r['ms']:.4f}", f"{r['gbs']:.0f}", f"{100 * r['gbs'] / PEAK_GBS:.1f}%"]
            for r in sorted(sel, key=lambda r: (r["head_dim"], r["group"]))]
    return _table(["D", "G", "Hq", "Hkv", "B", "ctx", "P", "ms", "GB/s", "% HBM"], body)


def decode_table(rows, section):
    sel = [r for r in rows if r["section"] == section]
    if not sel:
        return ""
    impls = []
    for r in sel:
        if r["impl"] not in impls:
            impls.append(r["impl"])
    by_case = defaultdict(dict)
    for r in sel:
        by_case[(r["batch"], r["ctx"])][r["impl"]] = r
    body = []
    for (b, c), rs in sorted(by_case.items()):
        cells = [b, c]
        for i in impls:
            r = rs.get(i)
            cells.append(f"{r['gbs']:.0f}" if r else "-")
        ours = rs.get("paged_split")
        cells.append(f"{100 * ours['gbs'] / PEAK_GBS:.1f}%" if ours else "-")
        cells.append(ours.get("partition", "-") if ours else "-")
        cells.append(f"{ours['speedup_vs_torch_gather']}x" if ours and ours.get("speedup_vs_torch_gather") else "-")
        body.append(cells)
    return _table(["B", "max ctx"] + [f"{i} GB/s" for i in impls] + ["split % HBM", "P", "vs gather+SDPA"], body)


def ablation_table(rows, section="split_ablation"):
    sel = [r for r in rows if r["section"] == section]
    if not sel:
        return ""
    by_case = defaultdict(list)
    for r in sel:
        by_case[(r.get("heads", 32), r.get("kv_heads", 8), r["batch"], r["ctx"])].append(r)
    body = []
    for (hq, hkv, b, c), rs in sorted(by_case.items()):
        best = max(rs, key=lambda r: r["gbs"])
        curve = ", ".join(f"{r['partition']}:{r['gbs']:.0f}" for r in sorted(rs, key=lambda r: r["partition"]))
        body.append([f"{hq}/{hkv}", b, c, best["partition"], f"{best['gbs']:.0f}", curve])
    return _table(["Hq/Hkv", "B", "ctx", "best P", "best GB/s", "P:GB/s"], body)


def activity_table(rows):
    """TFLOP/s of each workload (columns) per input pattern (rows), and each
    prefill workload's rate as a share of the GEMM's under the same inputs."""
    sel = [r for r in rows if r["section"] == "input_activity"]
    if not sel:
        return ""
    works, pats, by = [], [], {}
    for r in sel:
        if r["workload"] not in works:
            works.append(r["workload"])
        if r["data"] not in pats:
            pats.append(r["data"])
        by[(r["data"], r["workload"])] = r["tflops"]
    gemm = next((w for w in works if "GEMM" in w), None)
    pre = [w for w in works if w != gemm]
    body = []
    for p in pats:
        cells = [p]
        for w in works:
            t = by.get((p, w))
            cells.append(f"{t:.0f} ({100 * t / PEAK_TFLOPS:.0f}%)" if t is not None else "-")
        g = by.get((p, gemm)) if gemm else None
        for w in pre:
            t = by.get((p, w))
            cells.append(f"{100 * t / g:.0f}%" if t is not None and g else "-")
        body.append(cells)
    return _table(["inputs"] + [f"{w} TFLOP/s" for w in works] + [f"{w} / GEMM" for w in pre], body)


def render(data):
    meta, rows = data["meta"], data["results"]
    lines = [f"# Attention kernels on {meta.get('gpu')} ({meta.get('arch')}, {meta.get('cu_count')} CUs)", ""]
    lines.append(f"torch {meta.get('torch')}, HIP {meta.get('hip')}, {meta.get('date')}.  "
                 f"Timing: {meta.get('timing')}.")
    if meta.get("sources_sha256"):
        lines.append(f"Kernel sources digest {meta['sources_sha256'][:12]}.")
    roofs = meta.get("roofs", {})
    lines += ["", f"Ceilings measured here: device copy {roofs.get('copy_gbs')} GB/s "
                  f"({100 * roofs.get('copy_gbs', 0) / PEAK_GBS:.0f}% of 8 TB/s), fp16 GEMM 8192^3 "
                  f"{roofs.get('fp16_gemm_tflops')} TFLOP/s ({100 * roofs.get('fp16_gemm_tflops', 0) / PEAK_TFLOPS:.0f}% "
                  f"of 2.5 PFLOP/s).", ""]
    lines.append("SDPA backends: " + ", ".join(f"{k}: {v}" for k, v in meta.get("sdpa_backends", {}).items()))
    pre = [r for r in rows if r["section"] == "prefill"]
    if pre:
        lines += ["", "## Prefill", "", prefill_tables(pre)]
        t = prefill_memory_tables(pre)
        if t:
            lines += ["", "### Prefill peak extra memory", "", t]
    for section, title in (("decode", "Paged decode (Hq=32, Hkv=8, D=128, page 16)"),
                           ("ragged", "Ragged batch")):
        t = decode_table(rows, section)
        if t:
            lines += ["", f"## {title}", "", t]
        t = decode_time_table(rows, section)
        if t:
            lines += ["", f"### {title}: time per call", "", t]
    t = head_group_table(rows)
    if t:
        lines += ["", "## Paged decode by head group (query heads per kv head)", "", t]
    t = ablation_table(rows)
    if t:
        lines += ["", "## Split-K partition ablation", "", t]
    t = ablation_table(rows, "split_ablation_ragged")
    if t:
        lines += ["", "## Split-K partition ablation, mixed context lengths (ctx = max)", "", t]
    t = activity_table(rows)
    if t:
        lines += ["", "## Rate against input bit activity (same kernels, same shapes)", "", t]
    t = worst_error_table(rows)
    if t:
        lines += ["", "## Worst error against fp32", "", t]
    t = head_group_error_table(rows)
    if t:
        lines += ["", "## Decode error by head group (fp16 P in the grouped-query kernels, fp32 P in the one-head "
                  "kernel; the same queries and K/V)", "", t]
    for key in ("failed_sections", "failed_cases"):
        if meta.get(key):
            lines += ["", f"{key.replace('_', ' ').capitalize()}: " + json.dumps(meta[key])]
    return "\n".join(lines) + "\n"


def main(argv=None):
    argv = sys.argv[1:] if argv is None else argv
    if len(argv) != 1:
        raise SystemExit("usage: python -m attnkernels.report results.json")
    with open(argv[0]) as f:
        sys.stdout.write(render(json.load(f)))
    return 0


if __name__ == "__main__":
    sys.exit(main())
