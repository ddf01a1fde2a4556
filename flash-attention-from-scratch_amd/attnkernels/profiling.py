"""rocprofv3 summaries of bench.py workloads (the files under ``profiles/``).

Runs on the host, after rocprofv3 ran ``python bench.py --only W`` on the GPU
and wrote its CSV files to RAW (by convention ``gpurun_out/praw/W``):

    python flash-attention-from-scratch_amd/attnkernels/profiling.py trace W RAW
        RAW/trace_kernel_trace.csv   rocprofv3 --kernel-trace ... -o trace
        RAW/bench_trace.json         bench.py's stdout in that run
        RAW/fetch_counter_collection.csv, RAW/write_counter_collection.csv
                                     rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE ... --calib-copy
      -> profiles/<kernel>_<W>.md and the W entry of profiles/traffic.json

    python flash-attention-from-scratch_amd/attnkernels/profiling.py counters W RAW ctr1 ctr2 ...
        RAW/<ctr>_counter_collection.csv + RAW/bench_<ctr>.json per pass
      -> profiles/<kernel>_<W>_counters.md

Only the dispatches of bench.py's K timed steps are summarised: bench.py
reports ``calls_before_timed`` (accuracy call, settle and warmup calls), and
every call launches each of this library's kernels once, so the timed
dispatches of kernel X are its dispatches number calls_before_timed ..
calls_before_timed + K - 1; K steps with an event at each boundary follow
(bench.py's per-step median), then the K flushed steps.  The trace-side step
time (start of one timed step's first kernel to the next one's) is the quantity
bench.py's events around the timed steps measure, so the two agree up to the
profiler's own cost.
"""
from __future__ import annotations

import argparse
import csv
import json
import re
import statistics
import subprocess
import sys
from collections import defaultdict
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent.parent
PROFILES = REPO / "profiles"
RESOURCE_USAGE = PKG / "_build" / "resource_usage.json"
COPY_KERNEL = "__amd_rocclr_copyBuffer"
CALIB_BYTES = 1 << 30         # bench.py --calib-copy: one plain 1 GiB device-to-device copy
NUM_XCD, NUM_CU, NUM_SIMD = 8, 256, 1024
PEAK = {"TFLOP/s": 2500.0, "GB/s": 8000.0}
# Shortest kernel whose clock is derived from GRBM_GUI_ACTIVE / duration: that
# counter also counts busy cycles around each dispatch, which inflate the
# derived clock of short kernels.
CLOCK_MIN_S = 250e-6


def zero_counters(c):
    """Counters of one kernel's table that read 0 on every pass."""
    names = {nn for (_, nn) in c}
    return sorted(n for n in names if all(v == 0 for (_, nn), v in c.items() if nn == n))


def short_name(name: str) -> str:
    """``ak::kernel<args>`` from a mangled (_ZN2ak...) or demangled kernel name;
    other names unchanged."""
    d = re.search(r"ak::(\w+)<([^>]*)>", name)
    if d and not name.startswith("_Z"):
        return f"{d.group(1)}<{d.group(2).replace(' ', '')}>"
    m = re.match(r"_ZN2ak(\d+)", name)
    if not m:
        return name
    n = int(m.group(1))
    i = m.end()
    base, rest = name[i:i + n], name[i + n:]
    args = []
    if rest.startswith("I"):
        for a in re.finditer(r"L([ib])(\d+)E", rest[1:rest.index("EE") + 1]):
            args.append(("true" if a.group(2) == "1" else "false") if a.group(1) == "b" else a.group(2))
    return f"{base}<{','.join(args)}>" if args else base


# bench.py's read-ceiling kernel (measured_ceilings): part of every run, of
# no workload.
CEILING_KERNELS = ("stream_checksum_kernel",)


def ours(name: str) -> bool:
    """A kernel of this library that belongs to the profiled workload."""
    return ("_ZN2ak" in name or "ak::" in name) and not any(k in name for k in CEILING_KERNELS)


def load_dispatches(path: Path):
    """[(short name, start ns, end ns, row)] of this library's kernels, in dispatch order."""
    rows = [r for r in csv.DictReader(open(path)) if ours(r["Kernel_Name"])]
    rows.sort(key=lambda r: int(r["Dispatch_Id"]))
    return [(short_name(r["Kernel_Name"]), int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r) for r in rows]


# bench.py's diagnostic input patterns (--inputs): a workload named W_<pattern>
# is bench.py's workload W run on those prefill inputs.
INPUT_PATTERNS = ("signs", "ones", "zeros")


def bench_args(workload: str) -> str:
    """The bench.py arguments that select ``workload``."""
    for p in INPUT_PATTERNS:
        if workload.endswith("_" + p):
            return f"--only {workload[:-len(p) - 1]} --inputs {p}"
    return f"--only {workload}"


def bench_record(path: Path, workload: str) -> dict:
    """The workload's entry in a bench.py JSON line (the headline line itself, or
    one of its ``workloads``)."""
    line = json.loads(path.read_text().strip().splitlines()[-1])
    common = {k: line.get(k) for k in ("steps", "warmup", "sources_sha256")}
    for w in line.get("workloads", []):
        if w.get("name") == workload:
            return {**w, **common}
    if "config" in line:  # the headline workload
        rec = dict(line)
        rec["workload"] = line["config"]["workload"]
        rec["flop_per_launch"] = line.get("flop_per_launch")
        return rec
    raise SystemExit(f"{workload}: not in {path}")


def by_kernel(dispatches):
    per = defaultdict(list)
    for name, s, e, row in dispatches:
        per[name].append((s, e, row))
    return per


def window(seq, n0, k):
    return seq[n0:n0 + k]


def stats_us(durs_ns):
    us = [d / 1e3 for d in durs_ns]
    return dict(n=len(us), mean=statistics.fmean(us), median=statistics.median(us), min=min(us), max=max(us))


def commit_note(digest):
    """Which commit the measured sources are, by their digest (bench.py reports
    the digest of the sources it ran; the GPU box has no git metadata)."""
    sys.path.insert(0, str(PKG.parent))
    from attnkernels import build  # noqa: E402

    try:
        head = subprocess.run(["git", "-C", str(REPO), "rev-parse", "--short", "HEAD"], capture_output=True,
                              text=True).stdout.strip()
    except OSError:
        head = "?"
    if digest and digest == build.sources_digest():
        return f"sources digest {digest[:12]} = the kernel sources of commit {head}"
    return f"sources digest {str(digest)[:12]} (differs from the tree at commit {head}: re-profile)"


def trace_summary(workload: str, raw: Path, out_dir: Path = PROFILES):
    rec = bench_record(raw / "bench_trace.json", workload)
    K, n0 = int(rec.get("steps") or 20), int(rec["calls_before_timed"])
    per = by_kernel(load_dispatches(raw / "trace_kernel_trace.csv"))
    if not per:
        raise SystemExit("no attnkernels dispatches in the trace")
    kstats, fstats = {}, {}
    for name, seq in per.items():
        tw, fw = window(seq, n0, K), window(seq, n0 + 2 * K, K)
        if len(tw) != K:
            raise SystemExit(f"{name}: {len(seq)} dispatches, cannot take {K} timed ones from #{n0}")
        kstats[name] = stats_us([e - s for s, e, _ in tw])
        if len(fw) == K:
            fstats[name] = stats_us([e - s for s, e, _ in fw])
    dom = max(kstats, key=lambda k: kstats[k]["mean"])
    # Trace-side steps: start of one timed call's first kernel to the next call's.
    firsts = [min(seq[i][0] for seq in per.values()) for i in range(n0, n0 + K)]
    steps_us = [(b - a) / 1e3 for a, b in zip(firsts[:-1], firsts[1:])]
    step_mean, step_med = statistics.fmean(steps_us), statistics.median(steps_us)
    unit = rec.get("unit", "TFLOP/s")
    work = rec.get("flop_per_launch") if unit == "TFLOP/s" else rec.get("bytes_per_step")
    scale = 1e12 if unit == "TFLOP/s" else 1e9
    fetch_scale = write_scale = None
    traffic = {}
    for which, counter in (("fetch", "FETCH_SIZE"), ("write", "WRITE_SIZE")):
        p = raw / f"{which}_counter_collection.csv"
        if not p.exists():
            continue
        calib, vals = counter_window(p, counter, raw / f"bench_{which}.json", workload)
        sc = CALIB_BYTES / 1024 / calib if calib else None
        if which == "fetch":
            fetch_scale = sc
        else:
            write_scale = sc
        for k, v in vals.items():
            traffic.setdefault(k, {})[which] = v
    cmd_dir = f"gpurun_out/praw/{workload}"
    sel = bench_args(workload)
    lines = [f"# rocprofv3: {dom} on `{workload}`", "",
             f"Workload: {rec.get('workload')} (MI355X, one GPU; inputs resident in HBM).", "",
             f"Measured: {commit_note(rec.get('sources_sha256'))}.", "",
             "Commands (repository root on the GPU box, `export TMPDIR=/tmp`), then the summary on the host:", "",
             f"    rocprofv3 --kernel-trace --stats --output-format csv -d {cmd_dir} -o trace -- python bench.py "
             f"{sel} --steps {K} --warmup {rec.get('warmup', 5)} --cpu-seconds 0 > {cmd_dir}/bench_trace.json"]
    for which, counter in (("fetch", "FETCH_SIZE"), ("write", "WRITE_SIZE")):
        if (raw / f"{which}_counter_collection.csv").exists():
            lines.append(f"    rocprofv3 --pmc {counter} --output-format csv -d {cmd_dir} -o {which} -- python bench.py "
                         f"{sel} --steps 3 --warmup 1 --settle-seconds 0 --cpu-seconds 0 --calib-copy "
                         f"> {cmd_dir}/bench_{which}.json")
    lines += [f"    python flash-attention-from-scratch_amd/attnkernels/profiling.py trace {workload} {cmd_dir}", "",
             f"## Kernel time over the {K} timed steps (`--kernel-trace`; dispatches #{n0}..#{n0 + K - 1} of each kernel)",
             "", "| kernel | dispatches | mean us | median us | min us | max us | flushed median us |",
             "|---|---:|---:|---:|---:|---:|---:|"]
    for name, st in sorted(kstats.items(), key=lambda kv: -kv[1]["mean"]):
        fm = f"{fstats[name]['median']:.1f}" if name in fstats else ""
        lines.append(f"| {name} | {st['n']} | {st['mean']:.1f} | {st['median']:.1f} | {st['min']:.1f} | "
                     f"{st['max']:.1f} | {fm} |")
    lines += ["", f"Steps in the trace (start of one timed step's first kernel to the next one's, {K - 1} steps): "
                  f"mean {step_mean:.1f} us, median {step_med:.1f} us.",
              f"bench.py in the same run (timed steps between two HIP events; median from marked steps): mean "
              f"{rec['kernel_ms_mean'] * 1e3:.1f} us, median {rec['kernel_ms_median'] * 1e3:.1f} us per step; "
              f"`ms_per_step` (wall clock) {rec['ms_per_step'] * 1e3:.1f} us."]
    if work:
        r_step, r_kern = work / (step_mean * 1e-6) / scale, work / (kstats[dom]["mean"] * 1e-6) / scale
        lines += ["", f"Algorithmic work per step: {work:.4g} {'FLOP' if unit == 'TFLOP/s' else 'bytes'}. "
                      f"Over the trace's step mean: {r_step:.1f} {unit} = {r_step / PEAK[unit]:.4f} of "
                      f"{PEAK[unit]:.0f} {unit}; over {dom}'s own mean: {r_kern:.1f} {unit} = "
                      f"{r_kern / PEAK[unit]:.4f}. bench.py's line in this run: achieved "
                      f"{rec.get('kernel_tflops') or rec.get('kernel_gbs') or rec.get('roofline', {}).get('achieved')} "
                      f"{unit}, frac {rec.get('frac_of_peak') or rec.get('roofline', {}).get('frac')}."]
    entry = None
    if traffic.get(dom, {}).get("fetch") is not None and fetch_scale and write_scale:
        lines += ["", "## HBM traffic (`--pmc FETCH_SIZE`, `--pmc WRITE_SIZE`, KiB per dispatch, timed steps)", "",
                  f"Calibration: the 1 GiB copy reads FETCH_SIZE = {CALIB_BYTES / 1024 / fetch_scale:.0f} KiB and "
                  f"WRITE_SIZE = {CALIB_BYTES / 1024 / write_scale:.0f} KiB: scale {fetch_scale:.3f} (fetch) and "
                  f"{write_scale:.3f} (write) to bytes.", "",
                  "| kernel | FETCH_SIZE KiB | WRITE_SIZE KiB | fetched | written |", "|---|---:|---:|---:|---:|"]
        for k, t in sorted(traffic.items()):
            f_, w_ = t.get("fetch", 0.0), t.get("write", 0.0)
            lines.append(f"| {k} | {f_:.0f} | {w_:.0f} | {f_ * 1024 * fetch_scale / 1e9:.4f} GB | "
                         f"{w_ * 1024 * write_scale / 1e9:.4f} GB |")
        fb = traffic[dom]["fetch"] * 1024 * fetch_scale
        wb = traffic[dom].get("write", 0.0) * 1024 * write_scale
        lines += ["", f"{dom}: HBM traffic {(fb + wb) / 1e9:.4f} GB per launch (fetch {fb / 1e9:.4f} + write "
                      f"{wb / 1e9:.4f})" + (f", {(fb + wb) / work:.3f}x the algorithmic bytes." if unit == "GB/s" and work
                                            else ".")]
        entry = dict(kernel=dom, avg_us=round(kstats[dom]["mean"], 2), median_us=round(kstats[dom]["median"], 2),
                     step_us=round(step_mean, 2), fetch_bytes=int(fb), write_bytes=int(wb),
                     traffic_bytes=int(fb) + int(wb), fetch_scale=round(fetch_scale, 4),
                     write_scale=round(write_scale, 4))
    out = out_dir / f"{dom.split('<')[0]}_{workload}.md"
    out.write_text("\n".join(lines) + "\n")
    if entry:
        entry["source"] = f"profiles/{out.name}"
        tj_path = out_dir / "traffic.json"
        tj = json.loads(tj_path.read_text()) if tj_path.exists() else {}
        tj[workload] = entry
        tj_path.write_text(json.dumps(tj, indent=1, sort_keys=True) + "\n")
    return out, dom, kstats[dom], step_mean


def counter_window(path: Path, counter: str, bench_json: Path, workload: str):
    """(calibration copy's value or None, {kernel: mean over the timed dispatches})."""
    rows = [r for r in csv.DictReader(open(path)) if r["Counter_Name"] == counter]
    rows.sort(key=lambda r: int(r["Dispatch_Id"]))
    calib = next((float(r["Counter_Value"]) for r in rows if r["Kernel_Name"] == COPY_KERNEL), None)
    per = defaultdict(list)
    for r in rows:
        if ours(r["Kernel_Name"]):
            per[short_name(r["Kernel_Name"])].append(float(r["Counter_Value"]))
    n0, K = 0, None
    if bench_json.exists():
        rec = bench_record(bench_json, workload)
        n0, K = int(rec["calls_before_timed"]), int(rec.get("steps") or 3)
    out = {}
    for k, v in per.items():
        sel = v[n0:n0 + K] if K else v
        out[k] = statistics.fmean(sel or v)
    return calib, out


def counters_summary(workload: str, raw: Path, passes, out_dir: Path = PROFILES):
    """Per kernel: every counter of every pass (mean over the timed dispatches,
    summed over XCDs), plus derived clock, MFMA utilisation, co-issue, LDS bank
    conflicts and occupancy against the compiler's register allocation."""
    usage = json.loads(RESOURCE_USAGE.read_text()) if RESOURCE_USAGE.exists() else {}
    usage = {short_name(k): v for k, v in usage.items()}
    vals, dur, meta, cmds = defaultdict(dict), defaultdict(list), {}, []
    digest = None
    for p in passes:
        bj = raw / f"bench_{p}.json"
        rec = bench_record(bj, workload)
        digest = digest or rec.get("sources_sha256")
        n0, K = int(rec["calls_before_timed"]), int(rec.get("steps") or 3)
        per = defaultdict(lambda: defaultdict(list))
        names = []
        for r in sorted(csv.DictReader(open(raw / f"{p}_counter_collection.csv")), key=lambda r: int(r["Dispatch_Id"])):
            if not ours(r["Kernel_Name"]):
                continue
            k = short_name(r["Kernel_Name"])
            per[k][r["Counter_Name"]].append(float(r["Counter_Value"]))
            if r["Counter_Name"] == "GRBM_GUI_ACTIVE":
                dur[k].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-9)
            meta[k] = r
            if r["Counter_Name"] not in names:
                names.append(r["Counter_Name"])
        for k, c in per.items():
            for n, v in c.items():
                vals[k][(p, n)] = statistics.fmean(v[n0:n0 + K] or v)
        cmds.append(f"    rocprofv3 --pmc {' '.join(names)} --output-format csv -d gpurun_out/praw/{workload} -o {p} -- "
                    f"python bench.py {bench_args(workload)} --steps {K} --warmup 1 --settle-seconds 0 --cpu-seconds 0 "
                    f"> gpurun_out/praw/{workload}/bench_{p}.json")
    outs = []
    for k, c in vals.items():
        def get(n):
            for (p, nn), v in c.items():
                if nn == n:
                    return v
            return None
        lines = [f"# rocprofv3 counters: {k} on `{workload}`", "",
                 f"Measured: {commit_note(digest)}.", "",
                 f"{len(passes)} counter passes (MI355X, one GPU), repository root on the GPU box, `export TMPDIR=/tmp`; "
                 "then the summary on the host:", "", *cmds,
                 f"    python flash-attention-from-scratch_amd/attnkernels/profiling.py counters {workload} "
                 f"gpurun_out/praw/{workload} {' '.join(passes)}", "",
                 "Values are per dispatch, averaged over the timed steps' dispatches and summed over the 8 XCDs "
                 "(GRBM_GUI_ACTIVE / 8 = one XCD's active cycles).", "",
                 "| counter | " + " | ".join(passes) + " |", "|---|" + "---:|" * len(passes)]
        for n in sorted({nn for (_, nn) in c}):
            if n in zero_counters(c):
                continue
            lines.append(f"| {n} | " + " | ".join(f"{c[(p, n)]:.4g}" if (p, n) in c else "" for p in passes) + " |")
        gui = (get("GRBM_GUI_ACTIVE") or 0) / NUM_XCD
        d_s = statistics.fmean(dur[k]) if dur[k] else 0.0
        zero = zero_counters(c)
        if zero:
            lines += ["", "Left out of the table: " + ", ".join(zero) + " (read 0 on every timed dispatch"
                      + ("; SQ_ACTIVE_INST_VMEM = 0 on a kernel that streams its data through vector loads is "
                         "not a count, so the counter does not count on this GPU" if "SQ_ACTIVE_INST_VMEM" in zero
                         else "") + ")."]
        lines += ["", "Derived:", ""]
        if gui and d_s >= CLOCK_MIN_S:
            lines.append(f"- kernel duration under the counters {d_s * 1e6:.1f} us; shader clock = GRBM_GUI_ACTIVE / 8 / "
                         f"duration = **{gui / d_s / 1e9:.2f} GHz** (peak engine clock 2.4 GHz)")
        elif gui and d_s:
            lines.append(f"- kernel duration under the counters {d_s * 1e6:.1f} us: too short to derive the clock. "
                         "GRBM_GUI_ACTIVE also counts busy cycles around the dispatch, which a kernel under "
                         f"{CLOCK_MIN_S * 1e6:.0f} us does not amortise (a 45 us decode kernel read 2.55 GHz, above "
                         "the 2.4 GHz peak); the ratios below that divide by GRBM_GUI_ACTIVE are lower bounds")
        mb, mi = get("SQ_VALU_MFMA_BUSY_CYCLES"), get("SQ_INSTS_MFMA")
        if mb is not None and gui:
            lines.append(f"- MFMA utilisation (SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE per XCD x 1024 SIMDs)) = "
                         f"**{mb / (gui * NUM_SIMD) * 100:.1f}%**" if mi else
                         "- no MFMA instructions: the kernel runs on the VALU by design")
        co = get("SQ_VALU_MFMA_COEXEC_CYCLES")
        if co is not None and mb:
            lines.append(f"- MFMA busy cycles co-issuing with VALU: {co / mb * 100:.1f}%")
        va, wc = get("SQ_ACTIVE_INST_VALU"), get("SQ_WAVE_CYCLES")
        if va is not None and gui:
            lines.append(f"- VALU issue: SQ_ACTIVE_INST_VALU x 4 / (1024 SIMDs x active cycles) = "
                         f"{va * 4 / (NUM_SIMD * gui) * 100:.1f}% of SIMD cycles")
        tr, iv = get("SQ_INSTS_VALU_TRANS_F32"), get("SQ_INSTS_VALU")
        if tr is not None and iv:
            lines.append(f"- transcendental share of VALU instructions: {tr / iv * 100:.1f}%")
        bc, la = get("SQ_LDS_BANK_CONFLICT"), get("SQ_LDS_IDX_ACTIVE")
        if bc is not None and la:
            lines.append(f"- LDS bank conflicts: {bc:.4g} cycles of {la:.4g} LDS-active ({bc / la * 100:.2f}%)")
        wa = get("SQ_WAIT_ANY")
        if wa is not None and wc:
            lines.append(f"- waves waiting (SQ_WAIT_ANY / SQ_WAVE_CYCLES): {wa / wc * 100:.1f}% of wave cycles")
        if wc and gui:
            res = f"- resident waves per CU = 4 x SQ_WAVE_CYCLES / (GRBM_GUI_ACTIVE per XCD) / 256 = **{4 * wc / gui / NUM_CU:.2f}**"
            u = usage.get(k)
            if u:
                res += (f"; the compiler's allocation: {u['VGPRs']} VGPRs + {u['AGPRs']} AGPRs, {u['VGPRs Spill']} spilled, "
                        f"{u['Occupancy']} waves per SIMD ({4 * u['Occupancy']} per CU), LDS {u['LDS Size']} B per "
                        f"workgroup of {int(meta[k].get('Workgroup_Size_X') or meta[k].get('Workgroup_Size', 64)) // 64} waves")
            lines.append(res)
        out = out_dir / f"{k.split('<')[0]}_{workload}_counters.md"
        out.write_text("\n".join(lines) + "\n")
        outs.append(out)
    return outs


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    sub = ap.add_subparsers(dest="cmd", required=True)
    t = sub.add_parser("trace")
    t.add_argument("workload")
    t.add_argument("raw", type=Path)
    c = sub.add_parser("counters")
    c.add_argument("workload")
    c.add_argument("raw", type=Path)
    c.add_argument("passes", nargs="+")
    a = ap.parse_args(argv)
    if a.cmd == "trace":
        out, dom, st, step = trace_summary(a.workload, a.raw)
        print(f"{out.relative_to(REPO)}: {dom} mean {st['mean']:.1f} us median {st['median']:.1f} us; "
              f"trace step mean {step:.1f} us")
    else:
        for out in counters_summary(a.workload, a.raw, a.passes):
            print(out.relative_to(REPO))


if __name__ == "__main__":
    main()
