"""attnkernels.profiling on synthetic rocprofv3 output (CPU): only the timed
dispatches are summarised, picked by bench.py's calls_before_timed, and the
trace-side step time is the start-to-start period of those steps."""
import csv
import json

import pytest

from attnkernels import profiling

HEADER = ["Kind", "Agent_Id", "Queue_Id", "Stream_Id", "Thread_Id", "Dispatch_Id", "Kernel_Id", "Kernel_Name",
          "Correlation_Id", "Start_Timestamp", "End_Timestamp", "LDS_Block_Size", "Scratch_Size", "VGPR_Count",
          "Accum_VGPR_Count", "SGPR_Count", "Workgroup_Size_X", "Workgroup_Size_Y", "Workgroup_Size_Z",
          "Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z"]
DEC = "void ak::paged_decode_kernel<128, 4>(_Float16 const*, int)"
RED = "void ak::paged_reduce_kernel<128>(float const*, int)"


def write_trace(path, calls):
    """calls: list of [(name, start, end)] per bench.py call; torch kernels in between."""
    rows, did = [], 0
    for kernels in calls:
        did += 1
        rows.append(["KERNEL_DISPATCH"] + [""] * 4 + [did, 1, "void at::native::fill_kernel()", did, 0, 1] +
                    [""] * 11)
        for name, s, e in kernels:
            did += 1
            rows.append(["KERNEL_DISPATCH"] + [""] * 4 + [did, 2, name, did, s, e] + [""] * 11)
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(HEADER)
        w.writerows(rows)


def test_short_names():
    assert profiling.short_name(DEC) == "paged_decode_kernel<128,4>"
    assert profiling.short_name("_ZN2ak20flash_prefill_kernelILi128ELb1ELb0ELi8EEEvPKDF16_") == \
        "flash_prefill_kernel<128,true,false,8>"
    assert not profiling.ours("void at::native::fill_kernel()")


def test_trace_summary_takes_only_the_timed_steps(tmp_path):
    n0, K = 7, 5
    calls, t = [], 0
    # settle/warmup calls, the K timed steps, K marked steps, K flushed steps
    for i in range(n0 + 3 * K):
        if i < n0:
            d = 300_000  # settle / warmup calls are slower: they must not enter the stats
        elif i < n0 + K:
            d = 100_000 + 1000 * (i - n0)
        elif i < n0 + 2 * K:
            d = 150_000  # marked steps: neither timed nor flushed
        else:
            d = 200_000  # flushed steps
        calls.append([(DEC, t, t + d), (RED, t + d + 2000, t + d + 7000)])
        t += d + 10_000
    raw = tmp_path / "raw"
    raw.mkdir()
    write_trace(raw / "trace_kernel_trace.csv", calls)
    rec = {"name": "decode_x", "workload": "paged decode test", "unit": "GB/s", "bytes_per_step": 1e9,
           "calls_before_timed": n0, "kernel_ms_mean": 0.112, "kernel_ms_median": 0.112, "ms_per_step": 0.113,
           "kernel_gbs": 8900.0, "frac_of_peak": 1.1}
    (raw / "bench_trace.json").write_text(json.dumps({"workloads": [rec], "steps": K, "warmup": 2,
                                                      "sources_sha256": "0" * 64}) + "\n")
    out_dir = tmp_path / "profiles"
    out_dir.mkdir()
    out, dom, st, step = profiling.trace_summary("decode_x", raw, out_dir)
    assert dom == "paged_decode_kernel<128,4>"
    assert st["n"] == K
    assert st["mean"] == pytest.approx(102.0)          # 100..104 us, the settle calls excluded
    assert st["median"] == pytest.approx(102.0)
    assert step == pytest.approx(101.5 + 10.0)         # K-1 start-to-start periods: 100..103 us + 10 us gap
    text = out.read_text()
    assert "dispatches #7..#11" in text and "flushed median" in text
    # the flushed column takes the last K calls, after the marked ones
    assert "| paged_decode_kernel<128,4> | 5 | 102.0 | 102.0 | 100.0 | 104.0 | 200.0 |" in text


def test_trace_summary_refuses_a_short_trace(tmp_path):
    raw = tmp_path / "raw"
    raw.mkdir()
    write_trace(raw / "trace_kernel_trace.csv", [[(DEC, 0, 10)]] * 3)
    (raw / "bench_trace.json").write_text(json.dumps({"workloads": [{"name": "w", "calls_before_timed": 2,
                                                                     "unit": "GB/s"}], "steps": 5}) + "\n")
    with pytest.raises(SystemExit):
        profiling.trace_summary("w", raw, tmp_path)


def test_resource_usage_remarks_parse():
    from attnkernels import build
    text = """x.hip:80:1: remark: Function Name: _ZN2ak19paged_decode_kernelILi64ELi1EEEv [-Rpass-analysis=kernel-resource-usage]
x.hip:80:1: remark:     VGPRs: 60 [-Rpass-analysis=kernel-resource-usage]
x.hip:80:1: remark:     Occupancy [waves/SIMD]: 8 [-Rpass-analysis=kernel-resource-usage]
x.hip:80:1: remark:     LDS Size [bytes/block]: 2112 [-Rpass-analysis=kernel-resource-usage]"""
    u = build.parse_resource_usage(text)
    assert u == {"_ZN2ak19paged_decode_kernelILi64ELi1EEEv": {"VGPRs": 60, "Occupancy": 8, "LDS Size": 2112}}


def test_bench_args_of_input_patterns():
    assert profiling.bench_args("decode_gqa16_d128") == "--only decode_gqa16_d128"
    assert profiling.bench_args("prefill_d128_n8192_causal_zeros") == "--only prefill_d128_n8192_causal --inputs zeros"
    assert profiling.bench_args("prefill_d64_n2048_signs") == "--only prefill_d64_n2048 --inputs signs"


CTR_HEADER = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value", "Start_Timestamp", "End_Timestamp",
              "Workgroup_Size"]
PRE = "void ak::flash_prefill_kernel<128, true, false, 8, 16>(_Float16 const*, int)"
CEIL = "ak::stream_checksum_kernel(unsigned int __vector(4) const*, unsigned long, unsigned long, unsigned int*)"


def test_counters_summary_rules(tmp_path):
    """Counters that read 0 on every timed dispatch are listed, not tabled;
    the clock is derived only for kernels of 250 us or more (a 50 us kernel
    whose GRBM_GUI_ACTIVE implies 2.55 GHz gets no clock line); bench.py's
    read-ceiling kernel gets no summary."""
    raw = tmp_path / "raw"
    raw.mkdir()
    n0, K = 2, 3
    kernels = {DEC: (50_000, 2.55e9), PRE: (1_000_000, 2.0e9), CEIL: (300_000, 2.4e9)}
    passes = {"ctr1": ("GRBM_GUI_ACTIVE", "SQ_WAVE_CYCLES", "SQ_ACTIVE_INST_VMEM"),
              "ctr2": ("GRBM_GUI_ACTIVE", "SQ_WAIT_ANY")}
    for p, names in passes.items():
        rows, did, t = [], 0, 0
        for _ in range(n0 + K):
            for name, (dur_ns, clock) in kernels.items():
                did += 1
                for c in names:
                    v = {"GRBM_GUI_ACTIVE": 8 * clock * dur_ns * 1e-9, "SQ_WAVE_CYCLES": 1e6,
                         "SQ_ACTIVE_INST_VMEM": 0.0, "SQ_WAIT_ANY": 3e5}[c]
                    rows.append([did, name, c, v, t, t + dur_ns, 256])
                t += dur_ns + 1000
        with open(raw / f"{p}_counter_collection.csv", "w", newline="") as f:
            w = csv.writer(f)
            w.writerow(CTR_HEADER)
            w.writerows(rows)
        (raw / f"bench_{p}.json").write_text(json.dumps({"workloads": [{"name": "w", "calls_before_timed": n0}],
                                                          "steps": K, "sources_sha256": "0" * 64}) + "\n")
    out_dir = tmp_path / "profiles"
    out_dir.mkdir()
    outs = {o.name: o.read_text() for o in profiling.counters_summary("w", raw, list(passes), out_dir)}
    assert set(outs) == {"paged_decode_kernel_w_counters.md", "flash_prefill_kernel_w_counters.md"}
    dec, pre = outs["paged_decode_kernel_w_counters.md"], outs["flash_prefill_kernel_w_counters.md"]
    assert "Left out of the table: SQ_ACTIVE_INST_VMEM" in dec and "| SQ_ACTIVE_INST_VMEM |" not in dec
    assert "too short to derive the clock" in dec and "GHz**" not in dec
    assert "**2.00 GHz**" in pre and "too short" not in pre
