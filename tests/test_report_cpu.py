"""CPU checks of the comparison-suite report (attnkernels.report) on a small
synthetic results file, and of the committed MI355X results."""
import json
from pathlib import Path

from attnkernels import report

ROOT = Path(__file__).resolve().parents[1]


def _rows():
    rows = []
    for impl, ms in (("flash_attention", 0.5), ("sdpa_fused", 1.0)):
        rows.append(dict(section="prefill", impl=impl, batch=2, heads=16, seq=8192, head_dim=128, causal=True,
                         ms=ms, tflops=2200.0 / ms / 2, peak_mem_mb=64.0, max_abs_err=5e-4,
                         speedup_vs_sdpa=1.0 / ms))
    for p, gbs in ((256, 3000.0), (512, 3600.0), (1024, 3100.0)):
        rows.append(dict(section="split_ablation", impl="paged_split", batch=1, ctx=4096, kv_heads=8,
                         partition=p, gbs=gbs, ms=1.0, max_abs_err=1e-5))
    rows.append(dict(section="decode", impl="paged_split", batch=4, ctx=4096, partition=512, gbs=4000.0,
                     ms=0.1, max_abs_err=1e-5, speedup_vs_torch_gather=5.0))
    rows.append(dict(section="decode", impl="torch_gather_sdpa", batch=4, ctx=4096, gbs=800.0, ms=0.5,
                     max_abs_err=1e-5, speedup_vs_torch_gather=1.0))
    for impl, mem, err in (("flash_attention", 32.0, 4e-4), ("sdpa_fused", 48.0, 9e-4)):
        rows.append(dict(section="prefill", impl=impl, batch=8, heads=16, seq=2048, head_dim=64, causal=False,
                         ms=0.1, tflops=700.0, peak_mem_mb=mem, max_abs_err=err, speedup_vs_sdpa=None))
    for g, gbs in ((1, 6000.0), (8, 4000.0)):
        rows.append(dict(section="decode_heads", impl="paged_split", batch=16, ctx=8192, heads=8 * g, kv_heads=8,
                         head_dim=128, group=g, partition=512, ms=0.09, gbs=gbs, max_abs_err=2e-5 * g,
                         **(dict(max_abs_err_one_head_path=2e-5) if g > 1 else {})))
    return rows


def test_render_synthetic():
    meta = dict(gpu="MI355X", arch="gfx950", cu_count=256, torch="x", hip="y", date="d", timing="t",
                roofs=dict(copy_gbs=4000.0, fp16_gemm_tflops=1250.0), sdpa_backends={"FLASH_ATTENTION": "ok"})
    md = report.render(dict(meta=meta, results=_rows()))
    assert "## Prefill" in md and "## Paged decode" in md and "## Split-K partition ablation" in md
    assert "| 2x8192 | 2200.0 | 1100.0 | 88.0% | 2.0x | 5.0e-04 |" in md
    assert "| 32/8 | 1 | 4096 | 512 | 3600 |" in md  # best partition of the ablation
    assert "| 4 | 4096 | 4000 | 800 | 50.0% | 512 | 5.0x |" in md
    assert "50% of 8 TB/s" in md and "50% of 2.5 PFLOP/s" in md
    # peak memory (non-causal only), time per call, head groups, worst error per implementation
    assert "### Prefill peak extra memory" in md
    assert "| 8x2048 | 32 | 48 |" in md
    assert "| 4 | 4096 | 0.1000 | 0.5000 |" in md
    assert "| 128 | 8 | 64 | 8 | 16 | 8192 | 512 | 0.0900 | 4000 | 50.0% |" in md
    assert "| prefill | sdpa_fused | 2 | 9.00e-04 |" in md
    assert "| prefill | flash_attention | 2 | 5.00e-04 |" in md
    assert "| decode | paged_split | 6 | 1.60e-04 |" in md
    # the grouped kernel's error beside the one-head kernel's on the same data
    assert "| 128 | 8 | 16 x 8192 | 1.60e-04 | 2.00e-05 |" in md
    assert "| 128 | 1 | 16 x 8192 | 2.00e-05 | (the same kernel) |" in md


def test_committed_results_render():
    data = json.loads((ROOT / "results" / "mi355x.json").read_text())
    md = report.render(data)
    assert md.startswith("# Attention kernels on")
    ours = [r for r in data["results"] if r["section"] == "prefill" and r["impl"] == "flash_attention"]
    assert ours and all(r["max_abs_err"] < 4e-3 for r in ours)
    dec = [r for r in data["results"] if r["impl"] == "paged_split"]
    assert dec and all(r["max_abs_err"] < 2e-3 for r in dec)


def test_activity_table():
    rows = []
    for data, pre, gemm in (("randn", 1000.0, 1250.0), ("zeros", 1400.0, 1750.0)):
        rows.append(dict(section="input_activity", impl="flash_attention", workload="prefill causal N=8192",
                         data=data, tflops=pre, ms=1.0, max_abs_err=1e-3))
        rows.append(dict(section="input_activity", impl="hipblaslt_gemm", workload="fp16 GEMM 8192^3",
                         data=data, tflops=gemm, ms=1.0, max_abs_err=0.0))
    md = report.activity_table(rows)
    assert "| inputs | prefill causal N=8192 TFLOP/s | fp16 GEMM 8192^3 TFLOP/s | prefill causal N=8192 / GEMM |" in md
    assert "| randn | 1000 (40%) | 1250 (50%) | 80% |" in md
    assert "| zeros | 1400 (56%) | 1750 (70%) | 80% |" in md
    meta = dict(gpu="MI355X", arch="gfx950", cu_count=256, torch="x", hip="y", date="d", timing="t",
                roofs=dict(copy_gbs=4000.0, fp16_gemm_tflops=1250.0), sdpa_backends={})
    assert "## Rate against input bit activity" in report.render(dict(meta=meta, results=rows))
