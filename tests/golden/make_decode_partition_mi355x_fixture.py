"""Write decode_partition_mi355x.json: for every case of the split-K ablations in
results/mi355x.json (python -m attnkernels.benchsuite on one MI355X; uniform and
mixed context lengths), the decode bandwidth of every partition.  A test checks
that decode_partition's default rule lands near the fastest one on 256 CUs.

    python tests/golden/make_decode_partition_mi355x_fixture.py [results.json]
"""
import json
import sys
from collections import defaultdict
from pathlib import Path

root = Path(__file__).resolve().parents[2]
src = Path(sys.argv[1]) if len(sys.argv) > 1 else root / "results" / "mi355x.json"
data = json.loads(src.read_text())
cases = defaultdict(list)
for r in data["results"]:
    if r["section"] in ("split_ablation", "split_ablation_ragged"):
        cases[(r["batch"], r["heads"], r["kv_heads"], r["ctx"], r["section"])].append(r)
rows = []
for (b, hq, hkv, ctx, sec), rs in sorted(cases.items()):
    best = max(rs, key=lambda r: r["gbs"])
    rows.append(dict(batch=b, num_heads=hq, num_kv_heads=hkv, max_context_len=ctx,
                     mixed_lengths=sec != "split_ablation",
                     best_partition=best["partition"],
                     gbs={str(r["partition"]): r["gbs"] for r in sorted(rs, key=lambda r: r["partition"])}))
out = dict(source="attnkernels.benchsuite split_ablation (" + data["meta"]["date"] + ")",
           cu_count=data["meta"]["cu_count"], rows=rows)
(Path(__file__).resolve().parent / "decode_partition_mi355x.json").write_text(json.dumps(out, indent=1) + "\n")
print(len(rows), "rows")
