"""Write decode_partition_mi355x.json: for every case of the split-K ablations in
results/mi355x.json (python -m attnkernels.benchsuite on one MI355X; uniform and
mixed context lengths), the decode bandwidth of every partition.  A test checks
that decode_partition's default rule lands near the fastest one on 256 CUs.

    python tests/golden/make_decode_partition_mi355x_fixture.py
"""
import json
from collections import defaultdict
from pathlib import Path

root = Path(__file__).resolve().parents[2]
data = json.loads((root / "results" / "mi355x.json").read_text())
cases = defaultdict(list)
for r in data["results"]:
    if r["section"] in ("split_ablation", "split_ablation_ragged"):
        cases[(r["batch"], r["kv_heads"], r["ctx"])].append(r)
rows = []
for (b, hkv, ctx), rs in sorted(cases.items()):
    best = max(rs, key=lambda r: r["gbs"])
    rows.append(dict(batch=b, num_kv_heads=hkv, max_context_len=ctx, mixed_lengths=rs[0]["section"] != "split_ablation",
                     best_partition=best["partition"],
                     gbs={str(r["partition"]): r["gbs"] for r in sorted(rs, key=lambda r: r["partition"])}))
out = dict(source="results/mi355x.json split_ablation (" + data["meta"]["date"] + ")",
           cu_count=data["meta"]["cu_count"], rows=rows)
(Path(__file__).resolve().parent / "decode_partition_mi355x.json").write_text(json.dumps(out, indent=1) + "\n")
print(len(rows), "rows")
