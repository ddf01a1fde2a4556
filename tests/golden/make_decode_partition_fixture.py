"""Write decode_partition_t4.json: the (batch, kv_heads, max_ctx) -> partition rows
that the reference's recorded T4 run holds (results/t4.json, rows with impl
"paged_split" in sections "decode" and "ragged"; sm_count from its meta).

Runs in the build container only (it reads /root/reference as JSON data);
the fixture it writes is committed and is all the tests read.
"""
import json
import sys
from pathlib import Path

src = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/results/t4.json")
data = json.loads(src.read_text())
rows = []
for r in data["results"]:
    if r.get("impl") == "paged_split" and r.get("section") in ("decode", "ragged"):
        rows.append(dict(batch=r["batch"], num_kv_heads=r["kv_heads"], max_context_len=r["ctx"],
                         partition=r["partition"], splits=r["splits"], section=r["section"]))
out = dict(source="sonhoang/flash-attention-from-scratch results/t4.json",
           sm_count=data["meta"]["sm_count"], gpu=data["meta"]["gpu"], rows=rows)
dst = Path(__file__).resolve().parent / "decode_partition_t4.json"
dst.write_text(json.dumps(out, indent=1) + "\n")
print(f"wrote {len(rows)} rows to {dst}")
