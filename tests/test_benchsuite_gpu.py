"""The comparison suite end to end on the GPU, at its quick sizes: the rows
each section emits, their accuracy column, and the report rendered from them."""
import json

import pytest

from conftest import TOL

pytestmark = pytest.mark.gpu


def test_quick_sections_emit_rows_and_render(tmp_path):
    from attnkernels import benchsuite, report

    out = tmp_path / "suite.json"
    assert benchsuite.main(["--quick", "--sections", "input_activity", "ragged", "--out", str(out)]) == 0
    data = json.loads(out.read_text())
    assert not data["meta"].get("failed_cases"), data["meta"].get("failed_cases")
    rows = data["results"]

    act = [r for r in rows if r["section"] == "input_activity"]
    # every pattern for every workload: two prefill shapes and the GEMM
    assert {r["data"] for r in act} == set(benchsuite.ACTIVITY)
    assert len(act) == 3 * len(benchsuite.ACTIVITY)
    for r in act:
        assert r["tflops"] > 0 and r["ms"] > 0
        if r["impl"] == "flash_attention":
            assert r["max_abs_err"] < TOL[r["head_dim"]], r

    rag = [r for r in rows if r["section"] == "ragged"]
    assert {r["impl"] for r in rag} == {"paged_split", "paged_nosplit", "torch_gather_sdpa"}
    for r in rag:
        assert r["gbs"] > 0 and r["max_abs_err"] < TOL[128], r

    md = report.render(data)
    assert "## Rate against input bit activity" in md and "## Ragged batch" in md
