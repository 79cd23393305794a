"""The matrix runner (``python -m small_q_attention_amd.matrix``), the drop-in for the
reference's ``scripts/run_gpu_matrix.py``: two small cases end to end, the JSONL
row schema of ``run_gpu_matrix.py:108-175`` (plus this build's columns), and
``--check-correctness`` within the parity bar."""

import json
import sys

import pytest

from small_q_attention_amd import matrix

pytestmark = pytest.mark.gpu

REFERENCE_KEYS = {"variant", "page_mode", "case", "status", "device", "p50_us", "p99_us",
                  "min_us", "max_us"}
CHECK_KEYS = {"max_abs_error", "max_rel_error"}
OWN_KEYS = {"kernel_p50_us", "merge_p50_us", "b2b_us", "kv_bytes", "kv_GBps", "pct_peak",
            "num_splits", "pages_per_split", "pools", "mall_resident", "within_tolerance"}


def test_runner_rows_and_correctness(tmp_path):
    out = tmp_path / "rows.jsonl"
    sys.__stderr__.write("\n[gpu-test] matrix runner: 2 cases x 2 variants\n")
    rc = matrix.main(["--variants", "auto", "v3", "--page-mode", "random", "--q-lens", "2",
                      "--kv-lens", "1024", "--batch-sizes", "1", "4", "--warmup", "1",
                      "--repeats", "3",
                      "--check-correctness", "--correctness-limit", "3", "--output", str(out)])
    assert rc == 0
    rows = [json.loads(line) for line in out.read_text().splitlines()]
    assert len(rows) == 4
    for row in rows:
        assert row["status"] == "ok", row
        assert REFERENCE_KEYS <= set(row) and OWN_KEYS - {"within_tolerance"} <= set(row)
        assert row["case"]["q_len"] == 2 and row["case"]["kv_len"] == 1024
        assert 0 < row["min_us"] <= row["p50_us"] <= row["max_us"]
        assert row["b2b_us"] > 0
        # A 4 MB (B1) or 16 MB (B4) KV set is rotated over pools totalling > 2 x the MALL.
        assert row["pools"] >= 3 and row["mall_resident"]
    checked = [r for r in rows if CHECK_KEYS <= set(r)]
    assert len(checked) == 3  # --correctness-limit
    for row in checked:
        assert row["within_tolerance"], row
        assert row["max_abs_error"] <= 2e-3 + 1e-2 * 4.0


def test_runner_defaults_run(tmp_path):
    """The reference runner's defaults (variants v0 v1, shared pages, chunk_keys 512)
    on one small case: rows carry the integer chunk size and the page mode."""
    out = tmp_path / "rows.jsonl"
    sys.__stderr__.write("\n[gpu-test] matrix runner: defaults, 1 case x 2 variants\n")
    rc = matrix.main(["--q-lens", "2", "--kv-lens", "1024", "--batch-sizes", "1",
                      "--warmup", "1", "--repeats", "3", "--output", str(out)])
    assert rc == 0
    rows = [json.loads(line) for line in out.read_text().splitlines()]
    assert [r["variant"] for r in rows] == ["v0", "v1"]
    for row in rows:
        assert row["status"] == "ok", row
        assert row["page_mode"] == "shared" and row["chunk_keys"] == 512
