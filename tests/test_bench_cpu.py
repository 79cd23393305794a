"""CPU checks of bench.py's bookkeeping (no GPU): the profile each workload's
traffic figure comes from, the traffic parser, and the one-GPU guard."""

import subprocess
import sys
from pathlib import Path

import bench

ROOT = Path(__file__).resolve().parents[1]


def test_profile_paths_name_committed_summaries():
    assert bench.profile_path("cfg3", 8, "fp16").name == "sqa_partial_kernel_cfg3_b16_q8_kv32768.txt"
    assert bench.profile_path("cfg3", 8, "e4m3").name.endswith("_kv32768_e4m3.txt")
    assert bench.profile_path("cfg5", 8, "fp16").name == "sqa_partial_kernel_cfg5_b16_q8_ragged.txt"
    for path in (bench.profile_path("cfg3", q, "fp16") for q in (2, 4, 8, 16)):
        assert path.exists(), path
    assert bench.profile_path("cfg3", 8, "bf16").exists()
    assert bench.profile_path("cfg3", 8, "e4m3").exists()


def test_traffic_parser(tmp_path):
    p = tmp_path / "s.txt"
    p.write_text("fetch_scale: 2.0\ntraffic_bytes_per_launch: 2169519363\n")
    assert bench._profiled_traffic(p) == 2169519363
    assert bench._profiled_traffic(tmp_path / "missing.txt") is None
    # The bench line's summary holds a traffic figure close to the algorithmic bytes.
    t = bench._profiled_traffic(bench.profile_path("cfg3", 8, "fp16"))
    assert t is not None and 1.0 <= t / 2147483648 < 1.05


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "one GPU only" in r.stderr
