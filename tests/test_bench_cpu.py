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
    assert bench.profile_path("cfg1", 2, "fp16").exists()
    assert bench.profile_path("cfg2", 4, "fp16").exists()


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


def test_profiled_times_parser(tmp_path):
    p = tmp_path / "sqa_partial_kernel_cfg2.txt"
    p.write_text("# rocprofv3 summary\nkernel | calls | avg_us\n"
                 "partial_kernel_timed_steps_avg_us: 26.79 (last 20 dispatches)\n"
                 "merge_kernel_timed_steps_avg_us: 4.52 (last 20 dispatches)\n")
    # A path outside the repository is reported as given.
    import bench as b

    old = b.ROOT
    b.ROOT = tmp_path
    try:
        got = b._profiled_times(p)
    finally:
        b.ROOT = old
    assert got == {"partial_us": 26.79, "merge_us": 4.52, "source": p.name}
    assert bench._profiled_times(tmp_path / "missing.txt") is None


class _Case:
    def __init__(self, seed):
        self.seed = seed


class _Inputs:
    def __init__(self):
        self.seeds = []

    def make_inputs(self, case, device, gen_device):
        self.seeds.append(case.seed)
        return ("set", case.seed)


def test_small_workloads_rotate_over_enough_pools():
    """KV sets under 512 MB are timed over >= 3 distinct pools totalling more than
    512 MB (cfg1: 4 MB -> 129 pools; cfg2: 134 MB -> 5); large ones use one."""
    for kv, want in ((4 << 20, 129), (134217728, 5), (600 << 20, 1), (2147483648, 1)):
        fake = _Inputs()
        sets = bench.input_sets(fake, _Case(7), kv)
        assert len(sets) == want
        assert len(set(fake.seeds)) == want  # distinct seeds, distinct pools
        if want > 1:
            assert want >= 3 and want * kv > bench.ROTATE_BELOW_BYTES


def test_metric_grid_covers_the_baseline_metric():
    """The grid is BASELINE's metric: q_len 2/4/8 x KV 8K/32K x batch 1/4/16 (18 points)."""
    import json

    metric = json.loads((ROOT / "BASELINE.json").read_text())["metric"]
    assert bench.METRIC == metric
    assert bench.GRID_Q_LENS == (2, 4, 8) and "q_len 2/4/8" in metric
    assert bench.GRID_KV_LENS == (8192, 32768) and "KV 8K/32K" in metric
    assert bench.GRID_BATCHES == (1, 4, 16) and "batch 1/4/16" in metric
