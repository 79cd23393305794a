"""``rocprof_summary.py`` on synthetic rocprofv3 CSVs: kernel names shortened,
byte counters calibrated by the 1 GiB copy, the bench's timed dispatches (the
last ``--steps`` of each kernel) averaged, and the lines bench.py reads back."""

import csv

import rocprof_summary

PARTIAL = ("void sqa::(anonymous namespace)::sqa_partial_kernel<2, 4, 4, 1, 128, "
           "sqa::(anonymous namespace)::ElemF16, sqa::(anonymous namespace)::KvNative<128>, 1>"
           "(sqa::PartialArgs)")
MERGE = "void sqa::(anonymous namespace)::sqa_merge_kernel<64, 128, sqa::(anonymous namespace)::ElemF16>(sqa::MergeArgs)"
PROBE = "(anonymous namespace)::sqa_read_probe_kernel(unsigned int const*, unsigned long, unsigned int*)"
COPY = "__amd_rocclr_copyBuffer"


def _write(path, header, rows):
    path.parent.mkdir(parents=True, exist_ok=True)
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)


def test_summary_of_synthetic_profiles(tmp_path):
    trace = tmp_path / "trace" / "x"
    _write(trace / "t_kernel_stats.csv", ["Name", "Calls", "AverageNs", "MinNs", "MaxNs"],
           [[PARTIAL, 4, 300000, 290000, 330000], [MERGE, 4, 5000, 4000, 6000],
            [PROBE, 2, 290000, 289000, 291000]])
    # Partial dispatches: two warmup ones first, then the two timed steps.
    trace_rows = []
    for i, dur in enumerate([330000, 310000, 290000, 270000]):
        trace_rows.append([PARTIAL, 1000 * i, 1000 * i + dur])
        trace_rows.append([MERGE, 1000 * i + 500, 1000 * i + 500 + 5000])
    _write(trace / "t_kernel_trace.csv", ["Kernel_Name", "Start_Timestamp", "End_Timestamp"],
           trace_rows)
    for kind, counter, copy_kib, part_kib in (("fetch", "FETCH_SIZE", 524288.0, 1048576.0),
                                              ("write", "WRITE_SIZE", 1048576.0, 8192.0)):
        _write(tmp_path / kind / "c_counter_collection.csv",
               ["Kernel_Name", "Counter_Name", "Counter_Value", "Grid_Size"],
               [[COPY, counter, copy_kib, 1 << 20], [PARTIAL, counter, part_kib, 65536],
                [PARTIAL, counter, part_kib, 65536]])
    out = tmp_path / "summary.txt"
    rocprof_summary.main(["--trace", str(tmp_path / "trace"), "--fetch", str(tmp_path / "fetch"),
                          "--write", str(tmp_path / "write"), "--kv-bytes", str(1 << 31),
                          "--steps", "2", "--workload", "synthetic", "--command", "cmd",
                          "--out", str(out)])
    text = out.read_text()
    fields = {ln.split(":", 1)[0]: ln.split(":", 1)[1].split()[0] for ln in text.splitlines()
              if ":" in ln and "|" not in ln and not ln.startswith("#")}
    # The copy reads 1 GiB and writes 1 GiB: 2**30 / (KiB * 1024) per counter.
    assert float(fields["fetch_scale"]) == 2.0 and float(fields["write_scale"]) == 1.0
    assert float(fields["partial_kernel_avg_us"]) == 300.0
    assert float(fields["partial_kernel_timed_steps_avg_us"]) == 280.0  # last two dispatches
    assert float(fields["merge_kernel_timed_steps_avg_us"]) == 5.0
    assert int(fields["traffic_bytes_per_launch"]) == 2 * 1048576 * 1024 + 8192 * 1024
    rows = [ln for ln in text.splitlines() if " | " in ln]
    names = [r.split(" | ")[0] for r in rows[1:]]
    assert "sqa_read_probe_kernel" in names
    assert any(n.startswith("sqa_partial_kernel<2, 4, 4, 1, 128, ElemF16") for n in names)
