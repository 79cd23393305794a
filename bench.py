"""Benchmark of the paged small-q attention op on one MI355X.

One step = one call of the op over one batch (inputs resident in HBM). The
workload is cfg3 (B16, q_len 8, KV 32768, Hq/Hkv 32/8, d 128,
page 16, 1% of K scaled x4, random page table over a 2x pool): the shape the
70%-of-peak target is stated for (KV = 32K, batch 16) and the largest single-GPU
config; its 2.15 GB of KV cannot sit in the 256 MB MALL, so the figure is HBM.

Prints ONE JSON line (the driver's contract). ``value`` is KV GB/s of the whole
call (KV bytes / mean call time); ``roofline`` uses the partial kernel's own
mean duration from HIP events the library records around it on the launch
stream; ``cpu_baseline`` times the loop-faithful CPU oracle on a bounded
sample of the same workload. ``per_q_len`` repeats the timing at q_len 2, 4
and 16 on the same KV pool. ``metric_grid`` times back-to-back whole calls at
every point of BASELINE's metric (q_len 2/4/8 x KV 8K/32K x batch 1/4/16), and
each point's p50 per synchronised Python call (the reference runner's method);
``other_configs`` the other single-GPU configs (cfg1, cfg2, cfg5), with the
committed rocprof figures beside this run's under ``rocprof_*`` keys. ``roofline.read_probe`` is the practical read
ceiling: the streaming-read probe (``read_probe.hip``) over ~2 GiB of the same
resident pool (``frac_of_read_probe`` = the partial kernel's rate over it).
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_HBM_GBPS = 8000.0  # MI355X HBM3E, AMD published peak
# KV sets smaller than this are timed over several distinct pools in turn, so
# repeats cannot be served from the 256 MB MALL (Infinity Cache).
ROTATE_BELOW_BYTES = 512 << 20


# rocprofv3 FETCH_SIZE + WRITE_SIZE summary of the partial kernel on this workload
# (calibrated against a plain 1 GiB copy); regenerated with the kernel. The bench
# line's is profiles/sqa_partial_kernel_cfg3_b16_q8_kv32768.txt.
def profile_path(config: str, q_len: int, kv_dtype: str, batch: int = 0, kv_len: int = 0) -> Path:
    if batch and kv_len:  # a uniform grid point (--batch / --kv-len)
        shape = f"b{batch}_q{q_len}_kv{kv_len}"
    else:
        shape = {"cfg1": f"cfg1_b1_q{q_len}_kv1024", "cfg2": f"cfg2_b4_q{q_len}_kv8192",
                 "cfg3": f"cfg3_b16_q{q_len}_kv32768", "cfg5": f"cfg5_b16_q{q_len}_ragged"}[config]
    suffix = "" if kv_dtype == "fp16" else f"_{kv_dtype}"
    return ROOT / "profiles" / f"sqa_partial_kernel_{shape}{suffix}.txt"


def _profile_fields(path: Path):
    """``key: value`` lines of a committed rocprof summary (first token of the value)."""
    out = {}
    try:
        for line in path.read_text().splitlines():
            if ":" in line and not line.startswith("#") and "|" not in line:
                key, val = line.split(":", 1)
                if val.split():
                    out[key.strip()] = val.split()[0]
    except OSError:
        pass
    return out


def _profiled_traffic(path: Path):
    """HBM bytes per partial-kernel launch from a committed counter summary, or None."""
    val = _profile_fields(path).get("traffic_bytes_per_launch")
    return int(float(val)) if val is not None else None


def _profiled_times(path: Path):
    """Partial and merge kernel durations (us, the bench's timed steps) from a committed
    rocprof summary, or None."""
    f = _profile_fields(path)
    if "partial_kernel_timed_steps_avg_us" not in f:
        return None
    out = {"partial_us": float(f["partial_kernel_timed_steps_avg_us"]),
           "source": str(path.relative_to(ROOT))}
    if "merge_kernel_timed_steps_avg_us" in f:
        out["merge_us"] = float(f["merge_kernel_timed_steps_avg_us"])
    return out
METRIC = "µs/call + achieved HBM GB/s (% peak), q_len 2/4/8, KV 8K/32K, batch 1/4/16"


def _parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="target CPU-baseline sample duration")
    ap.add_argument("--no-per-q", action="store_true", help="skip the q_len 2/4/16 extras")
    ap.add_argument("--q-len", type=int, default=0,
                    help="override the workload's q_len (profiling other rows per kv head)")
    ap.add_argument("--config", default="cfg3", choices=("cfg1", "cfg2", "cfg3", "cfg5"),
                    help="workload (cfg3 is the bench line; others for profiling)")
    ap.add_argument("--batch", type=int, default=0,
                    help="with --kv-len: time a uniform batch of this many sequences instead "
                         "of the config (profiling a metric-grid point)")
    ap.add_argument("--kv-len", type=int, default=0, help="keys per sequence (with --batch)")
    ap.add_argument("--kv-dtype", default="fp16", choices=("fp16", "bf16", "e4m3"),
                    help="element types of the timed workload (profiling the other kernels): "
                         "bf16 = bf16 Q/K/V/output, e4m3 = fp16 Q/output over an OCP e4m3 "
                         "cache; fp16 (the bench line) also reports both as extras")
    ap.add_argument("--grid-only", action="store_true",
                    help="print only the metric grid (q_len 2/4/8 x KV 8K/32K x batch 1/4/16)")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="first run 3 plain device copies of this many MiB (counter calibration)")
    return ap.parse_args()


def _events(torch, n):
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
    for e in evs:
        e.record()  # creates the underlying hipEvent_t
    torch.cuda.synchronize()
    return evs


def _caller(torch, lib, tensors):
    """The C entry for these tensors: ``sqa_paged_mtp_attention`` for fp16 Q/K/V, the
    general entry (``sqa_paged_attention``) for bf16 or e4m3 caches. Returns
    ``call(out, ws, num_splits, pages_per_split, stream, timing_events=None)``."""
    q, k, v, bt, sl = tensors
    if q.dtype == torch.float16 and k.dtype == torch.float16:
        def call(out, ws, ns, pps, handle, timing_events=None):
            lib.launch(q, k, v, bt, sl, out, ws, ns, pps, handle, timing_events=timing_events)
    else:
        scale = q.shape[-1] ** -0.5

        def call(out, ws, ns, pps, handle, timing_events=None):
            lib.launch_general(q, out, k, v, bt, sl, None, scale, 1.0, ns, pps, ws, handle,
                               timing_events=timing_events)
    return call


def input_sets(inputs, case, kv_bytes):
    """The workload's inputs on the device: one set, or, when its KV bytes are under
    ``ROTATE_BELOW_BYTES``, enough distinct sets (other seeds, at least 3) that together
    they exceed it; the timed calls cycle through them so no call finds its pages in
    the MALL from the call before."""
    import copy

    n = 1 if kv_bytes >= ROTATE_BELOW_BYTES else max(3, -(-ROTATE_BELOW_BYTES // kv_bytes) + 1)
    sets = []
    for i in range(n):
        c = copy.copy(case)
        c.seed = case.seed + 7919 * i
        sets.append(inputs.make_inputs(c, device="cuda", gen_device="cuda"))
    return sets


def time_calls(torch, lib, sets, plan, steps, warmup, kernel_events=True):
    """Time `steps` calls through the C ABI with a preallocated workspace, cycling
    through the input sets (see :func:`input_sets`).

    Two passes of `steps` calls: the first, bracketed by synchronisations with
    nothing inside it but the calls, gives the ms per call; the second records
    the library's timing events around each kernel (events between the
    kernels add a little time per call, so they stay out of the first pass and
    make the per-kernel figures upper bounds). Returns (ms per call, mean
    partial-kernel ms, mean merge-kernel ms, output of set 0); without
    `kernel_events` the second pass is skipped and the kernel figures are None.
    """
    q, k = sets[0][0], sets[0][1]
    num_splits, pps = plan
    outs = [torch.empty_like(t[0]) for t in sets]
    nbytes = lib.workspace_bytes(q.shape[0], q.shape[1], q.shape[2], k.shape[2], q.shape[3],
                                 num_splits, pps)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
    stream = torch.cuda.current_stream()
    handle = stream.cuda_stream
    calls = [_caller(torch, lib, t) for t in sets]
    n = len(sets)
    for i in range(max(warmup, n)):
        calls[i % n](outs[i % n], ws, num_splits, pps, handle)
    kev = _events(torch, 3 * steps)
    start, end = _events(torch, 2)
    torch.cuda.synchronize()
    start.record(stream)
    for i in range(steps):
        calls[i % n](outs[i % n], ws, num_splits, pps, handle)
    end.record(stream)
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(end)
    if not kernel_events:
        return total_ms / steps, None, None, outs[0]
    for i in range(steps):
        calls[i % n](outs[i % n], ws, num_splits, pps, handle,
                     timing_events=[e.cuda_event for e in kev[3 * i:3 * i + 3]])
    torch.cuda.synchronize()
    part = [kev[3 * i].elapsed_time(kev[3 * i + 1]) for i in range(steps)]
    merge = [kev[3 * i + 1].elapsed_time(kev[3 * i + 2]) for i in range(steps)]
    return total_ms / steps, statistics.mean(part), statistics.mean(merge), outs[0]


def p50_call_us(torch, sets, max_seq_len, warmup=5, repeats=15):
    """The reference runner's per-call latency (``run_gpu_matrix.py:63-81``): HIP events
    around each call of the Python entry, synchronised after each, warmup 5, repeats
    15, p50 in us. The call is ``paged_mtp_attention`` (the native entry: automatic
    plan, known ``max_seq_len``), so it includes the host-side checks, the output
    allocation and both launches, with the GPU idle before each call; it cycles
    through the same pools as the back-to-back timing."""
    from small_q_attention_amd import cuda as sqa

    n = len(sets)
    for i in range(warmup):
        sqa.paged_mtp_attention(*sets[i % n], 16, max_seq_len)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    samples = []
    for i in range(repeats):
        start.record()
        sqa.paged_mtp_attention(*sets[i % n], 16, max_seq_len)
        end.record()
        end.synchronize()
        samples.append(start.elapsed_time(end) * 1e3)
    return statistics.median(samples)


GRID_Q_LENS = (2, 4, 8)
GRID_KV_LENS = (8192, 32768)
GRID_BATCHES = (1, 4, 16)


def metric_grid(torch, lib, inputs, steps, warmup):
    """BASELINE's metric over its whole grid: q_len 2/4/8 x KV 8K/32K x batch 1/4/16
    (Hq/Hkv 32/8, d 128, page 16, fp16, random page tables over a 2x pool), each
    point the mean of back-to-back whole calls (partial + merge) through the C ABI
    with the automatic plan for a known max_seq_len (``us_per_call``), and the p50 of
    single synchronised calls through the Python entry, as the reference runner
    times them (``p50_call_us``, :func:`p50_call_us`); KV sets under
    ``ROTATE_BELOW_BYTES`` rotate over several pools (:func:`input_sets`). The
    pools of one (KV, batch) serve all three q_len (Q drawn per q_len)."""
    grid = {}
    for kv in GRID_KV_LENS:
        for b in GRID_BATCHES:
            case = inputs.uniform_case(b, max(GRID_Q_LENS), kv, seed=4000 + kv // 1024 + b)
            kvb = inputs.kv_bytes(case.seq_lens, case.num_kv_heads, case.head_dim)
            sets = input_sets(inputs, case, kvb)
            # At least 400 calls below 512 MB of KV (6-12 ms: a run of 100 such
            # calls varied by up to 10% from run to run on one box), 50 up to
            # 2 GB (~4-5 ms).
            n_steps = max(steps, 400 if kvb < ROTATE_BELOW_BYTES else
                          (50 if kvb < (2 << 30) else steps))
            for ql in GRID_Q_LENS:
                qsets = []
                for i, (q, k, v, bt, sl) in enumerate(sets):
                    g = torch.Generator(device="cuda").manual_seed(4100 + 10 * ql + i)
                    qx = torch.randn(b, ql, q.shape[2], q.shape[3], generator=g, device="cuda",
                                     dtype=torch.float16)
                    qsets.append((qx, k, v, bt, sl))
                plan = lib.plan_splits(0, b, ql, case.num_query_heads, case.num_kv_heads,
                                       case.head_dim, kv, sets[0][3].shape[1], 0)
                _ramp_clocks(torch, lib, qsets[0], plan, seconds=0.1)
                ms, _, _, out = time_calls(torch, lib, qsets, plan, n_steps, warmup,
                                           kernel_events=False)
                if not torch.isfinite(out).all():
                    raise SystemExit(f"non-finite output at q{ql} KV{kv} B{b}")
                gbps = kvb / (ms * 1e-3) / 1e9
                grid[f"q{ql}_kv{kv}_b{b}"] = {
                    "us_per_call": round(ms * 1e3, 2), "kv_GBps": round(gbps, 1),
                    "pct_peak": round(100.0 * gbps / PEAK_HBM_GBPS, 2), "kv_bytes": kvb,
                    "pools": len(sets), "steps": n_steps, "num_splits": plan[0],
                    "pages_per_split": plan[1],
                    "p50_call_us": round(p50_call_us(torch, qsets, kv), 2)}
                del qsets
            del sets
            torch.cuda.empty_cache()
    return grid


def read_probe(torch, lib, pool, steps):
    """The practical HBM read ceiling: ``sqa_read_probe`` of ``read_probe.hip`` (one
    workgroup per CU, contiguous chunks, 16-byte non-temporal loads) over the first
    ~2 GiB of the resident K pool, `steps` passes between two events. Returns (GB/s,
    bytes, us)."""
    import read_probe as probe

    probe_lib = probe.load(build_if_missing=False)
    blocks = lib.load().sqa_device_cu_count(0)
    flat = pool.view(-1).view(torch.uint8)
    unit = 16 * 256 * blocks
    nbytes = min(flat.numel(), 1 << 31) // unit * unit
    data = flat[:nbytes]
    sink = torch.empty(blocks * 256, dtype=torch.int32, device=pool.device)
    handle = torch.cuda.current_stream().cuda_stream
    for _ in range(3):
        probe.read_probe(data, sink, blocks, handle, probe_lib)
    start, end = _events(torch, 2)
    start.record()
    for _ in range(steps):
        probe.read_probe(data, sink, blocks, handle, probe_lib)
    end.record()
    torch.cuda.synchronize()
    us = start.elapsed_time(end) * 1e3 / steps
    return nbytes / (us * 1e-6) / 1e9, nbytes, us


def _ramp_clocks(torch, lib, tensors, plan, seconds=0.25):
    """Setup, not a step: run the op for ~0.25 s so GPU clocks settle before the
    warmup steps (the first calls of a process otherwise run up to ~10% slow)."""
    q, k = tensors[0], tensors[1]
    out = torch.empty_like(q)
    nbytes = lib.workspace_bytes(q.shape[0], q.shape[1], q.shape[2], k.shape[2], q.shape[3],
                                 plan[0], plan[1])
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
    handle = torch.cuda.current_stream().cuda_stream
    call = _caller(torch, lib, tensors)
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(20):
            call(out, ws, plan[0], plan[1], handle)
        torch.cuda.synchronize()


def cpu_baseline(torch, tensors, case, target_s):
    """Loop-faithful CPU oracle on whole sequences of the workload until ~target_s."""
    import oracle

    q, k, v, bt, sl = tensors
    page = case.page_size
    done, elapsed, kv_done = 0, 0.0, 0
    while done < case.batch and (elapsed < target_s or done == 0):
        b = done
        n = -(-int(case.seq_lens[b]) // page)
        ids = bt[b, :n].long()
        kc = k.index_select(0, ids).float().cpu()
        vc = v.index_select(0, ids).float().cpu()
        qc = q[b:b + 1].float().cpu()
        btc = torch.arange(n, dtype=torch.int32).unsqueeze(0)
        slc = sl[b:b + 1].cpu()
        t0 = time.perf_counter()
        oracle.paged_mtp_attention_reference(qc, kc, vc, btc, slc, page, case.num_kv_heads)
        elapsed += time.perf_counter() - t0
        kv_done += int(case.seq_lens[b]) * case.num_kv_heads * case.head_dim * 4
        done += 1
    per_seq_s = elapsed / done
    # cfg1 (B1 q_len2 KV1024, the reference's CPU-runnable case) in full, best of 3.
    from small_q_attention_amd import inputs

    c1 = inputs.baseline_configs()["cfg1"]
    q1, k1, v1, bt1, sl1 = inputs.make_inputs(c1)
    q1, k1, v1 = q1.float(), k1.float(), v1.float()
    cfg1_s = []
    for _ in range(3):
        t0 = time.perf_counter()
        oracle.paged_mtp_attention_reference(q1, k1, v1, bt1, sl1, c1.page_size, c1.num_kv_heads)
        cfg1_s.append(time.perf_counter() - t0)
    return {
        "value": round(kv_done / elapsed / 1e9, 4),
        "unit": "GB/s (KV bytes / CPU time)",
        "us_per_call": round(per_seq_s * case.batch * 1e6, 1),
        "cores": int(torch.get_num_threads()),
        "kind": "port",
        "sample": (f"{done} of {case.batch} sequences of the workload (full KV length "
                   f"{case.seq_lens[0]}, all {case.num_query_heads} heads), fp32 on .float() "
                   f"copies; us_per_call extrapolates to the whole batch"),
        "cfg1_us_per_call": round(min(cfg1_s) * 1e6, 1),
        "cpu_model": _cpu_model(),
        "os_cpu_count": os.cpu_count(),
    }


def _describe(name, case):
    lens = set(case.seq_lens)
    kv = (f"KV{case.seq_lens[0]}" if len(lens) == 1
          else f"ragged KV {min(lens)}..{max(lens)} (sum {sum(case.seq_lens)})")
    extra = (f", K x{case.k_outlier_scale:g} on {100 * case.k_outlier_frac:g}% of slots"
             if case.k_outlier_frac else "")
    return (f"{name}: B{case.batch} q_len{case.q_len} {kv} Hq/Hkv{case.num_query_heads}/"
            f"{case.num_kv_heads} d{case.head_dim} page{case.page_size}{extra}, "
            f"{case.page_mode} page table over a {case.pool_factor}x pool")


def _cpu_model():
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    args = _parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); this build has no "
              "multi-GPU path. Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch

    from small_q_attention_amd import _lib, inputs

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)
    torch.cuda.set_device(0)
    lib = _lib.load(build_if_missing=False)
    if args.copy_probe_mib > 0:
        # A plain copy kernel of known size: its FETCH_SIZE / WRITE_SIZE counters
        # calibrate the per-dispatch byte counts of the attention kernels.
        n = args.copy_probe_mib << 20
        src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if args.grid_only:
        print(json.dumps({"metric": METRIC, "metric_grid": metric_grid(
            torch, _lib, inputs, args.steps, args.warmup)}), flush=True)
        return
    case = inputs.baseline_configs()[args.config]
    if args.batch and args.kv_len:
        case = inputs.uniform_case(args.batch, args.q_len or 8, args.kv_len,
                                   seed=4000 + args.kv_len // 1024 + args.batch)
        args.config = f"b{args.batch}_kv{args.kv_len}"
    if args.q_len:
        case.q_len = args.q_len
    kvb16 = inputs.kv_bytes(case.seq_lens, case.num_kv_heads, case.head_dim)
    sets = []
    for q, k, v, bt, sl in input_sets(inputs, case, kvb16):
        if args.kv_dtype == "bf16":
            q, k, v = q.bfloat16(), k.bfloat16(), v.bfloat16()
        elif args.kv_dtype == "e4m3":
            k, v = k.to(torch.float8_e4m3fn), v.to(torch.float8_e4m3fn)
        sets.append((q, k, v, bt, sl))
    tensors = sets[0]
    q, k, v, bt, sl = tensors
    default_types = args.kv_dtype == "fp16"
    plan = _lib.plan_splits(0, case.batch, case.q_len, case.num_query_heads, case.num_kv_heads,
                            case.head_dim, case.max_seq_len, bt.shape[1], 0)
    _ramp_clocks(torch, _lib, tensors, plan)
    ms, part_ms, merge_ms, out = time_calls(torch, _lib, sets, plan, args.steps, args.warmup)
    if not torch.isfinite(out).all():
        raise SystemExit("non-finite output")
    prof = profile_path(args.config, case.q_len, args.kv_dtype, args.batch, args.kv_len)
    kvb = kvb16 * k.element_size() // 2
    value = kvb / (ms * 1e-3) / 1e9
    achieved = kvb / (part_ms * 1e-3) / 1e9
    result = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "us_per_call": round(ms * 1e3, 2),
        "pct_peak": round(100.0 * value / PEAK_HBM_GBPS, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"fp16": "fp16 in/out, fp32 accumulate",
                  "bf16": "bf16 in/out, fp32 accumulate",
                  "e4m3": "fp16 Q/out over an OCP e4m3 KV cache, fp32 accumulate"}[args.kv_dtype],
        "data": "synthetic: N(0,1) fp16 Q/K/V drawn on the device, seeded"
                + ("" if default_types else f", converted to {args.kv_dtype}"),
        "config": {
            "workload": _describe(args.config, case) + ("" if default_types else
                                                         f", {args.kv_dtype} K/V"),
            "batch": case.batch, "q_len": case.q_len,
            "kv_len": case.seq_lens[0] if len(set(case.seq_lens)) == 1 else "ragged",
            "num_splits": plan[0], "pages_per_split": plan[1],
            "kv_bytes": kvb, "alg_bytes": inputs.alg_bytes(case),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBPS, 4),
            "traffic": _profiled_traffic(prof),
            "traffic_source": str(prof.relative_to(ROOT)),
            "kernel": "sqa_partial_kernel",
            "kernel_us": round(part_ms * 1e3, 2),
            "merge_us": round(merge_ms * 1e3, 2),
        },
    }
    probe_gbps, probe_bytes, probe_us = read_probe(torch, _lib, k, args.steps)
    result["roofline"]["read_probe"] = {
        "GBps": round(probe_gbps, 1), "bytes": probe_bytes, "us": round(probe_us, 2),
        "frac_of_peak": round(probe_gbps / PEAK_HBM_GBPS, 4)}
    result["roofline"]["frac_of_read_probe"] = round(achieved / probe_gbps, 4)
    if not args.no_per_q and default_types:
        extra = {}
        for ql in (2, 4, 16):
            g = torch.Generator(device="cuda").manual_seed(100 + ql)
            qx = torch.randn(case.batch, ql, case.num_query_heads, case.head_dim,
                             generator=g, device="cuda", dtype=torch.float16)
            planx = _lib.plan_splits(0, case.batch, ql, case.num_query_heads, case.num_kv_heads,
                                     case.head_dim, case.max_seq_len, bt.shape[1], 0)
            msx, px, mx, _ = time_calls(torch, _lib, [(qx, k, v, bt, sl)], planx, args.steps,
                                        args.warmup)
            extra[f"q{ql}"] = {"us_per_call": round(msx * 1e3, 2),
                               "kv_GBps": round(kvb / (msx * 1e-3) / 1e9, 1),
                               "kernel_us": round(px * 1e3, 2),
                               "kernel_frac": round(kvb / (px * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4)}
        result["per_q_len"] = extra
        # The same workload with bf16 Q/K/V (general entry point).
        qb, kb, vb = q.bfloat16(), k.bfloat16(), v.bfloat16()
        outb = torch.empty_like(qb)
        nbytes = _lib.workspace_bytes(case.batch, case.q_len, case.num_query_heads,
                                      case.num_kv_heads, case.head_dim, plan[0], plan[1])
        wsb = torch.empty(max(nbytes, 1), dtype=torch.uint8, device="cuda")
        handle = torch.cuda.current_stream().cuda_stream

        def bf16_call(ev=None):
            _lib.launch_general(qb, outb, kb, vb, bt, sl, None, case.head_dim ** -0.5, 1.0,
                                plan[0], plan[1], wsb, handle, timing_events=ev)

        t0 = time.perf_counter()
        while time.perf_counter() - t0 < 0.1:  # settle clocks on the new kernel
            bf16_call()
            torch.cuda.synchronize()
        for _ in range(args.warmup):
            bf16_call()
        kev = _events(torch, 3 * args.steps)
        torch.cuda.synchronize()
        for i in range(args.steps):
            bf16_call([e.cuda_event for e in kev[3 * i:3 * i + 3]])
        torch.cuda.synchronize()
        pb = statistics.mean(kev[3 * i].elapsed_time(kev[3 * i + 1]) for i in range(args.steps))
        result["bf16"] = {"kernel_us": round(pb * 1e3, 2),
                          "kernel_frac": round(kvb / (pb * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4)}
        del qb, kb, vb, outb, wsb
        # fp16 queries over an OCP e4m3 cache of the same shape (half the KV bytes):
        # the workload's q_len, and q_len 16 (64 rows per kv head, the
        # compute-heaviest e4m3 kernel).
        k8, v8 = k.to(torch.float8_e4m3fn), v.to(torch.float8_e4m3fn)

        def fp8_kernel_ms(qx):
            plan8 = _lib.plan_splits(0, case.batch, qx.shape[1], case.num_query_heads,
                                     case.num_kv_heads, case.head_dim, case.max_seq_len,
                                     bt.shape[1], 0)
            n8 = _lib.workspace_bytes(case.batch, qx.shape[1], case.num_query_heads,
                                      case.num_kv_heads, case.head_dim, plan8[0], plan8[1])
            out8 = torch.empty_like(qx)
            ws8 = torch.empty(max(n8, 1), dtype=torch.uint8, device="cuda")

            def fp8_call(ev=None):
                _lib.launch_general(qx, out8, k8, v8, bt, sl, None, case.head_dim ** -0.5, 1.0,
                                    plan8[0], plan8[1], ws8, handle, timing_events=ev)

            t0 = time.perf_counter()
            while time.perf_counter() - t0 < 0.1:
                fp8_call()
                torch.cuda.synchronize()
            for _ in range(args.warmup):
                fp8_call()
            kev = _events(torch, 3 * args.steps)
            torch.cuda.synchronize()
            for i in range(args.steps):
                fp8_call([e.cuda_event for e in kev[3 * i:3 * i + 3]])
            torch.cuda.synchronize()
            return statistics.mean(kev[3 * i].elapsed_time(kev[3 * i + 1])
                                   for i in range(args.steps))

        p8 = fp8_kernel_ms(q)
        g16 = torch.Generator(device="cuda").manual_seed(case.seed + 16)
        q16 = torch.randn(case.batch, 16, case.num_query_heads, case.head_dim, generator=g16,
                          device="cuda", dtype=torch.float16)
        p16 = fp8_kernel_ms(q16)
        result["fp8_kv"] = {"kernel_us": round(p8 * 1e3, 2), "kv_bytes": kvb // 2,
                            "kernel_frac": round(kvb / 2 / (p8 * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4),
                            "speedup_vs_fp16_kv": round(part_ms / p8, 3),
                            "q16": {"kernel_us": round(p16 * 1e3, 2),
                                    "kernel_frac": round(kvb / 2 / (p16 * 1e-3) / 1e9 /
                                                         PEAK_HBM_GBPS, 4)}}
        del k8, v8, q16
    if not args.no_per_q and default_types:
        # The other single-GPU benchmark configs, same timing (extra fields only).
        others = {}
        del tensors, sets, q, k, v, bt, sl, out
        torch.cuda.empty_cache()
        for name in ("cfg1", "cfg2", "cfg5"):
            c = inputs.baseline_configs()[name]
            kb = inputs.kv_bytes(c.seq_lens, c.num_kv_heads, c.head_dim)
            ts = input_sets(inputs, c, kb)
            pl = _lib.plan_splits(0, c.batch, c.q_len, c.num_query_heads, c.num_kv_heads,
                                  c.head_dim, c.max_seq_len, ts[0][3].shape[1], 0)
            _ramp_clocks(torch, _lib, ts[0], pl, seconds=0.1)
            msx, px, mx, _ = time_calls(torch, _lib, ts, pl, args.steps, args.warmup)
            row = {"batch": c.batch, "q_len": c.q_len,
                   "kv_lens": "ragged" if name == "cfg5" else c.seq_lens[0], "kv_bytes": kb,
                   "pools": len(ts), "us_per_call": round(msx * 1e3, 2),
                   "call_kv_GBps": round(kb / (msx * 1e-3) / 1e9, 1),
                   # Upper bounds: the library's events between the kernels add time.
                   "partial_us_events": round(px * 1e3, 2), "merge_us_events": round(mx * 1e3, 2),
                   "num_splits": pl[0], "pages_per_split": pl[1]}
            # This run's figures: the whole call back to back, and the partial
            # kernel between the library's events.
            row["call_frac"] = round(kb / (msx * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4)
            row["kernel_frac_events"] = round(kb / (px * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4)
            # Not measured in this run: the committed rocprof summary of the same
            # workload (bench.py --config <name>), for comparison.
            prof_times = _profiled_times(profile_path(name, c.q_len, "fp16"))
            if prof_times is not None:
                row["rocprof_kernel_us"] = prof_times["partial_us"]
                row["rocprof_kernel_frac"] = round(
                    kb / (prof_times["partial_us"] * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4)
                if "merge_us" in prof_times:
                    row["rocprof_merge_us"] = prof_times["merge_us"]
                row["rocprof_source"] = prof_times["source"]
            others[name] = row
            del ts
            torch.cuda.empty_cache()
        result["other_configs"] = others
        result["metric_grid"] = metric_grid(torch, _lib, inputs, args.steps, args.warmup)
        tensors = inputs.make_inputs(case, device="cuda", gen_device="cuda")
    if not args.no_cpu_baseline and default_types:
        result["cpu_baseline"] = cpu_baseline(torch, tensors, case, args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
