"""Matrix timing runner: the drop-in for the reference's ``scripts/run_gpu_matrix.py``.

    python -m small_q_attention_amd.matrix --variants v3 auto --q-lens 2 4 8 16 \\
        --kv-lens 1024 8192 32768 --batch-sizes 1 4 16 --page-mode random

Defaults are the reference runner's (variants v0 v1, shared pages, 512 keys per
split, q_len 2 4 8, KV 1024 8192, batch 1 4).

Same CLI names and JSONL row schema as ``run_gpu_matrix.py:108-175`` (``variant,
page_mode, case, status, device, p50_us, p99_us, min_us, max_us``), timed the
same way (events around the Python call, warmup then repeats,
``run_gpu_matrix.py:63-81``), with the memory-aware skip of ``:146-153``. Rows
are appended to ``--output`` as they complete. Added columns:

* ``kernel_p50_us`` / ``merge_p50_us``: partial and merge kernels alone, from
  HIP events the library records around them on the launch stream, timed
  after ~0.1 s of back-to-back calls (clocks settled);
* ``kv_bytes``, ``kv_GBps`` and ``pct_peak`` (KV bytes over ``kernel_p50_us``),
  ``call_GBps`` (over ``p50_us``), ``num_splits``, ``pages_per_split``;
* ``pools``: cases whose calls read less KV than twice the 256 MB MALL rotate
  through this many distinct pools (their reads together at least twice the
  MALL) so repeats do not read from the cache (``mall_resident`` says whether
  one call's KV alone would fit);
* ``b2b_us``: mean time per call over ``repeats`` calls issued back to back
  through the C ABI (events only around the batch of calls), rotating the
  pools: what a decode loop sees, without the per-call synchronisation of
  ``p50_us`` and without the inter-kernel events of ``kernel_p50_us``, which
  are upper bounds.

``--check-correctness`` (with ``--correctness-limit``, default 3 cases, as in
``run_gpu_matrix.py:126-127,159-169``) adds ``max_abs_error`` and
``max_rel_error`` of the call's output against the float32 checker
(:mod:`small_q_attention_amd.checker`) rounded to fp16, as the reference runner
compares with its CPU oracle rounded to fp16, plus ``within_tolerance``
(``|a - r| <= 2e-3 + 1e-2 |r|``). The full parity suite is ``tests/``.
"""

from __future__ import annotations

import argparse
import itertools
import json
import statistics
import sys
import time
from pathlib import Path

PEAK_HBM_GBPS = 8000.0
MALL_BYTES = 256 << 20
CONFIG = Path(__file__).resolve().parent / "configs" / "core_matrix.json"


def load_cases(path: Path = CONFIG):
    """The fixed case product (``/root/reference/scripts/validate_matrix.py:8-14``)."""
    config = json.loads(Path(path).read_text(encoding="utf-8"))
    keys = ("q_len", "kv_len", "batch_size")
    fixed = ("dtype", "head_dim", "page_size", "num_query_heads", "num_kv_heads")
    cases = []
    for values in itertools.product(*(config[k] for k in keys)):
        case = dict(zip(keys, values))
        case.update({k: config[k] for k in fixed})
        cases.append(case)
    return config, cases


def _percentile(values, fraction):
    values = sorted(values)
    return values[min(len(values) - 1, int(fraction * len(values)))]


def _resolve(variant, case, chunk_keys):
    from . import cuda as sqa

    ck = None if chunk_keys == "auto" else int(chunk_keys)
    kv = case["kv_len"]
    if variant == "v0":
        return sqa.forward_v0, None
    if variant == "v1":
        return sqa.forward_v1, None
    if variant == "v2":
        return (lambda *a, **k: sqa.forward_v2(*a, chunk_keys=ck, **k)), ck
    if variant in ("v3", "v4"):
        f = sqa.forward_v3 if variant == "v3" else sqa.forward_v4
        return (lambda *a, **k: f(*a, chunk_keys=ck, max_seq_len=kv, **k)), ck
    if variant == "v5":
        return (lambda *a, **k: sqa.forward_v5(*a, chunk_keys=ck, token_group=case["token_group"],
                                                max_seq_len=kv, **k)), ck
    # "auto": the native entry with the automatic (CU-count) plan.
    return (lambda *a, **k: sqa.paged_mtp_attention(*a, max_seq_len=kv)), None


def _events(torch, n):
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
    for e in evs:
        e.record()
    return evs


def check_case(torch, forward, tensors, page_size, num_kv_heads):
    """``max_abs_error`` / ``max_rel_error`` of one call against the float32 checker
    rounded to fp16 (``run_gpu_matrix.py:159-169``), and the parity bar."""
    from .checker import attention_fp32

    actual = forward(*tensors, page_size)
    ref = torch.from_numpy(attention_fp32(*tensors, page_size, num_kv_heads))
    ref = ref.to(device=actual.device, dtype=torch.float16).float()
    err = (actual.float() - ref).abs()
    return {"max_abs_error": err.max().item(),
            "max_rel_error": (err / ref.abs().clamp_min(1e-5)).max().item(),
            "within_tolerance": bool((err <= 2e-3 + 1e-2 * ref.abs()).all().item())}


def measure_case(torch, variant, case, page_mode, chunk_keys, warmup, repeats, seed,
                 max_pools=160, check=False):
    from . import _lib, inputs

    c = inputs.uniform_case(case["batch_size"], case["q_len"], case["kv_len"], page_mode=page_mode,
                            seed=seed)
    # KV bytes one call reads (its pool holds twice the pages); sets that read
    # less than twice the MALL rotate, so no call finds its pages cached by
    # the call before.
    read_bytes = inputs.kv_bytes(c.seq_lens, c.num_kv_heads, c.head_dim)
    pools = 1
    if read_bytes < 2 * MALL_BYTES:
        pools = min(max_pools, max(2, -(-2 * MALL_BYTES // read_bytes)))
    sets = []
    for i in range(pools):
        c.seed = seed + 7919 * i
        sets.append(inputs.make_inputs(c, device="cuda", gen_device="cuda"))
    forward, ck = _resolve(variant, case, chunk_keys)
    page = c.page_size
    for i in range(warmup):
        forward(*sets[i % pools], page)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    samples = []
    for i in range(repeats):
        t = sets[i % pools]
        start.record()
        forward(*t, page)
        end.record()
        end.synchronize()
        samples.append(start.elapsed_time(end) * 1000.0)
    # Kernel-only timing through the C ABI with the library's event hooks.
    q, k, v, bt, sl = sets[0]
    plan_ck = 0 if ck is None else ck
    max_seq = case["kv_len"] if variant not in ("v0", "v1") else 0
    ns, pps = _lib.plan_splits(0, c.batch, c.q_len, c.num_query_heads, c.num_kv_heads,
                               c.head_dim, max_seq, bt.shape[1], plan_ck)
    nbytes = _lib.workspace_bytes(c.batch, c.q_len, c.num_query_heads, c.num_kv_heads,
                                  c.head_dim, ns, pps)
    ws = torch.empty(max(1, nbytes), dtype=torch.uint8, device="cuda")
    outs = [torch.empty_like(s[0]) for s in sets]
    stream = torch.cuda.current_stream().cuda_stream
    evs = _events(torch, 3 * repeats)
    # The synchronised calls above leave the GPU idle between calls; ~0.1 s of
    # back-to-back calls first lets the clocks settle, as bench.py does.
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 0.1:
        for i in range(4):
            _lib.launch(*sets[i % pools], outs[i % pools], ws, ns, pps, stream)
        torch.cuda.synchronize()
    b0, b1 = _events(torch, 2)
    torch.cuda.synchronize()
    b0.record()
    for i in range(repeats):
        _lib.launch(*sets[i % pools], outs[i % pools], ws, ns, pps, stream)
    b1.record()
    torch.cuda.synchronize()
    b2b = b0.elapsed_time(b1) * 1000.0 / repeats
    for i in range(repeats):
        s = sets[i % pools]
        _lib.launch(*s, outs[i % pools], ws, ns, pps, stream,
                    timing_events=[e.cuda_event for e in evs[3 * i:3 * i + 3]])
    torch.cuda.synchronize()
    part = [evs[3 * i].elapsed_time(evs[3 * i + 1]) * 1e3 for i in range(repeats)]
    merge = [evs[3 * i + 1].elapsed_time(evs[3 * i + 2]) * 1e3 for i in range(repeats)]
    kvb = inputs.kv_bytes(c.seq_lens, c.num_kv_heads, c.head_dim)
    kern = statistics.median(part) + statistics.median(merge)
    p50 = statistics.median(samples)
    row = {
        "p50_us": p50, "p99_us": _percentile(samples, 0.99), "min_us": min(samples),
        "max_us": max(samples),
        "kernel_p50_us": statistics.median(part), "merge_p50_us": statistics.median(merge),
        "b2b_us": b2b, "b2b_kv_GBps": kvb / (b2b * 1e-6) / 1e9,
        "kv_bytes": kvb, "kv_GBps": kvb / (kern * 1e-6) / 1e9,
        "pct_peak": 100.0 * kvb / (kern * 1e-6) / 1e9 / PEAK_HBM_GBPS,
        "call_GBps": kvb / (p50 * 1e-6) / 1e9,
        "num_splits": ns, "pages_per_split": pps, "pools": pools,
        "mall_resident": read_bytes <= MALL_BYTES,
    }
    if check:
        row.update(check_case(torch, forward, sets[0], page, c.num_kv_heads))
    del sets
    return row


def _chunk_keys(text):
    """``--chunk-keys``: an integer, as the reference runner takes it, or ``auto``."""
    if text == "auto":
        return text
    try:
        return int(text)
    except ValueError:
        raise argparse.ArgumentTypeError(f"an integer or 'auto', not {text!r}") from None


def build_parser():
    """The runner's CLI. Defaults are the reference runner's
    (``/root/reference/scripts/run_gpu_matrix.py:111-127``: variants v0 v1, shared
    pages, 512 keys per split, q_len 2 4 8, KV 1024 8192, batch 1 4), so an
    invocation that relies on them measures the same workload; ``auto`` (the
    CU-count plan, as variant or chunk size) and ``random`` page tables are
    opt-ins."""
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--variants", nargs="+", default=["v0", "v1"],
                    choices=("v0", "v1", "v2", "v3", "v4", "v5", "auto"))
    ap.add_argument("--chunk-keys", type=_chunk_keys, default=512,
                    help="KV entries per split for v2-v5, or 'auto' (CU-count plan); "
                         "variant 'auto' always uses the CU-count plan")
    ap.add_argument("--token-group", type=int, choices=(2, 4), default=2)
    ap.add_argument("--page-mode", choices=("shared", "unique", "random"), default="shared")
    ap.add_argument("--q-lens", nargs="+", type=int, default=[2, 4, 8])
    ap.add_argument("--kv-lens", nargs="+", type=int, default=[1024, 8192])
    ap.add_argument("--batch-sizes", nargs="+", type=int, default=[1, 4])
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--repeats", type=int, default=15)
    ap.add_argument("--limit", type=int, default=0, help="cases per variant; 0 = all")
    ap.add_argument("--check-correctness", action="store_true",
                    help="add max_abs_error / max_rel_error against the float32 checker")
    ap.add_argument("--correctness-limit", type=int, default=3,
                    help="cases checked when --check-correctness is given")
    ap.add_argument("--output", type=Path, help="JSONL file rows are appended to")
    return ap


def main(argv=None):
    import torch

    args = build_parser().parse_args(argv)
    if not torch.cuda.is_available():
        raise SystemExit("a ROCm GPU is required")
    if args.warmup < 0 or args.repeats < 1:
        raise SystemExit("warmup must be non-negative and repeats positive")
    config, _ = load_cases()
    fixed = {k: config[k] for k in ("dtype", "head_dim", "page_size", "num_query_heads",
                                     "num_kv_heads")}
    cases = [dict(q_len=q, kv_len=kv, batch_size=b, token_group=args.token_group, **fixed)
             for q, kv, b in itertools.product(args.q_lens, args.kv_lens, args.batch_sizes)]
    device_name = torch.cuda.get_device_name(0)
    checked = 0
    for variant in args.variants:
        for index, case in enumerate(cases):
            if args.limit and index >= args.limit:
                break
            physical = 1 if args.page_mode == "shared" else case["batch_size"]
            estimated = physical * case["kv_len"] * 8 * 128 * 2 * 2 * (2 if args.page_mode == "random" else 1)
            free_bytes, _ = torch.cuda.mem_get_info()
            row = {"variant": variant, "page_mode": args.page_mode, "case": case,
                   "device": device_name, "chunk_keys": args.chunk_keys}
            if estimated > int(free_bytes * 0.70):
                row.update(status="skipped", reason="estimated_memory_limit")
            else:
                check = args.check_correctness and checked < args.correctness_limit
                try:
                    row.update(status="ok", **measure_case(
                        torch, variant, case, args.page_mode, args.chunk_keys, args.warmup,
                        args.repeats, seed=1000 + index, check=check))
                    checked += int(check)
                except (ValueError, RuntimeError) as exc:
                    row.update(status="error", reason=str(exc))
            line = json.dumps(row, sort_keys=True)
            print(line, flush=True)
            if args.output:
                with open(args.output, "a", encoding="utf-8") as fh:
                    fh.write(line + "\n")
            torch.cuda.empty_cache()
    return 0


if __name__ == "__main__":
    sys.exit(main())
