"""The no-allocation entry point ``sqa_paged_mtp_attention_noalloc`` (include/sqa.h).

It runs the plan's kernels with the library's per-GPU device scratch in place of
a caller workspace. Called through the C ABI, it must give the same bits as
``sqa_paged_mtp_attention`` with a caller workspace, call after call: here two
calls in a row, the second on a smaller input (fewer sequences, shorter, other
plan), so leftovers of the first call in the shared scratch cannot leak into the
second. A plan larger than the scratch is refused before any launch.
"""

import ctypes

import pytest
import torch

from small_q_attention_amd import _lib, inputs

from tests._helpers import assert_parity

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 64 << 20  # SQA_NOALLOC_SCRATCH_BYTES


def _noalloc(lib, q, k, v, bt, sl, out, ns, pps, stream):
    b, q_len, hq, d = q.shape
    return lib.sqa_paged_mtp_attention_noalloc(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), bt.data_ptr(), sl.data_ptr(), out.data_ptr(),
        b, q_len, hq, k.shape[2], d, k.shape[0], k.shape[1], bt.shape[1], ns, pps, stream)


def _with_workspace(q, k, v, bt, sl, ns, pps, stream):
    b, q_len, hq, d = q.shape
    nbytes = _lib.workspace_bytes(b, q_len, hq, k.shape[2], d, ns, pps)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device="cuda")
    out = torch.empty_like(q)
    _lib.launch(q, k, v, bt, sl, out, ws if nbytes else None, ns, pps, stream)
    return out


# (label, case, chunk_keys): chunk_keys 0 = automatic plan.
CALLS = [
    ("balanced_b4_q4_kv8192", inputs.uniform_case(4, 4, 8192, seed=41), 0),
    ("fixed_b1_q8_ragged_small", inputs.Case(batch=1, q_len=8, seq_lens=[700], seed=42), 0),
    ("balanced_b3_q16_ragged", inputs.Case(batch=3, q_len=16, seq_lens=[2100, 40, 999], seed=43), 0),
    ("fixed_chunk128_b2_q2", inputs.Case(batch=2, q_len=2, seq_lens=[300, 33], seed=44), 128),
]


@pytest.mark.parametrize("first,second", [(0, 1), (2, 3)],
                         ids=["large_then_small", "q16_then_q2"])
def test_noalloc_matches_the_workspace_entry_point(first, second):
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    for index in (first, second):
        label, case, ck = CALLS[index]
        print(f"[noalloc] {label}", flush=True)
        tensors = tuple(t.cuda() for t in inputs.make_inputs(case))
        q, k, v, bt, sl = tensors
        ns, pps = _lib.plan_splits(0, case.batch, case.q_len, case.num_query_heads,
                                   case.num_kv_heads, case.head_dim, case.max_seq_len,
                                   bt.shape[1], ck)
        assert _lib.workspace_bytes(case.batch, case.q_len, case.num_query_heads,
                                    case.num_kv_heads, case.head_dim, ns, pps) <= SCRATCH_BYTES
        want = _with_workspace(q, k, v, bt, sl, ns, pps, stream)
        got = torch.full_like(q, float("nan"))
        rc = _noalloc(lib, q, k, v, bt, sl, got, ns, pps, stream)
        assert rc == 0, _lib.last_error(lib)
        torch.cuda.synchronize()
        assert torch.equal(got, want), label
        if index == 0:
            from oracle import attention_c64

            cpu = tuple(t.cpu() for t in tensors)
            assert_parity(got, attention_c64(*cpu, case.page_size, case.num_kv_heads),
                          batches=[0], label=label)


def test_noalloc_repeated_calls_are_stable():
    """Ten back-to-back calls on one stream give the workspace entry point's bits each time."""
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    case = inputs.Case(batch=5, q_len=4, seq_lens=[4000, 17, 1200, 3300, 64], seed=45)
    q, k, v, bt, sl = (t.cuda() for t in inputs.make_inputs(case))
    ns, pps = _lib.plan_splits(0, 5, 4, 32, 8, 128, 4000, bt.shape[1], 0)
    want = _with_workspace(q, k, v, bt, sl, ns, pps, stream)
    outs = [torch.empty_like(q) for _ in range(10)]
    for out in outs:
        assert _noalloc(lib, q, k, v, bt, sl, out, ns, pps, stream) == 0, _lib.last_error(lib)
    torch.cuda.synchronize()
    for out in outs:
        assert torch.equal(out, want)


def test_noalloc_refuses_a_plan_beyond_the_scratch():
    lib = _lib.load()
    case = inputs.uniform_case(1, 16, 1024, seed=46)
    q, k, v, bt, sl = (t.cuda() for t in inputs.make_inputs(case))
    # A fixed plan of one-page splits over 2048 pages of 64 rows: 2048 slots x 8 kv
    # heads x 64 rows x 130 floats = 545 MB of partials.
    ns, pps = 2048, 1
    assert _lib.workspace_bytes(1, 16, 32, 8, 128, ns, pps) > SCRATCH_BYTES
    out = torch.zeros_like(q)
    rc = _noalloc(lib, q, k, v, bt, sl, out, ns, pps, torch.cuda.current_stream().cuda_stream)
    assert rc == 3  # SQA_ERR_WORKSPACE
    assert "no-allocation" in _lib.last_error(lib)
    torch.cuda.synchronize()
    assert not out.any()  # nothing ran


# Run in a fresh process: the no-allocation call captured into a HIP graph, either
# as the process's first call of the entry point (the scratch address is looked up
# inside the capture) or after an eager warm-up call; replays must equal an eager
# call of the same entry point bit for bit.
_CAPTURE_SCRIPT = r"""
import sys
sys.path.insert(0, sys.argv[1])
import torch
from small_q_attention_amd import _lib, inputs
warm = sys.argv[2] == "warm"
lib = _lib.load(build_if_missing=False)
case = inputs.Case(batch=3, q_len=8, seq_lens=[3000, 700, 1900], seed=47)
q, k, v, bt, sl = (t.cuda() for t in inputs.make_inputs(case))
ns, pps = _lib.plan_splits(0, 3, 8, 32, 8, 128, 3000, bt.shape[1], 0)
assert ns > 1

def call(out, stream):
    return lib.sqa_paged_mtp_attention_noalloc(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), bt.data_ptr(), sl.data_ptr(), out.data_ptr(),
        3, 8, 32, 8, 128, k.shape[0], 16, bt.shape[1], ns, pps, stream)

eager = torch.empty_like(q)
if warm:
    assert call(eager, torch.cuda.current_stream().cuda_stream) == 0, _lib.last_error(lib)
    torch.cuda.synchronize()
static_out = torch.empty_like(q)
graph = torch.cuda.CUDAGraph()
s = torch.cuda.Stream()
s.wait_stream(torch.cuda.current_stream())
with torch.cuda.stream(s):
    with torch.cuda.graph(graph, stream=s):
        rc = call(static_out, s.cuda_stream)
torch.cuda.current_stream().wait_stream(s)
torch.cuda.synchronize()
if rc != 0:
    print("capture rc", rc, _lib.last_error(lib), flush=True)
    sys.exit(3)
if not warm:
    assert call(eager, torch.cuda.current_stream().cuda_stream) == 0, _lib.last_error(lib)
    torch.cuda.synchronize()
for i in range(3):
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(static_out, eager), f"replay {i}"
    junk = torch.randn(1 << 20, device="cuda").sum()
    torch.cuda.synchronize()
print("capture ok", flush=True)
"""


@pytest.mark.parametrize("order", ["cold", "warm"])
def test_noalloc_under_graph_capture(order):
    """The no-allocation entry point captured in a HIP graph in a fresh process: as
    the first call of the entry point (its scratch address is looked up during the
    capture) and after an eager warm-up call. Replays equal an eager call."""
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    print(f"[noalloc] graph capture, {order}", flush=True)
    r = subprocess.run([sys.executable, "-c", _CAPTURE_SCRIPT, str(root), order],
                       capture_output=True, text=True, timeout=110)
    assert r.returncode == 0, (r.returncode, r.stdout[-2000:], r.stderr[-2000:])
    assert "capture ok" in r.stdout


# Run in a fresh process: device free memory (hipMemGetInfo) around the first call
# of the workspace entry point, then around the first and second calls of the
# no-allocation entry point. The scratch lives in a code object of its own, with
# no kernels, which HIP loads (deferred loading, its default) when the scratch
# address is first looked up: a process that never calls the no-allocation entry
# point does not hold the scratch.
_MEMORY_SCRIPT = r"""
import sys
sys.path.insert(0, sys.argv[1])
import torch
from small_q_attention_amd import _lib, inputs

def free():
    torch.cuda.synchronize()
    return torch.cuda.mem_get_info()[0]

torch.zeros(1, device="cuda")
case = inputs.uniform_case(2, 4, 2048, seed=48)
q, k, v, bt, sl = (t.cuda() for t in inputs.make_inputs(case))
lib = _lib.load(build_if_missing=False)
ns, pps = _lib.plan_splits(0, 2, 4, 32, 8, 128, 2048, bt.shape[1], 0)
nbytes = _lib.workspace_bytes(2, 4, 32, 8, 128, ns, pps)
ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device="cuda")
want, got, again = torch.empty_like(q), torch.empty_like(q), torch.empty_like(q)
stream = torch.cuda.current_stream().cuda_stream

def noalloc(out):
    rc = lib.sqa_paged_mtp_attention_noalloc(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), bt.data_ptr(), sl.data_ptr(), out.data_ptr(),
        2, 4, 32, 8, 128, k.shape[0], 16, bt.shape[1], ns, pps, stream)
    assert rc == 0, _lib.last_error(lib)

f0 = free()
_lib.launch(q, k, v, bt, sl, want, ws, ns, pps, stream)
f1 = free()
noalloc(got)
f2 = free()
noalloc(again)
f3 = free()
assert torch.equal(got, want) and torch.equal(again, want)
print("held", f0 - f1, f1 - f2, f2 - f3, flush=True)
"""


def test_scratch_is_held_from_the_first_noalloc_call_on():
    """A process holds the 64 MiB scratch only once it calls the no-allocation entry
    point: the first workspace call takes well under it (the kernels' code object),
    the first no-allocation call at least the scratch, the second nothing more."""
    import os
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    env = {k: v for k, v in os.environ.items() if k != "HIP_ENABLE_DEFERRED_LOADING"}
    print("[noalloc] device memory held, fresh process", flush=True)
    r = subprocess.run([sys.executable, "-c", _MEMORY_SCRIPT, str(root)], capture_output=True,
                       text=True, timeout=110, env=env)
    assert r.returncode == 0, (r.returncode, r.stdout[-2000:], r.stderr[-2000:])
    line = [s for s in r.stdout.splitlines() if s.startswith("held ")][-1]
    workspace_call, first_noalloc, second_noalloc = (int(x) for x in line.split()[1:])
    print(f"[noalloc] held by the first workspace call {workspace_call >> 20} MiB, first "
          f"no-allocation call {first_noalloc >> 20} MiB, second {second_noalloc >> 20} MiB",
          flush=True)
    assert workspace_call < 32 << 20
    assert first_noalloc >= SCRATCH_BYTES
    assert abs(second_noalloc) < 8 << 20
