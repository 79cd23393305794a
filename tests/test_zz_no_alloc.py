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
