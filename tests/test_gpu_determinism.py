"""Run-to-run reproducibility at full size: the same inputs give the same output bits.

The reference's grid and chunking are fixed by the shapes
(``/root/reference/csrc/small_q_attention_ext.cu:1096-1099``), so identical calls
return identical bits. Here the plan is fixed by the shapes too: at the cfg3
shape (16 sequences of 32768 keys, the expected-page balanced plan that a known
``max_seq_len`` selects) the 64-row kernel (q_len 16) and the 32-row one (q_len 8)
must give equal bits

* for two eager calls in a row on one stream,
* for four replays of a captured graph (eager work between replays) against the
  eager result,
* for the no-allocation entry point against the workspace entry point.

Inputs are drawn on the device (a 4.3 GB pool); parity itself is covered by the
other GPU tests at this shape.
"""

import sys

import pytest
import torch

from small_q_attention_amd import _lib, cuda as sqa, inputs

pytestmark = pytest.mark.gpu

KV_LEN, BATCH = 32768, 16


@pytest.fixture(autouse=True)
def _announce(request):
    sys.__stderr__.write(f"\n[gpu-test] {request.node.nodeid}\n")
    sys.__stderr__.flush()


@pytest.fixture(scope="module")
def pool():
    # One 2x pool (4.3 GB) for every q_len: the caches and table do not depend on it.
    case = inputs.uniform_case(BATCH, 16, KV_LEN, seed=2300, k_outlier_frac=0.01)
    q, k, v, bt, sl = inputs.make_inputs(case, device="cuda", gen_device="cuda")
    yield k, v, bt, sl
    del k, v
    torch.cuda.empty_cache()


def _query(q_len):
    g = torch.Generator(device="cuda").manual_seed(2301 + q_len)
    return torch.randn(BATCH, q_len, 32, 128, generator=g, device="cuda", dtype=torch.float16)


@pytest.mark.parametrize("q_len", [16, 8])
def test_identical_calls_give_identical_bits(pool, q_len):
    k, v, bt, sl = pool
    q = _query(q_len)
    ns, pps = _lib.plan_splits(0, BATCH, q_len, 32, 8, 128, KV_LEN, bt.shape[1], 0)
    assert pps == -(KV_LEN // 16), (ns, pps)  # the expected-page balanced plan
    a = sqa.paged_mtp_attention(q, k, v, bt, sl, 16, KV_LEN)
    b = sqa.paged_mtp_attention(q, k, v, bt, sl, 16, KV_LEN)
    torch.cuda.synchronize()
    assert torch.isfinite(a.float()).all()
    assert torch.equal(a, b)
    # A fresh (uninitialised) workspace and one left by other calls give the same bits.
    stream = torch.cuda.current_stream().cuda_stream
    nbytes = _lib.workspace_bytes(BATCH, q_len, 32, 8, 128, ns, pps)
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    for fill in (0x00, 0x7F):
        ws.fill_(fill)
        out = torch.empty_like(q)
        _lib.launch(q, k, v, bt, sl, out, ws, ns, pps, stream)
        torch.cuda.synchronize()
        assert torch.equal(out, a), f"workspace filled with {fill:#x}"


@pytest.mark.parametrize("q_len", [16, 8])
def test_graph_replays_equal_the_eager_call(pool, q_len):
    k, v, bt, sl = pool
    q = _query(q_len)
    eager = sqa.paged_mtp_attention(q, k, v, bt, sl, 16, KV_LEN)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            sqa.paged_mtp_attention(q, k, v, bt, sl, 16, KV_LEN)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out = sqa.paged_mtp_attention(q, k, v, bt, sl, 16, KV_LEN)
    for i in range(4):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(static_out, eager), f"replay {i}"
        junk = torch.randn(1 << 20, device="cuda").sum()  # eager work between replays
        torch.cuda.synchronize()
        del junk
    del graph


def test_noalloc_equals_the_workspace_entry_point_at_q16(pool):
    k, v, bt, sl = pool
    q = _query(16)
    lib = _lib.load()
    ns, pps = _lib.plan_splits(0, BATCH, 16, 32, 8, 128, KV_LEN, bt.shape[1], 0)
    assert _lib.workspace_bytes(BATCH, 16, 32, 8, 128, ns, pps) <= 64 << 20
    stream = torch.cuda.current_stream().cuda_stream
    ref = sqa.paged_mtp_attention(q, k, v, bt, sl, 16, KV_LEN)
    for i in range(2):
        out = torch.empty_like(q)
        rc = lib.sqa_paged_mtp_attention_noalloc(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), bt.data_ptr(), sl.data_ptr(),
            out.data_ptr(), BATCH, 16, 32, 8, 128, k.shape[0], 16, bt.shape[1], ns, pps, stream)
        assert rc == 0, lib.sqa_last_error().decode()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"call {i}"
