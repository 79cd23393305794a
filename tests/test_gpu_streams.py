"""Eager calls on several streams of one GPU at once, as a server with one stream per
request group issues them. The Python entry points keep one workspace per (device,
stream), so calls whose kernels run concurrently on different streams never share
partials: each output must equal, bit for bit, the same call made alone on the
default stream. Covered: two streams fed alternately from one host thread, and
two host threads with a stream each (the C entry releases the GIL, so the host
calls overlap too); the cases mix the fixed plan, the balanced plan with an
expected page count, the packed plan over a ragged batch, and the 64-row kernel.
"""

import sys
import threading

import pytest
import torch

from small_q_attention_amd import cuda as sqa, inputs

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _announce(request):
    sys.__stderr__.write(f"\n[gpu-test] {request.node.nodeid}\n")
    sys.__stderr__.flush()


CASES = [
    ("uniform_b4_q8_kv8192", inputs.uniform_case(4, 8, 8192, seed=3001)),
    ("ragged_b3_q4", inputs.Case(batch=3, q_len=4, seq_lens=[5000, 300, 2200], seed=3002)),
    ("one_q16_kv4096", inputs.uniform_case(1, 16, 4096, seed=3003)),
    ("uniform_b8_q2_kv2048", inputs.uniform_case(8, 2, 2048, seed=3004)),
]


def _prepared():
    out = []
    for label, case in CASES:
        tensors = tuple(t.cuda() for t in inputs.make_inputs(case))
        out.append((label, tensors, case.max_seq_len))
    return out


def _call(tensors, max_seq_len):
    return sqa.paged_mtp_attention(*tensors, 16, max_seq_len)


def _alone(prepared):
    want = []
    for label, tensors, msl in prepared:
        want.append(_call(tensors, msl))
        torch.cuda.synchronize()
    return want


def test_two_streams_from_one_thread():
    prepared = _prepared()
    want = _alone(prepared)
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    got = {}
    for rep in range(6):  # alternate: stream 0 takes cases 0, 2; stream 1 cases 1, 3
        for i, (label, tensors, msl) in enumerate(prepared):
            with torch.cuda.stream(streams[i % 2]):
                got[(rep, i)] = _call(tensors, msl)
    torch.cuda.synchronize()
    for (rep, i), out in got.items():
        assert torch.equal(out, want[i]), (rep, prepared[i][0])


def test_two_threads_with_a_stream_each():
    prepared = _prepared()
    want = _alone(prepared)
    results, errors = {}, []
    start = threading.Barrier(2)

    def worker(t):
        try:
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.default_stream())
            start.wait()
            with torch.cuda.stream(s):
                for rep in range(8):
                    for i in (t, t + 2):
                        label, tensors, msl = prepared[i]
                        results[(t, rep, i)] = _call(tensors, msl)
            s.synchronize()
        except Exception as exc:  # reported by the main thread
            errors.append(repr(exc))

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(2)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=90)
    assert not any(th.is_alive() for th in threads), "a worker thread did not finish"
    assert not errors, errors
    torch.cuda.synchronize()
    assert len(results) == 2 * 8 * 2
    for (t, rep, i), out in results.items():
        assert torch.equal(out, want[i]), (t, rep, prepared[i][0])
