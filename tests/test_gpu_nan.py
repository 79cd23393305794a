"""Non-finite cache contents: a NaN among the keys or values a row sees makes the
row (or, for a value, that dimension of it) NaN, and no other row changes, as in
the reference, whose per-row loop reads only the keys and values the row sees
(``/root/reference/src/small_q_attention/reference.py:68-70``;
``/root/reference/csrc/small_q_attention_ext.cu:40-50``). Checked against the
float64 C oracle, which follows the same rule: NaN positions equal element for
element, every other output within the parity bar.

Placed: a NaN key in a prefix token (every row of that sequence and kv head), a
NaN value in a prefix token (one dimension of those rows), a NaN key in a draft
token (only the draft rows that see it: its score is masked to -inf before any
maximum or exponential for the others) and a NaN in one query (that row: all
its scores NaN, so its running max never leaves -inf). Each with fp16 and e4m3 caches,
q_len 2, 8 and 16 (the one-wave, 32-row and 64-row kernels), the automatic
(balanced) plan and a fixed plan of 128-key splits (so NaN partials go through
the merge).

A NaN or infinite *value* of a draft token that some draft row does not see is
the one place the kernel differs: the shared PV product multiplies it by that
row's zero probability, so the NaN reaches every draft row of the sequence and
kv head. ``test_nan_value_in_a_draft_token`` pins that behaviour.
"""

import sys

import numpy as np
import pytest
import torch

from oracle import attention_c64
from small_q_attention_amd import _lib, inputs
from tests._helpers import TOL_ABS, TOL_REL

pytestmark = pytest.mark.gpu

F8 = torch.float8_e4m3fn
LENS = [700, 1500, 333]


@pytest.fixture(autouse=True)
def _announce(request):
    sys.__stderr__.write(f"\n[gpu-test] {request.node.nodeid}\n")
    sys.__stderr__.flush()


def _inputs(q_len, kv, seed, lens=LENS):
    c = inputs.Case(batch=len(lens), q_len=q_len, seq_lens=lens, seed=seed)
    q, k, v, bt, sl = (t.cuda() for t in inputs.make_inputs(c))
    if kv == "e4m3":
        k, v = k.to(F8), v.to(F8)
    return q, k, v, bt, sl


def _poison(cache, bt, b, t, head, dim):
    """Set element (token t of sequence b, kv head, dim) of a cache to NaN."""
    page, slot = int(bt[b, t // 16]), t % 16
    if cache.dtype == F8:
        cache.view(torch.uint8)[page, slot, head, dim] = 0x7F  # e4m3 NaN
    else:
        cache[page, slot, head, dim] = float("nan")


def _run(q, k, v, bt, sl, chunk):
    b, q_len, hq, d = q.shape
    ns, pps = _lib.plan_splits(0, b, q_len, hq, k.shape[2], d, int(sl.max()), bt.shape[1], chunk)
    nbytes = _lib.workspace_bytes(b, q_len, hq, k.shape[2], d, ns, pps)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device="cuda")
    out = torch.empty_like(q)
    _lib.launch_general(q, out, k, v, bt, sl, None, d ** -0.5, 1.0, ns, pps, ws,
                        torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return out


def _compare(out, ref, label):
    a = out.float().cpu().numpy().astype(np.float64)
    r16 = ref.astype(np.float16).astype(np.float64)
    nan_a, nan_r = np.isnan(a), np.isnan(r16)
    assert nan_r.any(), f"{label}: the placement produced no NaN in the oracle"
    if not np.array_equal(nan_a, nan_r):
        at = np.argwhere(nan_a != nan_r)
        i = tuple(at[0])
        raise AssertionError(f"{label}: {len(at)} NaN positions differ from the oracle "
                             f"(kernel {int(nan_a.sum())} NaN, oracle {int(nan_r.sum())}), "
                             f"first {list(i)}: kernel {a[i]}, oracle {r16[i]}; "
                             f"rows {sorted(set(tuple(x[:3]) for x in at.tolist()))[:8]}")
    fin = ~nan_r
    assert np.isfinite(a[fin]).all(), label
    err = np.abs(a[fin] - r16[fin])
    assert np.all(err <= TOL_ABS + TOL_REL * np.abs(r16[fin])), f"{label}: max err {err.max()}"


@pytest.mark.parametrize("chunk", [0, 128])
@pytest.mark.parametrize("q_len", [2, 8, 16])
@pytest.mark.parametrize("kv", ["fp16", "e4m3"])
def test_nan_reaches_only_the_rows_that_see_it(kv, q_len, chunk):
    q, k, v, bt, sl = _inputs(q_len, kv, seed=1700 + q_len)
    _poison(k, bt, 1, 100, 3, 17)                       # prefix key: heads 12-15 of sequence 1
    _poison(v, bt, 2, 50, 0, 99)                        # prefix value: dim 99, heads 0-3 of seq 2
    _poison(k, bt, 0, LENS[0] - q_len + 1, 5, 64)       # draft key 1: rows qi >= 1, heads 20-23
    q[2, q_len - 1, 30, 7] = float("nan")               # a query: that row only (every score NaN)
    ref = attention_c64(*(t.cpu() for t in (q, k, v, bt, sl)), 16, 8)
    out = _run(q, k, v, bt, sl, chunk)
    _compare(out, ref, f"{kv} q{q_len} chunk{chunk}")
    # the draft row that does not see draft key 1 stays finite
    assert torch.isfinite(out[0, 0, 20:24].float()).all()
    assert torch.isnan(out[0, 1:, 20:24].float()).all()


@pytest.mark.parametrize("kv", ["fp16", "e4m3"])
def test_nan_value_in_a_draft_token(kv):
    """The kernel's one difference (module docstring): a NaN value in draft token 1
    reaches draft row 0 of the same sequence and kv head too, in that dimension; the
    rows that see the token match the oracle and every other row is untouched."""
    q_len = 4
    q, k, v, bt, sl = _inputs(q_len, kv, seed=1750)
    _poison(v, bt, 0, LENS[0] - q_len + 1, 2, 40)  # draft token 1, kv head 2 (heads 8-11), dim 40
    ref = attention_c64(*(t.cpu() for t in (q, k, v, bt, sl)), 16, 8)
    out = _run(q, k, v, bt, sl, 0).float().cpu().numpy()
    assert np.isnan(ref[0, 1:, 8:12, 40]).all() and not np.isnan(ref[0, 0, 8:12, 40]).any()
    assert np.isnan(out[0, :, 8:12, 40]).all()  # row 0 as well: 0 x NaN in the shared product
    keep = np.ones(out.shape, dtype=bool)
    keep[0, :, 8:12, 40] = False
    r16 = ref.astype(np.float16).astype(np.float64)
    assert np.isfinite(out[keep]).all()
    assert np.all(np.abs(out[keep] - r16[keep]) <= TOL_ABS + TOL_REL * np.abs(r16[keep]))


@pytest.mark.parametrize("q_len", [2, 8])
@pytest.mark.parametrize("kv", ["fp16", "e4m3"])
def test_nan_single_sequence_whole_ring_pieces(kv, q_len):
    """One sequence of 4096 keys: the automatic plan cuts it into 4-page splits,
    which the 16-bit kernels take in one softmax step over the whole register
    ring (scores of all pages, then one running-max update)."""
    lens = [4096]
    q, k, v, bt, sl = _inputs(q_len, kv, seed=1780 + q_len, lens=lens)
    ns, pps = _lib.plan_splits(0, 1, q_len, 32, 8, 128, 4096, bt.shape[1], 0)
    assert pps == 4, (ns, pps)
    _poison(k, bt, 0, 1000, 3, 17)                   # prefix key: heads 12-15
    _poison(v, bt, 0, 2000, 6, 5)                    # prefix value: dim 5 of heads 24-27
    _poison(k, bt, 0, lens[0] - q_len + 1, 5, 64)    # draft key 1: rows qi >= 1, heads 20-23
    q[0, q_len - 1, 30, 7] = float("nan")
    ref = attention_c64(*(t.cpu() for t in (q, k, v, bt, sl)), 16, 8)
    out = _run(q, k, v, bt, sl, 0)
    _compare(out, ref, f"{kv} q{q_len} one sequence")
    assert torch.isfinite(out[0, 0, 20:24].float()).all()
