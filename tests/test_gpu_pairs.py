"""Paired items on the GPU (the 64-row kernel with the expected-page plan).

Items 2k and 2k + 1 share 2P pages, the even one taking P + d and the odd one
P - d, d = round(P * delta): by default delta is fixed (0.03), under
``SQA_FLAG_ADAPTIVE_PAIRS`` it is read from a record in the workspace that the
merge kernel updates from the workgroups' page-loop times. Results must not
depend on delta:

* parity with the float64 oracle for delta forced to -0.1, -0.05, 0, 0.03 and
  0.1 (the bound), to NaN and to a record without its magic word (both: delta
  0), at q_len 16 (fp16 and bf16), cache pages of 16 and 64 tokens, and a tree
  mask;
* a default call gives the bits of an adaptive one whose record holds 0.03;
* after each call the record holds the magic word and a delta within the
  bound, and every loop-time record has been consumed (marked read);
* calls in a row (delta moving between them) stay within tolerance and the
  delta stays bounded;
* items of the largest size (2048 pages) hold the shift to 0 whatever the
  record says, so neither item of a pair outgrows the page-id table;
* without the flag the record is neither read nor written: any record gives the
  same output bits, and the record's bytes are left as they were.
"""

import struct
import sys

import numpy as np
import pytest
import torch

from oracle import attention_c64
from small_q_attention_amd import _lib, inputs
from small_q_attention_amd.masks import as_words, pack_draft_mask
from tests._helpers import assert_parity

pytestmark = pytest.mark.gpu

HKV, HQ, HD = 8, 32, 128
MAGIC = 0x51A70001  # the record's first word when its second holds a delta
ADAPTIVE = _lib.FLAG_ADAPTIVE_PAIRS


@pytest.fixture(autouse=True)
def _announce(request):
    sys.__stderr__.write(f"\n[gpu-test] {request.node.nodeid}\n")
    sys.__stderr__.flush()


def _tune_offset(batch, q_len, ns):
    """Byte offset of the delta record: behind the partial slots, (max, sum) pairs
    and the merge table."""
    rows = q_len * (HQ // HKV)
    return ns * HKV * rows * (HD + 2) * 4 + batch * 8


def _record(ws, off, ns, batch):
    raw = ws.view(torch.uint8)[off:off + 16 + (ns - batch) * 2 * 8].cpu().numpy()
    magic, delta = struct.unpack("<If", raw[:8].tobytes())
    info = raw[16:].view(np.int32)[1::2]
    return magic, delta, info


def _seed(ws, off, magic, delta):
    ws.view(torch.uint8)[off:off + 8] = torch.tensor(
        np.frombuffer(struct.pack("<If", magic, delta), dtype=np.uint8), device=ws.device)


@pytest.mark.parametrize("qdt,page,tree", [(torch.float16, 16, False), (torch.float16, 64, True),
                                            (torch.bfloat16, 16, False)],
                         ids=["page16", "page64-tree", "bf16"])
def test_paired_items_any_delta(qdt, page, tree):
    q_len, batch, seq_pages, n_items = 16, 2, 256, 16  # items of 32 pages, pairs of 64
    lens = [seq_pages * 16] * batch
    case = inputs.Case(batch=batch, q_len=q_len, seq_lens=lens, seed=1800 + page, page_size=page)
    q, k, v, bt, sl = inputs.make_inputs(case)
    q, k, v = q.to(qdt), k.to(qdt), v.to(qdt)
    mask = words = None
    if tree:
        g = torch.Generator().manual_seed(1801)
        vis = torch.rand(batch, q_len, q_len, generator=g) < 0.4
        vis[:, torch.arange(q_len), torch.arange(q_len)] = True
        mask = pack_draft_mask(vis)
        words = as_words(mask, batch, q_len).cuda()
    ref = attention_c64(q, k, v, bt, sl, page, HKV, draft_mask=mask)
    q, k, v, bt, sl = (t.cuda() for t in (q, k, v, bt, sl))
    ns, pps = batch + n_items, -seq_pages
    nbytes = _lib.workspace_bytes(batch, q_len, HQ, HKV, HD, ns, pps)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    off = _tune_offset(batch, q_len, ns)
    for magic, delta in [(MAGIC, -0.1), (MAGIC, -0.05), (MAGIC, 0.0), (MAGIC, 0.03),
                         (MAGIC, 0.1), (MAGIC, float("nan")), (0, 0.08)]:
        _seed(ws, off, magic, delta)
        out = torch.full_like(q, float("nan"))
        _lib.launch_general(q, out, k, v, bt, sl, words, HD ** -0.5, 1.0, ns, pps, ws,
                            torch.cuda.current_stream().cuda_stream, flags=ADAPTIVE)
        torch.cuda.synchronize()
        label = f"{qdt} page{page} tree={tree} delta={delta} magic={magic:#x}"
        assert_parity(out, ref, label=label)
        m, d, info = _record(ws, off, ns, batch)
        assert m == MAGIC and abs(d) <= 0.1 + 1e-7, (label, m, d)
        assert (info == 0).all(), label
    for i in range(4):  # the delta the kernels choose for themselves
        out = torch.full_like(q, float("nan"))
        _lib.launch_general(q, out, k, v, bt, sl, words, HD ** -0.5, 1.0, ns, pps, ws,
                            torch.cuda.current_stream().cuda_stream, flags=ADAPTIVE)
        torch.cuda.synchronize()
        assert_parity(out, ref, label=f"own delta, call {i}")
        m, d, _ = _record(ws, off, ns, batch)
        assert m == MAGIC and abs(d) <= 0.1 + 1e-7


def test_paired_items_at_the_item_size_limit():
    """Items of the largest size (2048 pages) with delta forced to its bound: the
    shift is held to 0 so that neither item of a pair exceeds the page-id table."""
    from tests._helpers import torch_fp32_reference

    q_len, batch, seq_pages, n_items = 16, 2, 4096, 4  # P = 2048
    lens = [seq_pages * 16] * batch
    case = inputs.Case(batch=batch, q_len=q_len, seq_lens=lens, seed=1850)
    q, k, v, bt, sl = inputs.make_inputs(case, device="cuda", gen_device="cuda")
    ns, pps = batch + n_items, -seq_pages
    ws = torch.zeros(_lib.workspace_bytes(batch, q_len, HQ, HKV, HD, ns, pps), dtype=torch.uint8,
                     device="cuda")
    off = _tune_offset(batch, q_len, ns)
    _seed(ws, off, MAGIC, 0.1)
    out = torch.full_like(q, float("nan"))
    _lib.launch_general(q, out, k, v, bt, sl, None, HD ** -0.5, 1.0, ns, pps, ws,
                        torch.cuda.current_stream().cuda_stream, flags=ADAPTIVE)
    torch.cuda.synchronize()
    ref = torch_fp32_reference(q, k, v, bt, sl, 16, HKV)
    assert_parity(out, ref, label="P = 2048, delta 0.1")
    fixed = torch.full_like(q, float("nan"))  # the default's fixed delta, held to 0 too
    _lib.launch_general(q, fixed, k, v, bt, sl, None, HD ** -0.5, 1.0, ns, pps, ws,
                        torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(fixed, out)


def test_without_the_flag_the_record_is_not_used():
    """Default calls pair items with the fixed delta: a record forcing delta to its
    bound changes no output bit, and neither the record nor the loop-time slots
    behind it are touched."""
    q_len, batch, seq_pages, n_items = 16, 2, 256, 16
    lens = [seq_pages * 16] * batch
    case = inputs.Case(batch=batch, q_len=q_len, seq_lens=lens, seed=1870)
    q, k, v, bt, sl = (t.cuda() for t in inputs.make_inputs(case))
    ns, pps = batch + n_items, -seq_pages
    nbytes = _lib.workspace_bytes(batch, q_len, HQ, HKV, HD, ns, pps)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    off = _tune_offset(batch, q_len, ns)
    outs = []
    for magic, delta in [(0, 0.0), (MAGIC, 0.1), (MAGIC, -0.1)]:
        _seed(ws, off, magic, delta)
        ws[off + 16:off + 16 + (ns - batch) * 2 * 8] = 0x5A
        before = ws[off:off + 16 + (ns - batch) * 2 * 8].clone()
        out = torch.full_like(q, float("nan"))
        _lib.launch_general(q, out, k, v, bt, sl, None, HD ** -0.5, 1.0, ns, pps, ws,
                            torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert torch.equal(ws[off:off + 16 + (ns - batch) * 2 * 8], before), (magic, delta)
        outs.append(out)
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    ref = attention_c64(*(t.cpu() for t in (q, k, v, bt, sl)), 16, HKV)
    assert_parity(outs[0], ref, label="flags 0")


@pytest.mark.parametrize("qdt", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_default_pairs_use_the_fixed_delta(qdt):
    """A default call (no flag) splits each pair at delta 0.03: the same bits as an
    adaptive call whose record holds 0.03, and within the parity bar of the
    float64 oracle. A record of 0 gives another split (other bits, same parity)."""
    q_len, batch, seq_pages, n_items = 16, 2, 256, 16  # P = 32: d = round(0.96) = 1
    lens = [seq_pages * 16] * batch
    case = inputs.Case(batch=batch, q_len=q_len, seq_lens=lens, seed=1890)
    q, k, v, bt, sl = inputs.make_inputs(case)
    q, k, v = q.to(qdt), k.to(qdt), v.to(qdt)
    ref = attention_c64(q, k, v, bt, sl, 16, HKV)
    q, k, v, bt, sl = (t.cuda() for t in (q, k, v, bt, sl))
    ns, pps = batch + n_items, -seq_pages
    ws = torch.zeros(_lib.workspace_bytes(batch, q_len, HQ, HKV, HD, ns, pps), dtype=torch.uint8,
                     device="cuda")
    off = _tune_offset(batch, q_len, ns)

    def call(flags, delta=None):
        if delta is not None:
            _seed(ws, off, MAGIC, delta)
        out = torch.full_like(q, float("nan"))
        _lib.launch_general(q, out, k, v, bt, sl, None, HD ** -0.5, 1.0, ns, pps, ws,
                            torch.cuda.current_stream().cuda_stream, flags=flags)
        torch.cuda.synchronize()
        return out

    default = call(0)
    assert_parity(default, ref, label=f"{qdt} default pairs")
    assert torch.equal(call(ADAPTIVE, 0.03), default)
    at_zero = call(ADAPTIVE, 0.0)
    assert_parity(at_zero, ref, label=f"{qdt} delta 0")
    assert not torch.equal(at_zero, default)
    assert torch.equal(call(0), default)
