"""GPU parity of OCP FP8 E4M3 KV caches (``torch.float8_e4m3fn``) with fp16 or bf16 queries.

Every e4m3 value is exact in fp16 and bf16 and the kernel widens K and V exactly
before the MFMAs; K fragments are loaded with another (equivalent) order of the
head dims than for 16-bit caches, so an e4m3 cache agrees with an fp16 (bf16)
cache holding the same values to fp32 rounding of the dot products, and with
the oracle at the usual bar ``|a - r| <= 2e-3 + 1e-2 |r|``. Per-tensor K / V
scales go into ``bmm1_scale`` / ``bmm2_scale``.
"""

import sys

import pytest
import torch

from oracle import attention_c64
from small_q_attention_amd import _lib, decode_api as fi, inputs
from small_q_attention_amd.masks import pack_draft_mask
from tests._helpers import assert_parity, compact_sequences

pytestmark = pytest.mark.gpu

F8 = torch.float8_e4m3fn
WORKSPACE = 64 << 20


@pytest.fixture(autouse=True)
def _announce(request):
    sys.__stderr__.write(f"\n[gpu-test] {request.node.nodeid}\n")
    sys.__stderr__.flush()


def _nhd(k, v):
    return torch.stack([k.view(torch.uint8), v.view(torch.uint8)], 1).view(F8).contiguous() \
        if k.dtype == F8 else torch.stack([k, v], 1).contiguous()


def _xqa(q, kv, bt, sl, q_len, ws, **kw):
    out = fi.xqa_batch_decode_with_kv_cache(q.reshape(-1, q.shape[2], q.shape[3]), kv, ws, bt,
                                            sl, int(sl.max()), kw.pop("s1", 128 ** -0.5),
                                            kw.pop("s2", 1.0), q_len_per_req=q_len, **kw)
    torch.cuda.synchronize()
    return out.view_as(q)


@pytest.mark.parametrize("qdt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("q_len", [2, 8, 16])
def test_fp8_cache_matches_wide_cache_bits(qdt, q_len):
    lens = [1, q_len, 33, 900, 5000]
    c = inputs.Case(batch=len(lens), q_len=q_len, seq_lens=lens, seed=1200 + q_len)
    q, k, v, bt, sl = (t.cuda() for t in inputs.make_inputs(c))
    q = q.to(qdt)
    k8, v8 = (k * 4).to(F8), (v * 4).to(F8)  # scaled to use e4m3's range; undone below
    kw, vw = k8.to(qdt), v8.to(qdt)
    ws = torch.zeros(WORKSPACE, dtype=torch.uint8, device="cuda")
    s1, s2 = 128 ** -0.5 / 4, 0.25  # k_scale, v_scale folded in
    a = _xqa(q, _nhd(k8, v8), bt, sl, q_len, ws, s1=s1, s2=s2)
    b = _xqa(q, _nhd(kw, vw), bt, sl, q_len, ws, s1=s1, s2=s2)
    assert a.dtype == qdt
    af, bf = a.float(), b.float()
    assert ((af - bf).abs() <= 2e-3 + 1e-2 * bf.abs()).all()
    ref = attention_c64(q.cpu(), k8.cpu(), v8.cpu(), bt.cpu(), sl.cpu(), 16, 8, scale=s1,
                        out_scale=s2)
    assert_parity(a, ref, label=f"{qdt} q{q_len}")


def test_fp8_cache_masks_hnd_and_large_pages():
    q_len, lens = 8, [5, 64, 700, 2500]
    c = inputs.Case(batch=len(lens), q_len=q_len, seq_lens=lens, seed=1300, page_size=32)
    q, k, v, bt, sl = (t.cuda() for t in inputs.make_inputs(c))
    k8, v8 = k.to(F8), v.to(F8)
    hnd = torch.stack([k8.view(torch.uint8), v8.view(torch.uint8)], 1)
    hnd = hnd.permute(0, 1, 3, 2, 4).contiguous().view(F8)
    g = torch.Generator().manual_seed(13)
    vis = torch.rand(len(lens), q_len, q_len, generator=g) < 0.5
    vis[:, torch.arange(q_len), torch.arange(q_len)] = True
    mask = pack_draft_mask(vis)
    ws = torch.zeros(WORKSPACE, dtype=torch.uint8, device="cuda")
    out = _xqa(q, hnd, bt, sl, q_len, ws, kv_layout="HND", mask=mask.cuda())
    ref = attention_c64(q.cpu(), k8.cpu(), v8.cpu(), bt.cpu(), sl.cpu(), 32, 8, draft_mask=mask)
    assert_parity(out, ref, label="fp8 HND p32 tree")


@pytest.mark.parametrize("chunk", [None, 16, 48, 1 << 20])
def test_fp8_64_rows_page_pairs(chunk):
    """64 rows per kv head (q_len 16, GQA 4) over an e4m3 cache under fp16 queries
    take the pages two at a time. Plans with 1- and 3-page splits leave a last
    pair without its second page; the lengths put the draft block and the
    sequence end on either page of a pair; the draft mask is a random tree, and
    the unused slots of every last page hold e4m3 NaN bytes."""
    q_len, lens = 16, [16, 17, 31, 32, 33, 47, 48, 49, 300, 1111]
    c = inputs.Case(batch=len(lens), q_len=q_len, seq_lens=lens, seed=1400 + (chunk or 0) % 97)
    q, k, v, bt, sl = inputs.make_inputs(c)
    kb, vb = k.to(F8).view(torch.uint8).clone(), v.to(F8).view(torch.uint8).clone()
    for b, n in enumerate(lens):
        last = int(bt[b, (n - 1) // 16])
        if n % 16:
            kb[last, n % 16:] = 0x7F  # e4m3 NaN
            vb[last, n % 16:] = 0x7F
    k8, v8 = kb.view(F8), vb.view(F8)
    g = torch.Generator().manual_seed(14)
    vis = torch.rand(len(lens), q_len, q_len, generator=g) < 0.5
    vis[:, torch.arange(q_len), torch.arange(q_len)] = True
    mask = pack_draft_mask(vis)
    plan = None if chunk is None else _lib.plan_splits(0, len(lens), q_len, 32, 8, 128,
                                                       max(lens), bt.shape[1], chunk)
    # No workspace buffer: the entry sizes it for the plan (1-page splits need ~190 MB).
    out = fi._run(q.cuda().reshape(-1, 32, 128), k8.cuda(), v8.cuda(), bt.cuda(), sl.cuda(),
                  max(lens), q_len, 128 ** -0.5, 1.0, mask.cuda(), None, None, plan=plan)
    torch.cuda.synchronize()
    ref = attention_c64(q, k8, v8, bt, sl, 16, 8, draft_mask=mask)
    assert_parity(out.view_as(q), ref, label=f"e4m3 q16 pairs ck{chunk}")


def test_fp8_full_size():
    """cfg3 shape with an e4m3 cache: agrees with the fp16 cache of the same values."""
    case = inputs.baseline_configs()["cfg3"]
    q, k, v, bt, sl = inputs.make_inputs(case, device="cuda", gen_device="cuda")
    kv8 = _nhd(k.to(F8), v.to(F8))
    kv16 = torch.empty(kv8.shape, dtype=torch.float16, device="cuda")
    kv16.copy_(kv8)
    del k, v
    torch.cuda.empty_cache()
    ws = torch.zeros(WORKSPACE, dtype=torch.uint8, device="cuda")
    a = _xqa(q, kv8, bt, sl, 8, ws)
    b = _xqa(q, kv16, bt, sl, 8, ws)
    assert torch.isfinite(a.float()).all()
    assert (a.float() - b.float()).abs().max().item() <= 2e-3
    raw = kv8.view(torch.uint8)  # gather the bytes; e4m3 again for the oracle
    cq, ck, cv, cbt, csl = compact_sequences(q, raw[:, 0], raw[:, 1], bt, sl, [4])
    assert_parity(a[4:5], attention_c64(cq, ck.view(F8), cv.view(F8), cbt, csl, 16, 8),
                  label="cfg3 fp8")
