"""GPU parity at head dims 64 and 256 (the reference's is 128).

The kernels are instantiated per head dim: Q and K fragments, V dwords per lane,
output blocks, ring depth (pages in flight hold about the same bytes) and the
merge kernel's dims per lane all follow D; head dim 256 holds at most 32 rows per
kv head. Bar: ``|a - r| <= 2e-3 + 1e-2 |r|`` against the float64 C oracle, which
takes D from the shapes (pinned at 64 and 256 on the CPU).
"""

import sys

import pytest
import torch

from oracle import attention_c64
from small_q_attention_amd import cuda as sqa, decode_api as fi, inputs
from small_q_attention_amd.masks import pack_draft_mask
from tests._helpers import assert_parity

pytestmark = pytest.mark.gpu

F8 = torch.float8_e4m3fn


@pytest.fixture(autouse=True)
def _announce(request):
    sys.__stderr__.write(f"\n[gpu-test] {request.node.nodeid}\n")
    sys.__stderr__.flush()


def _inputs(lens, q_len, d, seed, dtype=torch.float16, page=16, **kw):
    c = inputs.Case(batch=len(lens), q_len=q_len, seq_lens=lens, seed=seed, page_size=page,
                    head_dim=d, **kw)
    q, k, v, bt, sl = inputs.make_inputs(c)
    return q.to(dtype).cuda(), k.to(dtype).cuda(), v.to(dtype).cuda(), bt.cuda(), sl.cuda()


def _oracle(q, k, v, bt, sl, **kw):
    return attention_c64(q.cpu(), k.cpu(), v.cpu(), bt.cpu(), sl.cpu(), k.shape[1], k.shape[2],
                         **kw)


CASES = [(64, 2), (64, 4), (64, 8), (64, 16), (256, 2), (256, 4), (256, 8)]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("d,q_len", CASES)
def test_native_entry_every_plan(d, q_len, dtype):
    """Balanced plan, fixed plans of 128 keys per split and of 16 keys per split
    (hundreds of splits per row: the four-wave merge), single split."""
    lens = [1, q_len, 17, 700, 5000]
    q, k, v, bt, sl = _inputs(lens, q_len, d, 2000 + d + q_len, dtype, k_outlier_frac=0.05)
    ref = _oracle(q, k, v, bt, sl)
    for ck in (None, 128, 16, 1 << 20):
        out = sqa.paged_mtp_attention(q, k, v, bt, sl, 16, max(lens), chunk_keys=ck)
        torch.cuda.synchronize()
        assert out.dtype == dtype and out.shape == q.shape
        assert_parity(out, ref, label=f"d{d} q{q_len} {dtype} ck{ck}")


def test_single_sequence_fixed_plan():
    for d in (64, 256):
        q, k, v, bt, sl = _inputs([3000], 4, d, 2100 + d)
        out = sqa.paged_mtp_attention(q, k, v, bt, sl, 16, 3000)
        assert_parity(out, _oracle(q, k, v, bt, sl), label=f"d{d} batch 1")


def test_head_dim_256_row_limit_and_reference_names():
    q, k, v, bt, sl = _inputs([40], 16, 256, 2200)
    with pytest.raises(ValueError, match="at most 32"):
        sqa.paged_mtp_attention(q, k, v, bt, sl, 16, 40)
    q, k, v, bt, sl = _inputs([40], 4, 64, 2201)
    with pytest.raises(ValueError, match="head_dim"):
        sqa.forward_v3(q, k, v, bt, sl, 16, 512, 40)


@pytest.mark.parametrize("layout", ["NHD", "HND"])
@pytest.mark.parametrize("d", [64, 256])
def test_decode_api_masks_pages_and_scales(d, layout):
    q_len, lens = 8, [5, 64, 900, 2500]
    q, k, v, bt, sl = _inputs(lens, q_len, d, 2300 + d, page=32)
    kv = torch.stack([k, v], 1)
    if layout == "HND":
        kv = kv.transpose(2, 3)
    kv = kv.contiguous()
    g = torch.Generator().manual_seed(23)
    vis = torch.rand(len(lens), q_len, q_len, generator=g) < 0.5
    vis[:, torch.arange(q_len), torch.arange(q_len)] = True
    mask = pack_draft_mask(vis)
    ws = torch.zeros(64 << 20, dtype=torch.uint8, device="cuda")
    out = fi.xqa_batch_decode_with_kv_cache(q.reshape(-1, 32, d), kv, ws, bt, sl, max(lens),
                                            0.07, 0.5, q_len_per_req=q_len, mask=mask.cuda(),
                                            kv_layout=layout)
    torch.cuda.synchronize()
    ref = _oracle(q, k, v, bt, sl, draft_mask=mask, scale=0.07, out_scale=0.5)
    assert_parity(out.view_as(q), ref, label=f"d{d} {layout}")


@pytest.mark.parametrize("qdt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("d,q_len", [(64, 2), (64, 16), (256, 2), (256, 8)])
def test_fp8_cache(d, q_len, qdt):
    lens = [1, q_len, 33, 900, 4000]
    q, k, v, bt, sl = _inputs(lens, q_len, d, 2400 + d + q_len)
    q = q.to(qdt)
    k8, v8 = (k * 4).to(F8), (v * 4).to(F8)
    kv = torch.stack([k8.view(torch.uint8), v8.view(torch.uint8)], 1).view(F8).contiguous()
    ws = torch.zeros(64 << 20, dtype=torch.uint8, device="cuda")
    s1, s2 = d ** -0.5 / 4, 0.25
    out = fi.xqa_batch_decode_with_kv_cache(q.reshape(-1, 32, d), kv, ws, bt, sl, max(lens),
                                            s1, s2, q_len_per_req=q_len)
    torch.cuda.synchronize()
    assert out.dtype == qdt
    ref = _oracle(q, k8, v8, bt, sl, scale=s1, out_scale=s2)
    assert_parity(out.view_as(q), ref, label=f"fp8 d{d} q{q_len} {qdt}")


@pytest.mark.parametrize("q_len", [2, 4, 8])
@pytest.mark.parametrize("hq,hkv", [(32, 8), (64, 16)])
def test_two_heads_per_wave(hq, hkv, q_len):
    """Head dim 64 with up to 32 rows per kv head runs two kv heads per wave (8 rows:
    rows 0-7 and 8-15 of one block; 16 or 32 rows: one or two blocks per head): tree
    masks, scales, one and two head groups, B1 and ragged batches, every plan."""
    d = 64
    lens = [q_len, 9, 700, 3000]
    c = inputs.Case(batch=len(lens), q_len=q_len, seq_lens=lens, seed=2600 + hkv + q_len,
                    num_query_heads=hq, num_kv_heads=hkv, head_dim=d)
    q, k, v, bt, sl = (t.cuda() for t in inputs.make_inputs(c))
    g = torch.Generator().manual_seed(26)
    vis = torch.rand(len(lens), q_len, q_len, generator=g) < 0.5
    vis[:, torch.arange(q_len), torch.arange(q_len)] = True
    mask = pack_draft_mask(vis)
    ws = torch.zeros(64 << 20, dtype=torch.uint8, device="cuda")
    kv = torch.stack([k, v], 1).contiguous()
    out = fi.xqa_batch_decode_with_kv_cache(q.reshape(-1, hq, d), kv, ws, bt, sl, max(lens),
                                            0.09, 0.8, q_len_per_req=q_len, mask=mask.cuda())
    ref = attention_c64(q.cpu(), k.cpu(), v.cpu(), bt.cpu(), sl.cpu(), 16, hkv,
                        draft_mask=mask, scale=0.09, out_scale=0.8)
    assert_parity(out.view_as(q), ref, label=f"hq{hq} hkv{hkv} tree")
    plain = attention_c64(q.cpu(), k.cpu(), v.cpu(), bt.cpu(), sl.cpu(), 16, hkv)
    for ck in (None, 64, 1 << 20):
        got = sqa.paged_mtp_attention(q, k, v, bt, sl, 16, max(lens), chunk_keys=ck)
        assert_parity(got, plain, label=f"hq{hq} hkv{hkv} ck{ck}")
    one = inputs.Case(batch=1, q_len=q_len, seq_lens=[4500], seed=27, num_query_heads=hq,
                      num_kv_heads=hkv, head_dim=d)
    t1 = tuple(t.cuda() for t in inputs.make_inputs(one))
    assert_parity(sqa.paged_mtp_attention(*t1, 16),
                  attention_c64(*(x.cpu() for x in t1), 16, hkv), label=f"hq{hq} hkv{hkv} B1")


def test_wrapper_plan_checks_head_dim():
    d, q_len, lens = 64, 4, [50, 300]
    q, k, v, bt, sl = _inputs(lens, q_len, d, 2500)
    kv = torch.stack([k, v], 1).contiguous()
    pages = [(n + 15) // 16 for n in lens]
    indptr = torch.tensor([0, pages[0], pages[0] + pages[1]], dtype=torch.int32, device="cuda")
    ids = torch.cat([bt[b, :pages[b]] for b in range(2)]).contiguous()
    last = torch.tensor([(n - 1) % 16 + 1 for n in lens], dtype=torch.int32, device="cuda")
    ws = torch.zeros(64 << 20, dtype=torch.uint8, device="cuda")
    dec = fi.BatchDecodeWithPagedKVCacheWrapper(ws, "NHD")
    dec.plan(indptr, ids, last, 32, 8, d, 16, q_len_per_req=q_len)
    out = dec.run(q.reshape(-1, 32, d), kv)
    torch.cuda.synchronize()
    assert_parity(out.view_as(q), _oracle(q, k, v, bt, sl), label="wrapper d64")
    with pytest.raises(ValueError, match="head_dim"):
        dec.run(torch.zeros(2 * q_len, 32, 128, dtype=torch.float16, device="cuda"),
                torch.zeros(4, 2, 16, 8, 128, dtype=torch.float16, device="cuda"))
