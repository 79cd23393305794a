"""GPU parity of the general entry point (``sqa_paged_attention``) and the FlashInfer-shaped
API (``small_q_attention_amd.decode_api``) with the oracle.

Interleaved NHD / HND caches must give the same bits as the separate caches
(the kernel reads the same values through other strides); draft masks, scales
and CSR page lists are checked against the float64 C oracle at the parity bar
``|a - r| <= 2e-3 + 1e-2 |r|``.
"""

import sys

import numpy as np
import pytest
import torch

from oracle import attention_c64
from small_q_attention_amd import _lib, cuda as sqa, decode_api as fi, inputs
from small_q_attention_amd.masks import pack_draft_mask, spec_dec_mask
from tests._helpers import assert_parity, compact_sequences

pytestmark = pytest.mark.gpu

WORKSPACE = 64 << 20


@pytest.fixture(autouse=True)
def _announce(request):
    sys.__stderr__.write(f"\n[gpu-test] {request.node.nodeid}\n")
    sys.__stderr__.flush()


def _inputs(lens, q_len, seed, **kw):
    c = inputs.Case(batch=len(lens), q_len=q_len, seq_lens=lens, seed=seed, **kw)
    return tuple(t.cuda() for t in inputs.make_inputs(c))


def _nhd(k, v):
    return torch.stack([k, v], dim=1).contiguous()


def _hnd(k, v):
    return torch.stack([k, v], dim=1).permute(0, 1, 3, 2, 4).contiguous()


def _oracle(q, k, v, bt, sl, **kw):
    return attention_c64(q.cpu(), k.cpu(), v.cpu(), bt.cpu(), sl.cpu(), k.shape[1], k.shape[2],
                         **kw)


def _flat(q):
    return q.reshape(-1, q.shape[2], q.shape[3])


@pytest.mark.parametrize("q_len", [2, 8, 16])
def test_interleaved_layouts_give_the_same_bits(q_len):
    lens = [1, q_len, 333, 4100]
    q, k, v, bt, sl = _inputs(lens, q_len, seed=500 + q_len)
    base = sqa.paged_mtp_attention(q, k, v, bt, sl, 16, max(lens))
    ws = torch.zeros(WORKSPACE, dtype=torch.uint8, device="cuda")
    for layout, kv in (("NHD", _nhd(k, v)), ("HND", _hnd(k, v))):
        out = fi.xqa_batch_decode_with_kv_cache(_flat(q), kv, ws, bt, sl, max(lens), 128 ** -0.5,
                                                1.0, kv_layout=layout, q_len_per_req=q_len)
        torch.cuda.synchronize()
        assert torch.equal(out.view_as(base), base), layout
    # A (k_cache, v_cache) pair in HND order as well.
    hk = k.transpose(1, 2).contiguous()
    hv = v.transpose(1, 2).contiguous()
    out = fi.trtllm_batch_decode_with_kv_cache(_flat(q), (hk, hv), ws, bt, sl, max(lens),
                                               128 ** -0.5, 1.0, q_len_per_req=q_len)
    assert torch.equal(out.view_as(base), base)
    assert_parity(base, _oracle(q, k, v, bt, sl), label=f"q{q_len}")


def test_every_q_len_up_to_16():
    """Every draft length 1..16 (4 to 64 rows per kv head at GQA 4): one, two and four
    16-row blocks per wave with their padding rows, the causal chain and a random tree,
    on sequences from the draft length itself up to a few pages."""
    ws = torch.zeros(WORKSPACE, dtype=torch.uint8, device="cuda")
    for q_len in range(1, 17):
        lens = [q_len, q_len + 16, 700, 2500 + q_len]
        q, k, v, bt, sl = _inputs(lens, q_len, seed=650 + q_len)
        nhd = _nhd(k, v)
        g = torch.Generator().manual_seed(650 + q_len)
        vis = torch.rand(len(lens), q_len, q_len, generator=g) < 0.4
        vis[:, torch.arange(q_len), torch.arange(q_len)] = True
        tree = pack_draft_mask(vis)
        for mask in (None, tree):
            out = fi.xqa_batch_decode_with_kv_cache(_flat(q), nhd, ws, bt, sl, max(lens),
                                                    128 ** -0.5, 1.0, q_len_per_req=q_len,
                                                    mask=None if mask is None else mask.cuda())
            torch.cuda.synchronize()
            ref = _oracle(q, k, v, bt, sl, draft_mask=mask)
            assert_parity(out.view_as(q), ref,
                          label=f"q{q_len} {'tree' if mask is not None else 'causal'}")


@pytest.mark.parametrize("q_len", [2, 4, 8, 16])
def test_draft_masks(q_len):
    """Causal packed mask = the default chain (same bits); full and random tree masks vs
    the oracle, on sequences shorter than, equal to and far longer than the draft."""
    lens = [max(1, q_len - 1), q_len, 17, 700, 5000]
    q, k, v, bt, sl = _inputs(lens, q_len, seed=600 + q_len)
    nhd = _nhd(k, v)
    ws = torch.zeros(WORKSPACE, dtype=torch.uint8, device="cuda")
    B = len(lens)

    def call(mask, **kw):
        o = fi.xqa_batch_decode_with_kv_cache(_flat(q), nhd, ws, bt, sl, max(lens), 128 ** -0.5,
                                              1.0, q_len_per_req=q_len, mask=mask, **kw)
        torch.cuda.synchronize()
        return o.view_as(q)

    default = call(None)
    assert torch.equal(call(spec_dec_mask(B, q_len, device="cuda")), default)
    full = spec_dec_mask(B, q_len, "full", device="cuda")
    assert_parity(call(full), _oracle(q, k, v, bt, sl, draft_mask=full.cpu()), label="full")
    g = torch.Generator().manual_seed(q_len)
    vis = torch.rand(B, q_len, q_len, generator=g) < 0.4
    vis[:, torch.arange(q_len), torch.arange(q_len)] = True
    tree = pack_draft_mask(vis)
    got = call(tree.cuda())
    assert_parity(got, _oracle(q, k, v, bt, sl, draft_mask=tree), label="tree")
    # Explicit fixed plans (several splits per sequence) agree with the automatic one.
    for ck in (32, 512):
        ns, pps = _lib.plan_splits(0, B, q_len, 32, 8, 128, max(lens), bt.shape[1], ck)
        out = torch.empty_like(q)
        words = torch.from_numpy(tree.numpy().view(np.int32)).cuda()
        wsb = torch.empty(max(1, _lib.workspace_bytes(B, q_len, 32, 8, 128, ns, pps)),
                          dtype=torch.uint8, device="cuda")
        _lib.launch_general(q, out, nhd[:, 0], nhd[:, 1], bt, sl, words, 128 ** -0.5, 1.0, ns,
                            pps, wsb, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert (out.float() - got.float()).abs().max().item() <= 2e-3, ck


def test_scales():
    q_len, lens = 4, [50, 3000]
    q, k, v, bt, sl = _inputs(lens, q_len, seed=700)
    ws = torch.zeros(WORKSPACE, dtype=torch.uint8, device="cuda")
    for s1, s2 in ((0.05, 0.5), (0.2, 2.0), (torch.tensor(0.1), torch.tensor(1.5))):
        out = fi.xqa_batch_decode_with_kv_cache(_flat(q), _nhd(k, v), ws, bt, sl, 3000, s1, s2,
                                                q_len_per_req=q_len)
        ref = _oracle(q, k, v, bt, sl, scale=float(s1), out_scale=float(s2))
        assert_parity(out.view_as(q), ref, label=f"{float(s1)},{float(s2)}")


def _csr(lens, page=16, seed=0, pool_pages=None):
    """Ragged CSR page lists over a shuffled pool, plus the cache pages they index."""
    g = torch.Generator().manual_seed(seed)
    counts = [-(-n // page) for n in lens]
    total = sum(counts)
    pool = pool_pages or 2 * total + 3
    ids = torch.randperm(pool, generator=g)[:total].to(torch.int32)
    indptr = torch.tensor([0] + list(np.cumsum(counts)), dtype=torch.int32)
    last = torch.tensor([(n - 1) % page + 1 if n else 1 for n in lens], dtype=torch.int32)
    return indptr, ids, last, pool


@pytest.mark.parametrize("q_len", [1, 3, 8])
def test_wrappers_over_csr_pages(q_len):
    lens = [q_len, 16, 1000, 37, 4096 + 5]
    indptr, ids, last, pool = _csr(lens, seed=q_len)
    g = torch.Generator().manual_seed(800 + q_len)
    hq, hkv = 32, 8
    kv = torch.randn(pool, 2, 16, hkv, 128, generator=g).half().cuda()
    q = torch.randn(len(lens) * q_len, hq, 128, generator=g).half().cuda()
    bt, sl = fi.csr_to_block_table(indptr, ids, last)
    assert sl.tolist() == lens
    q4 = q.view(len(lens), q_len, hq, 128)
    ref = _oracle(q4, kv[:, 0], kv[:, 1], bt, sl)
    ws = torch.zeros(WORKSPACE, dtype=torch.uint8, device="cuda")

    dec = fi.BatchDecodeWithPagedKVCacheWrapper(ws, "NHD", use_tensor_cores=True)
    dec.plan(indptr.cuda(), ids.cuda(), last.cuda(), hq, hkv, 128, 16, pos_encoding_mode="NONE",
             q_data_type=torch.float16, kv_data_type=torch.float16, q_len_per_req=q_len)
    for _ in range(2):  # plan once, run per layer
        assert_parity(dec.run(q, kv).view_as(q4), ref, label="decode")

    pre = fi.BatchPrefillWithPagedKVCacheWrapper(ws, "NHD")
    qo = torch.arange(0, (len(lens) + 1) * q_len, q_len, dtype=torch.int32, device="cuda")
    pre.plan(qo, indptr.cuda(), ids.cuda(), last.cuda(), hq, hkv, 128, 16, causal=True,
             pos_encoding_mode="NONE", logits_soft_cap=0.0, q_data_type=torch.float16,
             kv_data_type=torch.float16)
    assert_parity(pre.run(q, kv).view_as(q4), ref, label="prefill causal")
    pre.plan(qo, indptr.cuda(), ids.cuda(), last.cuda(), hq, hkv, 128, 16, causal=False)
    full = spec_dec_mask(len(lens), q_len, "full")
    ref_full = _oracle(q4, kv[:, 0], kv[:, 1], bt, sl, draft_mask=full)
    assert_parity(pre.run(q, kv).view_as(q4), ref_full, label="prefill full")

    hnd = kv.permute(0, 1, 3, 2, 4).contiguous()
    dec_h = fi.BatchDecodeWithPagedKVCacheWrapper(ws, "HND")
    dec_h.plan(indptr.cuda(), ids.cuda(), last.cuda(), hq, hkv, 128, 16, q_len_per_req=q_len)
    assert torch.equal(dec_h.run(q, hnd), dec.run(q, kv))


def test_wrapper_run_is_graph_capturable():
    q_len, lens = 8, [3000, 1200, 64]
    indptr, ids, last, pool = _csr(lens, seed=9)
    g = torch.Generator().manual_seed(9)
    kv = torch.randn(pool, 2, 16, 8, 128, generator=g).half().cuda()
    q = torch.randn(len(lens) * q_len, 32, 128, generator=g).half().cuda()
    ws = torch.zeros(WORKSPACE, dtype=torch.uint8, device="cuda")
    dec = fi.BatchDecodeWithPagedKVCacheWrapper(ws, "NHD")
    dec.plan(indptr.cuda(), ids.cuda(), last.cuda(), 32, 8, 128, 16, q_len_per_req=q_len)
    out = torch.empty_like(q)
    eager = dec.run(q, kv).clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        dec.run(q, kv, out=out)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        dec.run(q, kv, out=out)
    for i in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        junk = torch.randn(1 << 20, device="cuda").sum()
        torch.cuda.synchronize()
        del junk


def test_full_size_properties():
    """cfg3 shape (B16 q8 KV 32768): the NHD cache and a causal packed mask give the
    separate-cache bits; a tree mask changes only rows whose draft bits change."""
    case = inputs.baseline_configs()["cfg3"]
    q, k, v, bt, sl = inputs.make_inputs(case, device="cuda", gen_device="cuda")
    base = sqa.paged_mtp_attention(q, k, v, bt, sl, 16, 32768)
    ws = torch.zeros(WORKSPACE, dtype=torch.uint8, device="cuda")
    nhd = _nhd(k, v)
    del k, v
    torch.cuda.empty_cache()
    mask = spec_dec_mask(16, 8, device="cuda")
    out = fi.xqa_batch_decode_with_kv_cache(_flat(q), nhd, ws, bt, sl, 32768, 128 ** -0.5, 1.0,
                                            q_len_per_req=8, mask=mask)
    torch.cuda.synchronize()
    assert torch.equal(out.view_as(base), base)
    vis = torch.tril(torch.ones(8, 8, dtype=torch.bool)).repeat(16, 1, 1)
    vis[3, 5, 2] = False  # sequence 3, row 5 no longer sees draft token 2
    out = fi.xqa_batch_decode_with_kv_cache(_flat(q), nhd, ws, bt, sl, 32768, 128 ** -0.5, 1.0,
                                            q_len_per_req=8, mask=pack_draft_mask(vis).cuda())
    torch.cuda.synchronize()
    out = out.view_as(base)
    changed = (out != base).flatten(2).any(-1)  # [B, Q]
    assert changed[3, 5]
    # Other rows move at most by rounding (the wave's rescale points can shift).
    others = torch.ones_like(changed)
    others[3, 5] = False
    assert (out.float() - base.float()).abs().amax((2, 3))[others].max().item() <= 2e-3
    # Sequence 3 against the oracle with its mask.
    cq, ck, cv, cbt, csl = compact_sequences(q, nhd[:, 0], nhd[:, 1], bt, sl, [3])
    ref = attention_c64(cq, ck, cv, cbt, csl, 16, 8, draft_mask=pack_draft_mask(vis[3:4]))
    assert_parity(out[3:4], ref, label="cfg3 tree row")


def test_workspace_and_argument_checks():
    q, k, v, bt, sl = _inputs([100, 200], 4, seed=1)
    small = torch.zeros(64, dtype=torch.uint8, device="cuda")
    with pytest.raises(ValueError, match="workspace"):
        fi.xqa_batch_decode_with_kv_cache(_flat(q), _nhd(k, v), small, bt, sl, 200, 0.1, 1.0,
                                          q_len_per_req=4)
    with pytest.raises(ValueError, match="window"):
        fi.xqa_batch_decode_with_kv_cache(_flat(q), _nhd(k, v), None, bt, sl, 200, 0.1, 1.0, 8,
                                          q_len_per_req=4)
    with pytest.raises(ValueError, match="rows"):
        fi.xqa_batch_decode_with_kv_cache(_flat(q), _nhd(k, v), None, bt, sl, 200, 0.1, 1.0,
                                          q_len_per_req=2)
    with pytest.raises(ValueError, match="draft mask"):
        fi.xqa_batch_decode_with_kv_cache(_flat(q), _nhd(k, v), None, bt, sl, 200, 0.1, 1.0,
                                          q_len_per_req=4, mask=spec_dec_mask(2, 2).cuda())


def _as_16_token_pages(k, v, bt, page):
    """The same cache memory viewed as 16-token pages: cache page p is 16-token
    pages p * r .. p * r + r - 1 (r = page / 16)."""
    r = page // 16
    k16 = k.view(k.shape[0] * r, 16, k.shape[2], k.shape[3])
    v16 = v.view(v.shape[0] * r, 16, v.shape[2], v.shape[3])
    sub = torch.arange(r, dtype=torch.int32, device=bt.device)
    bt16 = (bt[:, :, None] * r + sub).reshape(bt.shape[0], -1).contiguous()
    return k16, v16, bt16


@pytest.mark.parametrize("page", [32, 64, 128, 256])
@pytest.mark.parametrize("q_len", [2, 8, 16])
def test_larger_cache_pages(page, q_len):
    """32- to 256-token cache pages through the reference boundary and the
    FlashInfer-shaped calls: parity with the oracle, and the same bits as the same
    memory addressed as 16-token pages."""
    lens = [1, q_len, page - 1, page, page + 1, 700, 5000]
    c = inputs.Case(batch=len(lens), q_len=q_len, seq_lens=lens, seed=900 + page + q_len,
                    page_size=page)
    q, k, v, bt, sl = (t.cuda() for t in inputs.make_inputs(c))
    ref = _oracle(q, k, v, bt, sl)
    auto = sqa.paged_mtp_attention(q, k, v, bt, sl, page, max(lens))
    assert_parity(auto, ref, label=f"p{page} auto")
    assert_parity(sqa.forward_v3(q, k, v, bt, sl, page, 128, max(lens)), ref, label="v3 c128")
    assert_parity(sqa.forward_v0(q, k, v, bt, sl, page), ref, label="v0")
    k16, v16, bt16 = _as_16_token_pages(k, v, bt, page)
    assert torch.equal(sqa.paged_mtp_attention(q, k16, v16, bt16, sl, 16, max(lens)), auto)
    ws = torch.zeros(WORKSPACE, dtype=torch.uint8, device="cuda")
    g = torch.Generator().manual_seed(page + q_len)
    vis = torch.rand(len(lens), q_len, q_len, generator=g) < 0.5
    vis[:, torch.arange(q_len), torch.arange(q_len)] = True
    mask = pack_draft_mask(vis)
    out = fi.xqa_batch_decode_with_kv_cache(_flat(q), _hnd(k, v), ws, bt, sl, max(lens),
                                            128 ** -0.5, 1.0, kv_layout="HND",
                                            q_len_per_req=q_len, mask=mask.cuda())
    assert_parity(out.view_as(q), _oracle(q, k, v, bt, sl, draft_mask=mask), label="HND tree")


def test_larger_cache_pages_full_size():
    """cfg3 shape with 64-token pages: the same bits as the 16-token view of the memory."""
    case = inputs.baseline_configs()["cfg3"]
    case.page_size = 64
    q, k, v, bt, sl = inputs.make_inputs(case, device="cuda", gen_device="cuda")
    out64 = sqa.paged_mtp_attention(q, k, v, bt, sl, 64, 32768)
    k16, v16, bt16 = _as_16_token_pages(k, v, bt, 64)
    out16 = sqa.paged_mtp_attention(q, k16, v16, bt16, sl, 16, 32768)
    torch.cuda.synchronize()
    assert torch.isfinite(out64.float()).all()
    assert torch.equal(out64, out16)
    cq, ck, cv, cbt, csl = compact_sequences(q, k16, v16, bt16, sl, [0, 11])
    assert_parity(out64[[0, 11]], attention_c64(cq, ck, cv, cbt, csl, 16, 8), label="cfg3 p64")


def test_buffers_off_the_device_or_misshaped_raise_before_any_launch():
    """Every raw-pointer argument is checked before the launch: host memory, the wrong
    length or a strided view raises ValueError and leaves ``out`` untouched."""
    q_len, lens = 4, [100, 200]
    q, k, v, bt, sl = _inputs(lens, q_len, seed=2)
    ws = torch.zeros(WORKSPACE, dtype=torch.uint8, device="cuda")
    out = torch.full_like(_flat(q), float("nan"))
    mask = spec_dec_mask(2, q_len)
    wide = torch.zeros(2, 2 * bt.shape[1], dtype=torch.int32, device="cuda")
    wide[:, ::2] = bt
    cases = {
        "block_tables on the host": dict(block_tables=bt.cpu()),
        "seq_lens on the host": dict(seq_lens=sl.cpu()),
        "seq_lens shorter than the batch": dict(seq_lens=sl[:1]),
        "strided block_tables": dict(block_tables=wide[:, ::2]),
        "strided seq_lens": dict(seq_lens=torch.stack([sl, sl], 1)[:, 0]),
        "value cache on the host": dict(kv_cache=(k, v.cpu())),
        "mask on the host": dict(mask=mask),
        "workspace on the host": dict(workspace_buffer=ws.cpu()),
        "out on the host": dict(out=out.cpu()),
    }
    for label, change in cases.items():
        args = dict(query=_flat(q), kv_cache=_nhd(k, v), workspace_buffer=ws, block_tables=bt,
                    seq_lens=sl, max_seq_len=200, bmm1_scale=0.1, bmm2_scale=1.0, out=out,
                    q_len_per_req=q_len, mask=mask.cuda())
        args.update(change)
        with pytest.raises(ValueError):
            fi.xqa_batch_decode_with_kv_cache(**args)
        torch.cuda.synchronize()
        assert torch.isnan(out).all(), label


def test_wrapper_plans_host_csr_onto_the_workspace_device():
    """CSR lists on the host (FlashInfer allows it) are moved to the workspace's GPU at
    plan time, so run() reads device memory."""
    q_len, lens = 2, [700, 33, 4000]
    indptr, ids, last, pool = _csr(lens, seed=21)
    g = torch.Generator().manual_seed(21)
    kv = torch.randn(pool, 2, 16, 8, 128, generator=g).half().cuda()
    q = torch.randn(len(lens) * q_len, 32, 128, generator=g).half().cuda()
    ws = torch.zeros(WORKSPACE, dtype=torch.uint8, device="cuda")
    dec = fi.BatchDecodeWithPagedKVCacheWrapper(ws, "NHD")
    dec.plan(indptr, ids, last, 32, 8, 128, 16, q_len_per_req=q_len)
    bt, sl = fi.csr_to_block_table(indptr, ids, last)
    q4 = q.view(len(lens), q_len, 32, 128)
    assert_parity(dec.run(q, kv).view_as(q4), _oracle(q4, kv[:, 0], kv[:, 1], bt, sl))


def test_wrapper_run_scales():
    """run(k_scale=, q_scale=, v_scale=): the first two multiply the softmax scale, the
    last the output (per-tensor FP8 scales in FlashInfer)."""
    q_len, lens = 4, [300, 2000]
    indptr, ids, last, pool = _csr(lens, seed=22)
    g = torch.Generator().manual_seed(22)
    kv = torch.randn(pool, 2, 16, 8, 128, generator=g).half().cuda()
    q = torch.randn(len(lens) * q_len, 32, 128, generator=g).half().cuda()
    ws = torch.zeros(WORKSPACE, dtype=torch.uint8, device="cuda")
    dec = fi.BatchDecodeWithPagedKVCacheWrapper(ws, "NHD")
    dec.plan(indptr.cuda(), ids.cuda(), last.cuda(), 32, 8, 128, 16, q_len_per_req=q_len,
             sm_scale=0.2)
    bt, sl = fi.csr_to_block_table(indptr, ids, last)
    q4 = q.view(len(lens), q_len, 32, 128)
    got = dec.run(q, kv, k_scale=0.5, q_scale=torch.tensor(0.75), v_scale=2.0)
    ref = _oracle(q4, kv[:, 0], kv[:, 1], bt, sl, scale=0.2 * 0.5 * 0.75, out_scale=2.0)
    assert_parity(got.view_as(q4), ref, label="scales")


def test_cuda_graph_wrapper_replans_in_place():
    """use_cuda_graph=True: plan() copies each new plan into buffers fixed by the first, so
    one captured run() serves every later plan (new lengths, new pages), each replay
    checked against the oracle; a plan that changes the batch or outgrows the buffers
    raises."""
    q_len, hq, hkv = 4, 32, 8
    lens_seq = [[900, 40, 2500], [1500, 700, 16], [4000, 4, 333]]
    g = torch.Generator().manual_seed(23)
    pool = 2 * sum(-(-n // 16) for lens in lens_seq for n in lens) + 7
    kv = torch.randn(pool, 2, 16, hkv, 128, generator=g).half().cuda()
    q = torch.randn(3 * q_len, hq, 128, generator=g).half().cuda()
    ws = torch.zeros(WORKSPACE, dtype=torch.uint8, device="cuda")
    indices_buf = torch.zeros(600, dtype=torch.int32, device="cuda")
    dec = fi.BatchDecodeWithPagedKVCacheWrapper(ws, "NHD", use_cuda_graph=True,
                                                paged_kv_indices_buffer=indices_buf)
    csrs = [_csr(lens, seed=30 + i, pool_pages=pool) for i, lens in enumerate(lens_seq)]
    indptr, ids, last, _ = csrs[0]
    dec.plan(indptr, ids, last, hq, hkv, 128, 16, q_len_per_req=q_len)
    out = torch.empty_like(q)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        dec.run(q, kv, out=out)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        dec.run(q, kv, out=out)
    q4 = q.view(3, q_len, hq, 128)
    for rnd in range(2):
        for i, (indptr, ids, last, _) in enumerate(csrs):
            dec.plan(indptr, ids, last, hq, hkv, 128, 16, q_len_per_req=q_len)
            out.fill_(float("nan"))
            graph.replay()
            torch.cuda.synchronize()
            bt, sl = fi.csr_to_block_table(indptr, ids, last)
            assert_parity(out.view_as(q4), _oracle(q4, kv[:, 0], kv[:, 1], bt, sl),
                          label=f"round {rnd} plan {i}")
            junk = torch.randn(1 << 20, device="cuda").sum()  # eager work between replays
            torch.cuda.synchronize()
            del junk
    with pytest.raises(ValueError, match="re-plan"):
        two = _csr([100, 200], seed=40, pool_pages=pool)
        dec.plan(two[0], two[1], two[2], hq, hkv, 128, 16, q_len_per_req=q_len)
    with pytest.raises(ValueError, match="graph buffers"):
        big = _csr([16 * 700, 16, 16], seed=41, pool_pages=pool + 800)
        dec.plan(big[0], big[1], big[2], hq, hkv, 128, 16, q_len_per_req=q_len)
