"""KV caches larger than 4 GiB: pages whose byte offset in the cache lies past
2^32 (a 288 GB GPU holds pools of tens of GB). Each K and V cache here is 6 GiB
(196608 pages of 32 KiB); the block tables take pages from above the 4 GiB
boundary, across it and from below it, and every page no sequence owns holds a
poison value (100), so a page address computed in 32 bits, or any other wrong
page, shows in the output. Automatic plan (balanced), the reference's fixed
512-key plan, and an e4m3 cache of 6 GiB through the FlashInfer-shaped entry,
each against the float64 C oracle over the sequences' own pages.
"""

import sys

import pytest
import torch

from oracle import attention_c64
from small_q_attention_amd import cuda as sqa, decode_api as fi, inputs
from tests._helpers import assert_parity, compact_sequences

pytestmark = pytest.mark.gpu

PAGE_BYTES = 16 * 8 * 128 * 2  # page 16, 8 kv heads, head dim 128, fp16
POOL_PAGES = (6 << 30) // PAGE_BYTES  # 6 GiB per cache
HIGH = (4 << 30) // PAGE_BYTES  # first page wholly past 4 GiB
LENS = [5000, 2300, 777]


@pytest.fixture(autouse=True)
def _announce(request):
    sys.__stderr__.write(f"\n[gpu-test] {request.node.nodeid}\n")
    sys.__stderr__.flush()


def _tables(lens, g):
    """Block tables: sequence 0 above 4 GiB, sequence 1 across it, sequence 2 below."""
    pages = [-(-n // 16) for n in lens]
    spans = [(HIGH + 1000, POOL_PAGES), (HIGH - pages[1] // 2, HIGH + pages[1]), (0, 4096)]
    bt = torch.zeros(len(lens), max(pages), dtype=torch.int32)
    for b, (n, (lo, hi)) in enumerate(zip(pages, spans)):
        bt[b, :n] = (lo + torch.randperm(hi - lo, generator=g)[:n]).to(torch.int32)
    return bt


def _inputs(q_len, dtype=torch.float16):
    g = torch.Generator().manual_seed(2600 + q_len)
    bt = _tables(LENS, g)
    q = torch.randn(len(LENS), q_len, 32, 128, generator=g).to(dtype).cuda()
    k = torch.full((POOL_PAGES, 16, 8, 128), 100.0, dtype=dtype, device="cuda")
    v = torch.full((POOL_PAGES, 16, 8, 128), 100.0, dtype=dtype, device="cuda")
    used = torch.cat([bt[b, :-(-n // 16)] for b, n in enumerate(LENS)]).long().cuda()
    gd = torch.Generator(device="cuda").manual_seed(2700 + q_len)
    k[used] = torch.randn(len(used), 16, 8, 128, generator=gd, device="cuda").to(dtype)
    v[used] = torch.randn(len(used), 16, 8, 128, generator=gd, device="cuda").to(dtype)
    sl = torch.tensor(LENS, dtype=torch.int32, device="cuda")
    return q, k, v, bt.cuda(), sl


@pytest.mark.parametrize("q_len", [2, 8, 16])
def test_pages_past_4gib_fp16(q_len):
    q, k, v, bt, sl = _inputs(q_len)
    assert int(bt.max()) * PAGE_BYTES >= 4 << 30
    print(f"[large-pool] fp16 q{q_len}: caches {k.numel() * 2 >> 30} GiB each, "
          f"highest page {int(bt.max())}", flush=True)
    auto = sqa.paged_mtp_attention(q, k, v, bt, sl, 16, max(LENS))
    fixed = sqa.forward_v3(q, k, v, bt, sl, 16, 512, max(LENS)) if q_len <= 8 else None
    torch.cuda.synchronize()
    cpu = compact_sequences(q, k, v, bt, sl, range(len(LENS)))
    ref = attention_c64(*cpu, 16, 8)
    assert_parity(auto, ref, label=f"auto q{q_len}")
    if fixed is not None:
        assert_parity(fixed, ref, label=f"fixed 512-key plan q{q_len}")
    del q, k, v
    torch.cuda.empty_cache()


@pytest.mark.parametrize("q_len", [4, 16])
def test_pages_past_4gib_e4m3(q_len):
    """An interleaved NHD e4m3 cache ``[P, 2, 16, Hkv, D]`` of 6 GiB: page p's K at
    byte 32 KiB x p, so sequence 0's pages lie past 4 GiB here too (the fp8
    kernels' page addresses)."""
    f8 = torch.float8_e4m3fn
    q, k, v, bt, sl = _inputs(q_len)
    k8, v8 = k.to(f8), v.to(f8)
    del k, v
    torch.cuda.empty_cache()
    kv = torch.stack([k8.view(torch.uint8), v8.view(torch.uint8)], 1).view(f8)
    assert kv.numel() == 2 * POOL_PAGES * 16 * 8 * 128
    print(f"[large-pool] e4m3 q{q_len}: cache {kv.numel() >> 30} GiB", flush=True)
    ws = torch.zeros(64 << 20, dtype=torch.uint8, device="cuda")
    out = fi.xqa_batch_decode_with_kv_cache(q.reshape(-1, 32, 128), kv, ws, bt, sl, max(LENS),
                                            128 ** -0.5, 1.0, q_len_per_req=q_len)
    torch.cuda.synchronize()
    out = out.view_as(q)
    cq, ck, cv, cbt, csl = compact_sequences(q, k8.view(torch.uint8), v8.view(torch.uint8), bt, sl,
                                             range(len(LENS)))
    ref = attention_c64(cq, ck.view(f8).half(), cv.view(f8).half(), cbt, csl, 16, 8)
    assert_parity(out, ref, label=f"e4m3 q{q_len}")
