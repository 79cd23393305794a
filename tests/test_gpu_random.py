"""Seeded random sweep of the general entry point against the float64 C oracle.

Each case draws, from a fixed seed: batch (1-12), draft length, kv heads (1-8)
and GQA group (1-8), head dim (64/128/256), query type (fp16/bf16), cache type
(the query's or e4m3), cache page (16-256 tokens), cache layout (NHD/HND),
causal or random tree mask, softmax and output scales, ragged lengths (from the
draft length itself to a few thousand tokens) and K outliers, and runs
``xqa_batch_decode_with_kv_cache`` (automatic plan); cases the native entry takes
also run through ``paged_mtp_attention`` with a random fixed plan. Bar:
``|a - r| <= 2e-3 + 1e-2 |r|`` against the oracle rounded to the output type.
"""

import os
import random
import sys

import pytest
import torch

from oracle import attention_c64
from small_q_attention_amd import cuda as sqa, decode_api as fi, inputs
from small_q_attention_amd.masks import pack_draft_mask
from tests._helpers import assert_parity

pytestmark = pytest.mark.gpu

F8 = torch.float8_e4m3fn
N_CASES = int(os.environ.get("SQA_RANDOM_CASES", "120"))  # more for a longer sweep


@pytest.fixture(autouse=True)
def _announce(request):
    sys.__stderr__.write(f"\n[gpu-test] {request.node.nodeid}\n")
    sys.__stderr__.flush()


def draw(i):
    rng = random.Random(7000 + i)
    d = rng.choice([64, 128, 128, 256])
    hkv = rng.choice([1, 2, 4, 8])
    group = rng.choice([1, 2, 4, 8])
    max_rows = 32 if d == 256 else 64
    while group > max_rows:
        group //= 2
    q_len = rng.randint(1, min(16, max_rows // group))
    batch = rng.randint(1, 12)
    lens = [rng.choice([q_len, q_len + rng.randint(0, 40), rng.randint(q_len, 3000)])
            for _ in range(batch)]
    qdt = rng.choice([torch.float16, torch.bfloat16])
    return dict(d=d, hkv=hkv, hq=hkv * group, q_len=q_len, lens=lens, qdt=qdt,
                chunk=rng.choice([None, 16, 64, 512, 1 << 20]),
                fp8=rng.random() < 0.3, page=rng.choice([16, 16, 32, 64, 128, 256]),
                layout=rng.choice(["NHD", "HND"]), tree=rng.random() < 0.4,
                s1=d ** -0.5 * rng.uniform(0.5, 2.0), s2=rng.uniform(0.5, 2.0),
                outliers=rng.choice([0.0, 0.05]), seed=8000 + i)


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_case(i):
    p = draw(i)
    label = (f"case {i}: d{p['d']} hq{p['hq']}/hkv{p['hkv']} q{p['q_len']} B{len(p['lens'])} "
             f"{p['qdt']} fp8={p['fp8']} page{p['page']} {p['layout']} tree={p['tree']}")
    sys.__stderr__.write(label + "\n")
    c = inputs.Case(batch=len(p["lens"]), q_len=p["q_len"], seq_lens=p["lens"], seed=p["seed"],
                    num_query_heads=p["hq"], num_kv_heads=p["hkv"], head_dim=p["d"],
                    page_size=p["page"], k_outlier_frac=p["outliers"])
    q, k, v, bt, sl = inputs.make_inputs(c)
    q = q.to(p["qdt"])
    if p["fp8"]:
        k, v = k.to(F8), v.to(F8)
        kv = torch.stack([k.view(torch.uint8), v.view(torch.uint8)], 1).view(F8)
    else:
        k, v = k.to(p["qdt"]), v.to(p["qdt"])
        kv = torch.stack([k, v], 1)
    if p["layout"] == "HND":
        kv = kv.permute(0, 1, 3, 2, 4)
    kv = kv.contiguous().cuda()
    mask = None
    if p["tree"]:
        g = torch.Generator().manual_seed(p["seed"])
        vis = torch.rand(len(p["lens"]), p["q_len"], p["q_len"], generator=g) < 0.4
        vis[:, torch.arange(p["q_len"]), torch.arange(p["q_len"])] = True
        mask = pack_draft_mask(vis)
    ws = torch.zeros(128 << 20, dtype=torch.uint8, device="cuda")
    out = fi.xqa_batch_decode_with_kv_cache(
        q.reshape(-1, p["hq"], p["d"]).cuda(), kv, ws, bt.cuda(), sl.cuda(), max(p["lens"]),
        p["s1"], p["s2"], kv_layout=p["layout"], q_len_per_req=p["q_len"],
        mask=None if mask is None else mask.cuda())
    torch.cuda.synchronize()
    assert out.dtype == p["qdt"]
    ref = attention_c64(q, k, v, bt, sl, p["page"], p["hkv"], draft_mask=mask, scale=p["s1"],
                        out_scale=p["s2"])
    assert_parity(out.view_as(q), ref, label=label)
    # Plain causal cases the native entry takes (q_len 2/4/8/16, 16-bit caches),
    # with a random fixed plan as well.
    if not p["fp8"] and not p["tree"] and p["q_len"] in sqa.SUPPORTED_Q_LENS:
        got = sqa.paged_mtp_attention(q.cuda(), k.cuda(), v.cuda(), bt.cuda(), sl.cuda(),
                                      p["page"], max(p["lens"]), chunk_keys=p["chunk"])
        plain = attention_c64(q, k, v, bt, sl, p["page"], p["hkv"])
        assert_parity(got, plain, label=f"{label} native ck{p['chunk']}")
