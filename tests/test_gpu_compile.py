"""The op boundary under ``torch.compile`` with ``fullgraph=True`` (no graph break
allowed) and under ``torch.export``: the checks trace as guards and the graph calls
the ``sqa::paged_mtp_attention_planned`` custom op, which plans the splits at run
time; its output must equal the eager call's bit for bit wherever the plan is the
same (a known ``max_seq_len``, or the whole block-table row), and pass the parity
bar where the eager call measures ``max_seq_len`` with a host sync (the traced call
plans over the row instead). With ``dynamic=True`` one graph serves every batch
size. Backends ``eager`` and ``aot_eager`` (no code generation: the graph is the op
between torch's own tensor ops).
"""

import sys

import pytest
import torch

from small_q_attention_amd import cuda as sqa, inputs
from tests._helpers import torch_fp32_reference, assert_parity

pytestmark = pytest.mark.gpu

CASE = inputs.Case(batch=3, q_len=8, seq_lens=[900, 40, 2100], seed=19)


@pytest.fixture(autouse=True)
def _announce(request):
    sys.__stderr__.write(f"\n[gpu-test] {request.node.nodeid}\n")
    sys.__stderr__.flush()
    torch._dynamo.reset()
    yield
    torch._dynamo.reset()


def _tensors(seed=19, seq_lens=None):
    lens = CASE.seq_lens if seq_lens is None else seq_lens
    c = inputs.Case(batch=len(lens), q_len=CASE.q_len, seq_lens=lens, seed=seed)
    return tuple(t.cuda() for t in inputs.make_inputs(c))


# (name, call): each call's eager plan is the one its traced call computes, except
# forward_v2, whose eager call measures max_seq_len.
CALLS = [
    ("native", lambda q, k, v, bt, sl: sqa.paged_mtp_attention(q, k, v, bt, sl, 16, 2100)),
    ("native_row", lambda q, k, v, bt, sl: sqa.paged_mtp_attention(q, k, v, bt, sl, 16)),
    ("v0", lambda q, k, v, bt, sl: sqa.forward_v0(q, k, v, bt, sl, 16)),
    ("v1", lambda q, k, v, bt, sl: sqa.forward_v1(q, k, v, bt, sl, 16)),
    ("v3", lambda q, k, v, bt, sl: sqa.forward_v3(q, k, v, bt, sl, 16, 512, 2100)),
    ("v4_auto", lambda q, k, v, bt, sl: sqa.forward_v4(q, k, v, bt, sl, 16, None, 2100)),
    ("v5", lambda q, k, v, bt, sl: sqa.forward_v5(q, k, v, bt, sl, 16, 512, 2, 2100)),
]


@pytest.mark.parametrize("backend", ["eager", "aot_eager"])
@pytest.mark.parametrize("name,call", CALLS, ids=[c[0] for c in CALLS])
def test_compile_fullgraph_equals_eager(name, call, backend):
    t = _tensors()
    eager = call(*t)
    compiled = torch.compile(call, backend=backend, fullgraph=True)
    got = compiled(*t)
    torch.cuda.synchronize()
    assert torch.equal(got, eager), name
    # Other inputs of the same shapes reuse the graph and follow their own data.
    t2 = _tensors(seed=23)
    got2 = compiled(*t2)
    torch.cuda.synchronize()
    assert torch.equal(got2, call(*t2)), name


def test_compile_fullgraph_measured_max_seq_len_plans_over_the_row():
    """forward_v2 measures max_seq_len eagerly (a host sync); traced, it plans over
    the block-table row: same keys, the merge's order differs, within the bar."""
    t = _tensors()
    call = lambda q, k, v, bt, sl: sqa.forward_v2(q, k, v, bt, sl, 16, 512)  # noqa: E731
    eager = call(*t)
    got = torch.compile(call, backend="aot_eager", fullgraph=True)(*t)
    torch.cuda.synchronize()
    ref = torch_fp32_reference(*t, 16, 8)
    assert_parity(got, ref, label="traced v2")
    assert (got.float() - eager.float()).abs().max().item() <= 2e-3


def test_compile_dynamic_batch_with_one_graph():
    """dynamic=True: batches of 2, 3 and 5 sequences (other lengths, block-table
    widths and pools) through one compiled frame, each equal to its eager call."""
    from torch._dynamo.testing import CompileCounter

    counter = CompileCounter()
    call = lambda q, k, v, bt, sl: sqa.paged_mtp_attention(q, k, v, bt, sl, 16, 3000)  # noqa: E731
    compiled = torch.compile(call, backend=counter, fullgraph=True, dynamic=True)
    for seed, lens in ((31, [3000, 700]), (32, [1200, 16, 2999]),
                       (33, [50, 3000, 800, 2048, 9])):
        t = _tensors(seed, lens)
        got = compiled(*t)
        torch.cuda.synchronize()
        assert torch.equal(got, call(*t)), lens
    assert counter.frame_count == 1, counter.frame_count


def test_compile_with_torch_ops_around_the_call():
    """The op inside a larger compiled function (a scaled query in, a reduction out)."""
    t = _tensors()

    def step(q, k, v, bt, sl):
        out = sqa.paged_mtp_attention(q * 0.5, k, v, bt, sl, 16, 2100)
        return out.float().square().sum(dim=-1)

    got = torch.compile(step, backend="aot_eager", fullgraph=True)(*t)
    torch.cuda.synchronize()
    assert torch.equal(got, step(*t))


def test_export_holds_the_custom_op():
    t = _tensors()

    class Attention(torch.nn.Module):
        def forward(self, q, k, v, bt, sl):
            return sqa.paged_mtp_attention(q, k, v, bt, sl, 16, 2100)

    ep = torch.export.export(Attention(), t)
    targets = [str(n.target) for n in ep.graph.nodes if n.op == "call_function"]
    assert any("sqa.paged_mtp_attention" in x for x in targets), targets
    got = ep.module()(*t)
    torch.cuda.synchronize()
    assert torch.equal(got, sqa.paged_mtp_attention(*t, 16, 2100))


def _cache(k, v, layout):
    """Interleaved ``[P, 2, 16, Hkv, D]`` (NHD) or ``[P, 2, Hkv, 16, D]`` (HND) from
    ``[P, 16, Hkv, D]`` K and V (e4m3 stacked through their bytes)."""
    f8 = torch.float8_e4m3fn
    if layout == "HND":
        k, v = k.transpose(1, 2), v.transpose(1, 2)
    if k.dtype == f8:
        return torch.stack([k.view(torch.uint8), v.view(torch.uint8)], 1).contiguous().view(f8)
    return torch.stack([k, v], 1).contiguous()


@pytest.mark.parametrize("layout,kv_dtype,qdt,tree,with_out", [
    ("NHD", "fp16", torch.float16, False, False),
    ("HND", "e4m3", torch.float16, True, False),
    ("NHD", "bf16", torch.bfloat16, False, True),
], ids=["nhd_fp16", "hnd_e4m3_tree", "nhd_bf16_out"])
def test_compile_fullgraph_xqa_decode(layout, kv_dtype, qdt, tree, with_out):
    """The FlashInfer-shaped call traced into ``sqa::paged_attention_planned``: equal
    to the eager call (the workspace's contents never matter)."""
    from small_q_attention_amd import decode_api as fi
    from small_q_attention_amd.masks import pack_draft_mask

    q, k, v, bt, sl = _tensors()
    q = q.to(qdt)
    if kv_dtype == "e4m3":
        k, v = k.to(torch.float8_e4m3fn), v.to(torch.float8_e4m3fn)
    elif kv_dtype == "bf16":
        k, v = k.to(torch.bfloat16), v.to(torch.bfloat16)
    kv = _cache(k, v, layout)
    b, q_len = q.shape[0], q.shape[1]
    mask = None
    if tree:
        g = torch.Generator().manual_seed(5)
        vis = torch.rand(b, q_len, q_len, generator=g) < 0.5
        vis[:, torch.arange(q_len), torch.arange(q_len)] = True
        mask = pack_draft_mask(vis).cuda()
    qf = q.reshape(b * q_len, 32, 128)
    ws = torch.zeros(64 << 20, dtype=torch.uint8, device="cuda")

    def decode(qf, kv, bt, sl, out):
        return fi.xqa_batch_decode_with_kv_cache(qf, kv, ws, bt, sl, 2100, 128 ** -0.5, 0.75,
                                                 kv_layout=layout, q_len_per_req=q_len,
                                                 mask=mask, out=out)

    out_e = torch.empty_like(qf) if with_out else None
    eager = decode(qf, kv, bt, sl, out_e)
    out_c = torch.full_like(qf, float("nan")) if with_out else None
    got = torch.compile(decode, backend="aot_eager", fullgraph=True)(qf, kv, bt, sl, out_c)
    torch.cuda.synchronize()
    assert torch.equal(got, eager)
    if with_out:
        assert torch.equal(out_c, eager)


def test_compile_fullgraph_wrapper_run():
    """A planned decode wrapper's run() traced: equal to its eager run()."""
    from small_q_attention_amd import decode_api as fi

    lens = [3000, 1200, 64]
    q_len, hq, hkv = 8, 32, 8
    counts = [-(-n // 16) for n in lens]
    g = torch.Generator().manual_seed(9)
    pool = 2 * sum(counts) + 3
    ids = torch.randperm(pool, generator=g)[:sum(counts)].to(torch.int32).cuda()
    indptr = torch.tensor([0] + [sum(counts[:i + 1]) for i in range(len(counts))],
                          dtype=torch.int32).cuda()
    last = torch.tensor([(n - 1) % 16 + 1 for n in lens], dtype=torch.int32).cuda()
    kv = torch.randn(pool, 2, 16, hkv, 128, generator=g).half().cuda()
    q = torch.randn(len(lens) * q_len, hq, 128, generator=g).half().cuda()
    ws = torch.zeros(64 << 20, dtype=torch.uint8, device="cuda")
    dec = fi.BatchDecodeWithPagedKVCacheWrapper(ws, "NHD")
    dec.plan(indptr, ids, last, hq, hkv, 128, 16, q_len_per_req=q_len)
    eager = dec.run(q, kv)
    got = torch.compile(lambda q, kv: dec.run(q, kv), backend="aot_eager", fullgraph=True)(q, kv)
    torch.cuda.synchronize()
    assert torch.equal(got, eager)
