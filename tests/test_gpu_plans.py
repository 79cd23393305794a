"""Split plans on the GPU: the balanced plan's expected page count and the fixed
plan's merge markers.

* ``pages_per_split = -P`` (``sqa_plan_splits`` with a known ``max_seq_len``):
  the kernels assume every sequence spans P pages while the lengths are read
  and fall back to the plan the lengths give when they do not. Uniform, ragged
  and shorter-than-promised batches must give the same bits as the plain
  balanced plan (``pages_per_split = 0``), and parity with the oracle.
* Fixed plans: the merge reads every split of a sequence without its length;
  splits past a sequence's pages write "no keys" and a sequence finished by the
  partial kernel writes "done". A workspace full of NaN (and of the previous
  call's partials) must not leak into the output.
"""

import sys

import pytest
import torch

from oracle import attention_c64
from small_q_attention_amd import _lib, inputs
from tests._helpers import assert_parity

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _announce(request):
    sys.__stderr__.write(f"\n[gpu-test] {request.node.nodeid}\n")
    sys.__stderr__.flush()


def _gpu(case):
    return tuple(t.cuda() for t in inputs.make_inputs(case))


def _oracle(tensors, page=16, hkv=8):
    return attention_c64(*(t.cpu() for t in tensors), page, hkv)


def _run(tensors, ns, pps, fill=float("nan"), ws=None):
    q, k, v, bt, sl = tensors
    nbytes = _lib.workspace_bytes(q.shape[0], q.shape[1], q.shape[2], k.shape[2], q.shape[3],
                                  ns, pps)
    if ws is None:
        ws = torch.full((max(nbytes, 4) // 4,), fill, dtype=torch.float32, device="cuda")
    out = torch.full_like(q, float("nan"))
    _lib.launch(q, k, v, bt, sl, out, ws if nbytes else None, ns, pps,
                torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return out, ws


@pytest.mark.parametrize("q_len", [2, 8, 16])
def test_expected_pages_give_the_plain_balanced_bits(q_len):
    promise = 3000
    batches = {
        "uniform": [promise] * 5,
        "ragged": [promise, promise - 1, 17, 0, promise, q_len],
        "all_shorter": [2000] * 5,
        "one_longer_page": [promise] * 4 + [promise + 16],
    }
    for label, lens in batches.items():
        case = inputs.Case(batch=len(lens), q_len=q_len, seq_lens=lens, seed=1200 + q_len)
        q, k, v, bt, sl = _gpu(case)
        # A block table wider than any sequence (as in serving), so the promise is
        # not capped by the table: "all_shorter" expects more pages than any has,
        # "one_longer_page" has one sequence a page past the promise.
        wide = torch.zeros(len(lens), (promise + 15) // 16 + 2, dtype=torch.int32, device="cuda")
        wide[:, :bt.shape[1]] = bt
        tensors = (q, k, v, wide, sl)
        ns, pps = _lib.plan_splits(0, len(lens), q_len, 32, 8, 128, promise, wide.shape[1], 0)
        assert pps == -((promise + 15) // 16), label
        spec, _ = _run(tensors, ns, pps)
        plain, _ = _run(tensors, ns, 0)
        assert torch.equal(spec, plain), label
        assert_parity(spec, _oracle(tensors), label=f"{label} q{q_len}")


def test_expected_pages_at_full_size():
    """cfg2 (B4 q_len 4 KV 8192, uniform): the expected-page plan against the plain one."""
    case = inputs.baseline_configs()["cfg2"]
    tensors = inputs.make_inputs(case, device="cuda", gen_device="cuda")
    ns, pps = _lib.plan_splits(0, 4, 4, 32, 8, 128, 8192, tensors[3].shape[1], 0)
    assert pps == -512
    spec, _ = _run(tensors, ns, pps)
    plain, _ = _run(tensors, ns, 0)
    assert torch.equal(spec, plain)
    assert torch.isfinite(spec.float()).all()


@pytest.mark.parametrize("q_len", [4, 16])
def test_fixed_plan_merge_markers(q_len):
    """Empty sequences, one-split sequences (finished by the partial kernel) and
    multi-split ones in one fixed plan, over a NaN workspace, then again over the
    first call's leftovers with other lengths."""
    runs = [[0, 5, 16, 17, 700, 4096 + 3], [4096 + 3, 0, 700, 17, 16, q_len]]
    ws = None
    for i, lens in enumerate(runs):
        case = inputs.Case(batch=len(lens), q_len=q_len, seq_lens=lens, seed=1300 + 10 * q_len + i)
        tensors = _gpu(case)
        bt = tensors[3]
        ns, pps = _lib.plan_splits(0, len(lens), q_len, 32, 8, 128, max(lens), bt.shape[1], 256)
        assert pps == 16 and ns > 1
        out, ws = _run(tensors, ns, pps, ws=ws)
        assert torch.isfinite(out.float()).all(), lens
        assert_parity(out, _oracle(tensors), label=f"fixed q{q_len} run {i}")


def _plan_table(ws, tensors, ns):
    """The (first slot, count) table the partial kernel leaves in the workspace
    behind the partial sums and (max, sum) pairs of every slot."""
    q, k = tensors[0], tensors[1]
    batch, q_len, hq, hd = q.shape
    hkv = k.shape[2]
    items = ns * hkv * q_len * (hq // hkv)
    off = items * (hd + 2)
    return ws[off:off + 2 * batch].view(torch.int32).view(batch, 2).cpu().tolist()


# Seam gap of the balanced plan at head dim 128 with 16-bit K/V (four kv heads, a
# 32 KiB page per workgroup): what a second piece costs a workgroup, in pages;
# 8 for the 8-wave kernel of 33..64 rows (q_len 16 at GQA 4).
SEAM_PAGES = 5
SEAM_PAGES_64_ROWS = 8


def _packed_layout(lens, items, page=16, seam=SEAM_PAGES):
    """Brute force from the plan's definition: pages laid end to end in batch order,
    cut into items of P = clamp(ceil(total / items), 4, 2048) pages; the part of
    item i in sequence b goes to slot i + b. In a ragged batch (and when P >= 4 *
    seam), every sequence start off an item boundary of that layout is preceded by
    `seam` empty positions first (unless that needs items over 2048 pages). Returns
    P and each sequence's slots."""
    pages = [(n + page - 1) // page for n in lens]
    start = [sum(pages[:b]) for b in range(len(pages))]
    total = sum(pages)
    P = min(max(-(-total // items), 4), 2048)
    if seam and P >= 4 * seam and any(n != pages[0] for n in pages):
        gaps = [seam if n > 0 and start[b] % P else 0 for b, n in enumerate(pages)]
        vstart = [start[b] + sum(gaps[:b + 1]) for b in range(len(pages))]
        if total + sum(gaps) <= items * 2048:
            start, total = vstart, total + sum(gaps)
            P = min(max(-(-total // items), 4), 2048)
    slots = [sorted({(start[b] + j) // P + b for j in range(n)}) for b, n in enumerate(pages)]
    return P, slots


@pytest.mark.parametrize("q_len", [4, 8, 16])
def test_packed_items_cross_sequences(q_len):
    """Balanced plans with few work items: items span the ends of many sequences
    (dozens of pieces in one workgroup when there are one or two items), sequences
    inside one piece go straight to the output, empty ones are zeros. The table the
    merge reads must match the plan's definition, slots must be distinct and below
    num_splits, and the output must match the oracle; with an expected page count
    (every sequence the same length) the bits must equal the plain plan's."""
    g = torch.Generator().manual_seed(1400 + q_len)
    lens = torch.randint(0, 700, (40,), generator=g).tolist()
    lens[3] = lens[17] = 0
    lens[5], lens[6] = 1, 16
    ragged = _gpu(inputs.Case(batch=len(lens), q_len=q_len, seq_lens=lens, seed=1410 + q_len))
    ref = _oracle(ragged)
    for n_items in (1, 2, 3, 7, 64):
        ns = len(lens) + n_items
        out, ws = _run(ragged, ns, 0)
        assert_parity(out, ref, label=f"ragged items {n_items} q{q_len}")
        assert torch.all(out[3] == 0) and torch.all(out[17] == 0)
        _, slots = _packed_layout(lens, n_items,
                                  seam=SEAM_PAGES_64_ROWS if q_len * 4 > 32 else SEAM_PAGES)
        table = _plan_table(ws, ragged, ns)
        used = []
        for b, (first, count) in enumerate(table):
            assert count == len(slots[b]), (n_items, b)
            if count:
                assert list(range(first, first + count)) == slots[b], (n_items, b)
                used += slots[b]
        assert len(used) == len(set(used)) and max(used) < ns

    same = [333] * 9
    uni = _gpu(inputs.Case(batch=len(same), q_len=q_len, seq_lens=same, seed=1420 + q_len))
    pages = (333 + 15) // 16
    for n_items in (1, 2, 4, 5):
        ns = len(same) + n_items
        spec, ws = _run(uni, ns, -pages)
        plain, _ = _run(uni, ns, 0)
        assert torch.equal(spec, plain), n_items
        _, slots = _packed_layout(same, n_items)
        assert [list(range(f, f + c)) for f, c in _plan_table(ws, uni, ns)] == slots
        assert_parity(spec, _oracle(uni), label=f"uniform items {n_items} q{q_len}")


@pytest.mark.parametrize("qdt,fp8,layout,page,tree,q_len", [
    (torch.bfloat16, False, "HND", 64, True, 8),
    (torch.float16, True, "NHD", 32, True, 16),
    (torch.bfloat16, True, "HND", 256, False, 4),
    (torch.float16, False, "NHD", 128, True, 5),
])
def test_packed_items_through_the_general_entry(qdt, fp8, layout, page, tree, q_len):
    """Items crossing many sequence ends with the general entry's options: bf16
    queries, e4m3 caches, interleaved NHD / HND caches, cache pages of 32 to 256
    tokens (item boundaries inside a cache page) and tree masks (every piece reads
    its own sequence's mask rows), at 1, 3 and 16 work items."""
    from small_q_attention_amd.masks import as_words, pack_draft_mask

    f8 = torch.float8_e4m3fn
    g = torch.Generator().manual_seed(1500 + page + q_len)
    lens = [q_len + int(x) for x in torch.randint(0, 900, (23,), generator=g)]
    lens[4] = q_len
    case = inputs.Case(batch=len(lens), q_len=q_len, seq_lens=lens, seed=1510 + page,
                       page_size=page)
    q, k, v, bt, sl = inputs.make_inputs(case)
    q = q.to(qdt)
    if fp8:
        k, v = k.to(f8), v.to(f8)
        kv = torch.stack([k.view(torch.uint8), v.view(torch.uint8)], 1).view(f8)
    else:
        k, v = k.to(qdt), v.to(qdt)
        kv = torch.stack([k, v], 1)
    if layout == "HND":
        kv = kv.permute(0, 1, 3, 2, 4).contiguous()
        kview, vview = kv[:, 0].transpose(1, 2), kv[:, 1].transpose(1, 2)
    else:
        kv = kv.contiguous()
        kview, vview = kv[:, 0], kv[:, 1]
    kview, vview = kview.cuda(), vview.cuda()
    mask = words = None
    if tree:
        vis = torch.rand(len(lens), q_len, q_len, generator=g) < 0.4
        vis[:, torch.arange(q_len), torch.arange(q_len)] = True
        mask = pack_draft_mask(vis)
        words = as_words(mask, len(lens), q_len).cuda()
    ref = attention_c64(q, k, v, bt, sl, page, 8, draft_mask=mask)
    qd, btd, sld = q.cuda(), bt.cuda(), sl.cuda()
    for n_items in (1, 3, 16):
        ns = len(lens) + n_items
        nbytes = _lib.workspace_bytes(len(lens), q_len, 32, 8, 128, ns, 0)
        ws = torch.full((nbytes // 4,), float("nan"), dtype=torch.float32, device="cuda")
        out = torch.full_like(qd, float("nan"))
        _lib.launch_general(qd, out, kview, vview, btd, sld, words, 128 ** -0.5, 1.0, ns, 0, ws,
                            torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert_parity(out, ref, label=f"{qdt} fp8={fp8} {layout} page{page} tree={tree} "
                                      f"q{q_len} items {n_items}")


def test_balanced_plan_with_no_pages_at_all():
    """Every sequence empty: no work item has a piece, the table counts are all 0
    and the merge writes zeros over a NaN output and workspace (plain plan and the
    expected-page one, whose expectation fails)."""
    lens = [0] * 5
    tensors = _gpu(inputs.Case(batch=5, q_len=4, seq_lens=[16] * 5, seed=1600))
    q, k, v, bt, _ = tensors
    sl = torch.zeros(5, dtype=torch.int32, device="cuda")
    for pps in (0, -1):
        ns = 5 + 7
        out, ws = _run((q, k, v, bt, sl), ns, pps)
        assert torch.all(out == 0), pps
        assert [c for _, c in _plan_table(ws, (q, k, v, bt, sl), ns)] == [0] * len(lens)


@pytest.mark.parametrize("q_len", [2, 4, 8])
def test_pieces_that_fit_the_register_ring(q_len):
    """Fixed plans of 1..4 pages per split and a balanced plan of 4-page items take
    the whole ring in one softmax step (pieces of at most 4 pages at head dim 128):
    pieces of 1..4 pages, partial last pages, the draft block inside the last
    page or spanning two, against the float64 oracle."""
    lens = [q_len, 17, 31, 64, 65, 100, 2 * q_len + 1, 260]
    case = inputs.Case(batch=len(lens), q_len=q_len, seq_lens=lens, seed=1900 + q_len)
    tensors = _gpu(case)
    ref = _oracle(tensors)
    for pps in (1, 2, 3, 4):
        ns = -(-max(-(-n // 16) for n in lens) // pps)
        out, _ = _run(tensors, ns, pps)
        assert_parity(out, ref, label=f"q{q_len} fixed {pps} pages")
    uni = _gpu(inputs.Case(batch=4, q_len=q_len, seq_lens=[1000] * 4, seed=1950 + q_len))
    pages = (1000 + 15) // 16
    ns = 4 + pages  # items of 4 pages (63 pages x 4 sequences over 63 items)
    out, _ = _run(uni, ns, -pages)
    assert_parity(out, _oracle(uni), label=f"q{q_len} balanced 4-page items")
