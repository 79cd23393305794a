"""GPU parity of the HIP kernels (through the op boundary and the C ABI) with the oracle.

Restates the reference's GPU correctness drivers
(``/root/reference/scripts/build_and_test_v0.py``..``_v5.py``: kv 33/1024/8192,
reversed page tables, chunk 128/512/1<<20, explicit and measured max_seq_len)
with q_len 16 added, and covers what they leave out: ragged batches on a
scattered 2x pool, rows that see no key, NaN in unused page slots, padding
block-table entries, the golden fixtures, determinism, streams and graph
capture. Bar: ``|a - r| <= 2e-3 + 1e-2 |r|`` against the float64 C oracle
rounded to fp16.
"""

import sys

import numpy as np
import pytest
import torch

from oracle import attention_c64
from small_q_attention_amd import _lib, cuda as sqa, inputs
from tests._helpers import assert_parity, parity_stats
from tests.test_golden import FIXTURES, load_fixture

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _announce(request):
    sys.__stderr__.write(f"\n[gpu-test] {request.node.nodeid}\n")
    sys.__stderr__.flush()


def _to_gpu(tensors):
    return tuple(t.cuda() for t in tensors)


def _oracle(tensors, page=16, hkv=8):
    q, k, v, bt, sl = (t.cpu() for t in tensors)
    return attention_c64(q, k, v, bt, sl, page, hkv)


def _variants(kv_len):
    """(label, callable) pairs covering every forward_vN and chunking the reference drivers use."""
    out = [
        ("v0", lambda *t: sqa.forward_v0(*t, 16)),
        ("v1", lambda *t: sqa.forward_v1(*t, 16, 512)),  # positional 512 lands in verbose
        ("auto", lambda *t: sqa.paged_mtp_attention(*t, 16, kv_len)),
        ("auto_nosync", lambda *t: sqa.paged_mtp_attention(*t, 16)),
    ]
    for ck in (128, 512, 1 << 20):
        out.append((f"v2_c{ck}", lambda *t, ck=ck: sqa.forward_v2(*t, 16, ck)))
    for ck in (128, 512):
        out.append((f"v3_c{ck}", lambda *t, ck=ck: sqa.forward_v3(*t, 16, ck, kv_len)))
        out.append((f"v3_c{ck}_autolen", lambda *t, ck=ck: sqa.forward_v3(*t, 16, ck, 0)))
        out.append((f"v4_c{ck}", lambda *t, ck=ck: sqa.forward_v4(*t, 16, ck, kv_len)))
    for tg in (2, 4):
        out.append((f"v5_tg{tg}", lambda *t, tg=tg: sqa.forward_v5(
            *t, 16, chunk_keys=512, token_group=tg, max_seq_len=kv_len)))
    return out


@pytest.mark.parametrize("q_len", [2, 4, 8, 16])
@pytest.mark.parametrize("kv_len", [33, 1024, 8192])
def test_reference_driver_cases(q_len, kv_len):
    """build_and_test_v0..v5: B=1, reversed pages, every variant and chunking."""
    case = inputs.uniform_case(1, q_len, kv_len, page_mode="shared", seed=99 + q_len + kv_len)
    tensors = _to_gpu(inputs.make_inputs(case))
    ref = _oracle(tensors)
    outs = {}
    for label, fwd in _variants(kv_len):
        outs[label] = fwd(*tensors)
        torch.cuda.synchronize()
        assert_parity(outs[label], ref, label=f"{label} q{q_len} kv{kv_len}")
    # Every variant runs the same kernels; different split plans agree closely.
    base = outs["v0"].float()
    for label, o in outs.items():
        assert (o.float() - base).abs().max().item() <= 2e-3, label


@pytest.mark.parametrize("q_len", [2, 4, 8])
@pytest.mark.parametrize("kv_len", [33, 1024])
def test_reference_v5_unique_pages(q_len, kv_len):
    """build_and_test_v5: batch 2, 'unique' per-request page ranges."""
    case = inputs.uniform_case(2, q_len, kv_len, page_mode="unique", seed=5000 + q_len * 17 + kv_len)
    tensors = _to_gpu(inputs.make_inputs(case))
    ref = _oracle(tensors)
    for tg in ((2,) if q_len == 2 else (2, 4)):
        out = sqa.forward_v5(*tensors, 16, chunk_keys=512, token_group=tg, max_seq_len=kv_len)
        assert_parity(out, ref, label=f"v5 tg{tg}")


@pytest.mark.parametrize("name", FIXTURES)
def test_golden_fixtures(name):
    case, tensors, expected, _ = load_fixture(name)
    tensors = _to_gpu(tensors)
    out = sqa.paged_mtp_attention(*tensors, 16, max(case.seq_lens))
    assert_parity(out, expected.astype(np.float64), label=name)
    out2 = sqa.forward_v2(*tensors, 16, 16)  # one page per split: many splits
    assert_parity(out2, expected.astype(np.float64), label=name + " many splits")


@pytest.mark.parametrize("q_len", [2, 4, 8, 16])
def test_ragged_batch_on_scattered_pool(q_len):
    lens = [1, q_len, q_len + 1, 16, 17, 31, 300, 1000]
    case = inputs.Case(batch=len(lens), q_len=q_len, seq_lens=lens, seed=300 + q_len)
    tensors = _to_gpu(inputs.make_inputs(case))
    ref = _oracle(tensors)
    for ck in (None, 16, 64, 512):
        out = sqa.paged_mtp_attention(*tensors, 16, 1000, chunk_keys=ck)
        st = assert_parity(out, ref, label=f"q{q_len} ck{ck}")
        assert st["max_abs_vs_f64_oracle"] < 2e-3


@pytest.mark.parametrize("q_len", [2, 8, 16])
def test_balanced_plan_on_a_skewed_batch(q_len):
    """The automatic plan for 2..256 sequences (pages_per_split 0): one long sequence
    among empty, tiny and short ones. The batch's pages are cut into equal work items
    on the device from seq_lens; sequences inside one item are written by the partial
    kernel, the rest by the merge, sequences without pages as zeros."""
    lens = [0, 1, q_len - 1, q_len, 16, 17, 200, 37000, 5, 0, 900, 4096]
    case = inputs.Case(batch=len(lens), q_len=q_len, seq_lens=lens, seed=400 + q_len)
    tensors = _to_gpu(inputs.make_inputs(case))
    bt = tensors[3]
    ns, pps = _lib.plan_splits(0, len(lens), q_len, 32, 8, 128, max(lens), bt.shape[1], 0)
    assert pps == -((max(lens) + 15) // 16) and ns > len(lens)  # balanced, expecting the longest
    ref = _oracle(tensors)
    out = sqa.paged_mtp_attention(*tensors, 16, max(lens))
    assert_parity(out, ref, label=f"balanced q{q_len}")
    fixed = sqa.paged_mtp_attention(*tensors, 16, max(lens), chunk_keys=512)
    assert (out.float() - fixed.float()).abs().max().item() <= 2e-3
    assert torch.all(out[0] == 0) and torch.all(out[9] == 0)


def test_single_sequence_automatic_plans():
    """One sequence (the fixed automatic plan; 128 slots per kv-head group on 256
    CUs): splits of at least 4 pages, and past 32 rows per kv head at least 8 once
    the sequence spans more than 256 pages; then parity on one short case of each."""
    def plan(q_len, kv):
        return _lib.plan_splits(0, 1, q_len, 32, 8, 128, kv, kv // 16, 0)
    cus = _lib.load().sqa_device_cu_count(0)
    if cus != 256:
        pytest.skip(f"plan figures below are for 256 CUs (this device: {cus})")
    assert plan(2, 1024) == (16, 4) and plan(2, 8192) == (128, 4)
    assert plan(8, 1024) == (16, 4) and plan(8, 4096) == (64, 4)
    assert plan(8, 8192) == (128, 4) and plan(16, 8192) == (64, 8)
    assert plan(8, 32768) == (128, 16)
    for q_len, kv in ((8, 1000), (16, 4000)):
        case = inputs.Case(batch=1, q_len=q_len, seq_lens=[kv], seed=470 + q_len)
        tensors = _to_gpu(inputs.make_inputs(case))
        assert_parity(sqa.paged_mtp_attention(*tensors, 16, kv), _oracle(tensors),
                      label=f"B1 q{q_len} kv{kv}")


def test_balanced_plan_at_the_batch_limit():
    """256 sequences (the balanced plan's limit; four per lane of the plan's wave)
    and 257 (fixed plan), on a block table wide enough that the 2048-page split cap
    sets the slot count."""
    for batch in (256, 257):
        g = torch.Generator().manual_seed(batch)
        lens = torch.randint(0, 400, (batch,), generator=g).tolist()
        case = inputs.Case(batch=batch, q_len=4, seq_lens=lens, seed=batch)
        q, k, v, bt, sl = inputs.make_inputs(case)
        wide = torch.zeros(batch, 4096, dtype=torch.int32)  # 2x the cap: slots >= 2 * batch
        wide[:, :bt.shape[1]] = bt
        tensors = _to_gpu((q, k, v, wide, sl))
        ns, pps = _lib.plan_splits(0, batch, 4, 32, 8, 128, 0, 4096, 0)
        if batch == 256:
            assert pps == 0 and ns >= batch + batch * 4096 // 2048
        else:
            assert pps > 0
        out = sqa.paged_mtp_attention(*tensors, 16)
        assert_parity(out, _oracle(tensors), label=f"B{batch}")


@pytest.mark.parametrize("hq,hkv,q_len", [
    (8, 8, 4),    # group 1 (MHA)
    (16, 2, 8),   # group 8, one head group with two idle waves
    (32, 1, 2),   # group 32 (MQA): 64 rows on one kv head
    (12, 6, 8),   # second head group with two idle waves
    (24, 3, 4),   # group 8, three kv heads
])
def test_other_head_counts(hq, hkv, q_len):
    """Head layouts beyond the reference's 32/8 on the native entry: the row map
    r = qi * group + g, kv heads that leave waves of a workgroup idle, and all three
    plans (balanced, fixed, single split)."""
    lens = [1, 700, 33, 2900]
    case = inputs.Case(batch=len(lens), q_len=q_len, seq_lens=lens, seed=hq * 10 + hkv,
                       num_query_heads=hq, num_kv_heads=hkv)
    tensors = _to_gpu(inputs.make_inputs(case))
    ref = _oracle(tensors, hkv=hkv)
    for ck in (None, 256, 1 << 20):
        out = sqa.paged_mtp_attention(*tensors, 16, max(lens), chunk_keys=ck)
        assert_parity(out, ref, label=f"hq{hq} hkv{hkv} q{q_len} ck{ck}")
    one = _to_gpu(inputs.make_inputs(inputs.Case(batch=1, q_len=q_len, seq_lens=[5000],
                                                 seed=7, num_query_heads=hq,
                                                 num_kv_heads=hkv)))
    assert_parity(sqa.paged_mtp_attention(*one, 16), _oracle(one, hkv=hkv),
                  label=f"hq{hq} hkv{hkv} B1")


def test_rows_without_visible_keys_are_zero():
    """seq_len < q_len: rows qi < q_len - seq_len see nothing and are written as 0
    (reference v2-v5 merge, csrc/small_q_attention_ext.cu:365); seq_len 0 gives 0."""
    case = inputs.Case(batch=3, q_len=8, seq_lens=[3, 0, 8], seed=11)
    tensors = _to_gpu(inputs.make_inputs(case))
    for ck in (None, 16):
        out = sqa.paged_mtp_attention(*tensors, 16, 8, chunk_keys=ck).float().cpu()
        assert torch.all(out[0, :5] == 0) and torch.all(out[0, 5:].abs().sum(-1) > 0)
        assert torch.all(out[1] == 0)
        assert_parity(out.half(), _oracle(tensors), label=f"ck{ck}")


def test_garbage_outside_the_sequence_is_never_used():
    """NaN in the unused slots of last pages and in the page padding entries point to."""
    case = inputs.Case(batch=3, q_len=4, seq_lens=[20, 33, 47], seed=12)
    q, k, v, bt, sl = inputs.make_inputs(case)
    ref = attention_c64(q, k, v, bt, sl, 16, 8)
    k, v = k.clone(), v.clone()
    nan_page = k.shape[0]
    k = torch.cat([k, torch.full_like(k[:1], float("nan"))])
    v = torch.cat([v, torch.full_like(v[:1], float("nan"))])
    bt = torch.cat([bt, torch.zeros(3, 4, dtype=torch.int32)], 1)
    for b, n in enumerate(sl.tolist()):
        pages = -(-n // 16)
        bt[b, pages:] = nan_page
        last = int(bt[b, pages - 1])
        k[last, n % 16 or 16:] = float("nan")
        v[last, n % 16 or 16:] = float("nan")
    tensors = _to_gpu((q, k, v, bt, sl))
    for ck in (None, 16):
        out = sqa.paged_mtp_attention(*tensors, 16, 0, chunk_keys=ck)
        assert_parity(out, ref, label=f"ck{ck}")


def test_outliers_and_multi_page_drafts():
    for q_len, lens in ((16, [17, 31, 32, 33]), (8, [9, 15, 16, 17])):
        case = inputs.Case(batch=4, q_len=q_len, seq_lens=lens, seed=13 + q_len,
                           k_outlier_frac=0.2, k_outlier_scale=4.0)
        tensors = _to_gpu(inputs.make_inputs(case))
        assert_parity(sqa.paged_mtp_attention(*tensors, 16, max(lens)), _oracle(tensors),
                      label=f"q{q_len}")


def test_deterministic_and_split_plans_agree():
    case = inputs.Case(batch=2, q_len=8, seq_lens=[4000, 2500], seed=14)
    tensors = _to_gpu(inputs.make_inputs(case))
    a = sqa.paged_mtp_attention(*tensors, 16, 4000)
    b = sqa.paged_mtp_attention(*tensors, 16, 4000)
    assert torch.equal(a, b)
    single = sqa.forward_v3(*tensors, 16, 1 << 20, 4000)
    many = sqa.forward_v3(*tensors, 16, 16, 4000)
    assert (single.float() - many.float()).abs().max().item() <= 1e-3
    ref = _oracle(tensors)
    for o in (a, single, many):
        assert_parity(o, ref)


def test_runs_on_the_callers_stream():
    case = inputs.Case(batch=2, q_len=4, seq_lens=[700, 900], seed=15)
    tensors = _to_gpu(inputs.make_inputs(case))
    ref = _oracle(tensors)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        out = sqa.paged_mtp_attention(*tensors, 16, 900)
    side.synchronize()
    assert_parity(out, ref)


def test_graph_capture_and_replay():
    """The op has no host sync and no allocation outside torch's allocator, so it captures.

    Replays several times with eager work in between; every replay must equal the
    eager result bit for bit.
    """
    case = inputs.Case(batch=2, q_len=8, seq_lens=[3000, 1200], seed=16)
    tensors = _to_gpu(inputs.make_inputs(case))
    eager = sqa.paged_mtp_attention(*tensors, 16, 3000)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            sqa.paged_mtp_attention(*tensors, 16, 3000)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out = sqa.paged_mtp_attention(*tensors, 16, 3000)
    for i in range(4):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(static_out, eager), f"replay {i}"
        junk = torch.randn(1 << 20, device="cuda").sum()  # eager work between replays
        torch.cuda.synchronize()
        del junk


def test_custom_op_matches_the_eager_path():
    """Eager calls skip the dispatcher; the registered ``sqa::paged_mtp_attention`` op
    (used under torch.compile/export) runs the same launch and gives the same bits,
    and its fake implementation shapes the output without running anything."""
    case = inputs.Case(batch=3, q_len=8, seq_lens=[900, 40, 2100], seed=19)
    tensors = _to_gpu(inputs.make_inputs(case))
    ns, pps = _lib.plan_splits(0, 3, 8, 32, 8, 128, 2100, tensors[3].shape[1], 0)
    eager = sqa.paged_mtp_attention(*tensors, 16, 2100)
    _lib.custom_op()  # registers the op
    via_op = torch.ops.sqa.paged_mtp_attention(*tensors, ns, pps)
    torch.cuda.synchronize()
    assert torch.equal(eager, via_op)
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode() as mode:
        fakes = [mode.from_tensor(t) for t in tensors]
        shaped = _lib.custom_op()(*fakes, ns, pps)
    assert shaped.shape == eager.shape and shaped.dtype == eager.dtype


def test_c_abi_direct_with_caller_workspace():
    """sqa_paged_mtp_attention through ctypes with a caller-owned workspace and events."""
    case = inputs.Case(batch=3, q_len=4, seq_lens=[500, 64, 1500], seed=17)
    tensors = _to_gpu(inputs.make_inputs(case))
    q, k, v, bt, sl = tensors
    ns, pps = _lib.plan_splits(0, 3, 4, 32, 8, 128, 1500, bt.shape[1], 256)
    assert ns > 1
    ws = torch.empty(_lib.workspace_bytes(3, 4, 32, 8, 128, ns, pps), dtype=torch.uint8, device="cuda")
    out = torch.empty_like(q)
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    for e in evs:
        e.record()
    _lib.launch(q, k, v, bt, sl, out, ws, ns, pps, torch.cuda.current_stream().cuda_stream,
                timing_events=[e.cuda_event for e in evs])
    torch.cuda.synchronize()
    assert evs[0].elapsed_time(evs[1]) > 0
    assert_parity(out, _oracle(tensors))
    small = torch.empty(16, dtype=torch.uint8, device="cuda")
    with pytest.raises(RuntimeError, match="workspace"):
        _lib.launch(q, k, v, bt, sl, out, small, ns, pps, 0)


@pytest.mark.parametrize("batch,kv,q_len", [(1, 8192, 2), (4, 2048, 8), (16, 600, 4)])
def test_output_only_8_byte_aligned(batch, kv, q_len):
    """The C ABI asks for an 8-byte aligned output: the merge (and the partial
    kernel's direct rows) store 8 bytes at a time, so an output 8 bytes past a
    16-byte boundary gets the same bits as an aligned one."""
    case = inputs.uniform_case(batch, q_len, kv, seed=5300 + batch)
    q, k, v, bt, sl = _to_gpu(inputs.make_inputs(case))
    ns, pps = _lib.plan_splits(0, batch, q_len, 32, 8, 128, kv, bt.shape[1], 0)
    ws = torch.empty(max(1, _lib.workspace_bytes(batch, q_len, 32, 8, 128, ns, pps)),
                     dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    aligned = torch.empty_like(q)
    _lib.launch(q, k, v, bt, sl, aligned, ws, ns, pps, stream)
    buf = torch.full((q.numel() + 4,), float("nan"), dtype=q.dtype, device="cuda")
    shifted = buf[4:].view_as(q)
    assert shifted.data_ptr() % 16 == 8
    _lib.launch(q, k, v, bt, sl, shifted, ws, ns, pps, stream)
    torch.cuda.synchronize()
    assert torch.equal(shifted, aligned)
    assert torch.isnan(buf[:4]).all()  # nothing written before the output


def test_parity_stats_flags_a_planted_mistake():
    """The checker itself: an oracle off by one visible key fails the bar."""
    case = inputs.Case(batch=1, q_len=4, seq_lens=[40], seed=18)
    tensors = _to_gpu(inputs.make_inputs(case))
    out = sqa.paged_mtp_attention(*tensors, 16, 40)
    q, k, v, bt, sl = (t.cpu() for t in tensors)
    wrong = attention_c64(q, k, v, bt, sl - 1, 16, 8)  # every row sees one key less
    assert not parity_stats(out, wrong)["ok"]


def test_one_pass_fast_path_matches_the_checked_path(monkeypatch):
    """``forward_v0..v5`` and the native entry check a valid fp16 call in one pass
    before launching: the result must be bit-equal to the fully checked path's, the
    full checks must not run for it, and invalid GPU inputs must still raise the
    reference's errors."""
    case = inputs.Case(batch=3, q_len=4, seq_lens=[700, 33, 1500], seed=1500)
    q, k, v, bt, sl = inputs.make_inputs(case, device="cuda")
    sqa.forward_v3(q, k, v, bt, sl, 16)  # first call: library loaded, GPU seen
    checked = {
        "v0": sqa.load_v0().forward(q, k, v, bt, sl, 16),
        "v2": sqa.load_v2().forward_v2(q, k, v, bt, sl, 16, 256),
        "v3": sqa.load_v3().forward_v3(q, k, v, bt, sl, 16, 512, 1500),
        "v5": sqa.load_v5().forward_v5(q, k, v, bt, sl, 16, None, 4, 0),
        "native": sqa._run(q, k, v, bt, sl, 16, None, 1500),
    }

    def no_full_checks(*args, **kwargs):
        raise AssertionError("the full checks ran for a valid call")

    with monkeypatch.context() as m:
        m.setattr(sqa, "_check_python_contract", no_full_checks)
        m.setattr(sqa, "_check_launcher_contract", no_full_checks)
        fast = {
            "v0": sqa.forward_v0(q, k, v, bt, sl, 16),
            "v2": sqa.forward_v2(q, k, v, bt, sl, 16, 256),
            "v3": sqa.forward_v3(q, k, v, bt, sl, 16, 512, 1500),
            "v5": sqa.forward_v5(q, k, v, bt, sl, 16, None, 4),
            "native": sqa.paged_mtp_attention(q, k, v, bt, sl, 16, 1500),
        }
    for name in checked:
        assert torch.equal(fast[name], checked[name]), name
    assert_parity(fast["v3"], _oracle((q, k, v, bt, sl)), label="fast path v3")
    with pytest.raises(ValueError):
        sqa.forward_v3(q.transpose(1, 2).contiguous().transpose(1, 2), k, v, bt, sl, 16)
    with pytest.raises(ValueError):
        sqa.forward_v3(q.bfloat16(), k, v, bt, sl, 16)
    with pytest.raises(ValueError):
        sqa.forward_v3(q[:, :, :16].contiguous(), k, v, bt, sl, 16)  # GQA group 2
    with pytest.raises(ValueError):
        sqa.forward_v5(q, k, v, bt, sl, 16, 512, 3)
    with pytest.raises(RuntimeError):
        sqa.forward_v3(q, k, v, bt, sl.long(), 16)
    with pytest.raises(RuntimeError):
        sqa.forward_v0(q, k, v[:-1], bt, sl, 16)
