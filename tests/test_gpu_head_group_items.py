"""Items per head group on the GPU: e4m3 caches of 1 KiB token rows (8 kv heads
of 128 dims) at up to 32 rows per kv head, with the expected-page plan. The two
head groups then cut the batch's pages into different numbers of items (the
group reading the slower half of each token row, picked from bit 9 of the K
pool's address, gets the shorter ones), each with its own region of partial
slots, merge table and item size.

Checked against the float64 C oracle with the pools at each combination of 0
and 512 bytes past a 2 MiB boundary (which flips the slower group and the share),
for uniform batches that hold the promise and batches shorter than promised
(the device falls back to the packed plan of each group), at q_len 2 and 8;
repeated calls give the same bits.
"""

import sys

import pytest
import torch

from oracle import attention_c64
from small_q_attention_amd import _lib, inputs
from tests._helpers import assert_parity

pytestmark = pytest.mark.gpu

F8 = torch.float8_e4m3fn
HKV, HQ, HD = 8, 32, 128


@pytest.fixture(autouse=True)
def _announce(request):
    sys.__stderr__.write(f"\n[gpu-test] {request.node.nodeid}\n")
    sys.__stderr__.flush()


def _placed(t, offset):
    """A copy of `t` on the device starting `offset` bytes past a 2 MiB boundary."""
    nbytes = t.numel() * t.element_size()
    raw = torch.empty(nbytes + (4 << 20), dtype=torch.uint8, device="cuda")
    base = (-raw.data_ptr()) % (2 << 20) + offset
    view = raw[base:base + nbytes].view(t.dtype).view(t.shape)
    view.copy_(t.cuda())
    assert view.data_ptr() % (2 << 20) == offset
    return view


@pytest.mark.parametrize("k_off,v_off", [(0, 0), (512, 0), (0, 512), (512, 512)])
@pytest.mark.parametrize("q_len", [2, 8])
def test_head_group_items_at_every_pool_placement(q_len, k_off, v_off):
    promise = 4096
    for label, lens in (("uniform", [promise] * 4), ("shorter", [promise, 3000, promise - 7, 17])):
        case = inputs.Case(batch=len(lens), q_len=q_len, seq_lens=lens,
                           seed=2400 + q_len + k_off // 64 + v_off // 32)
        q, k, v, bt, sl = inputs.make_inputs(case)
        k8, v8 = k.to(F8), v.to(F8)
        ref = attention_c64(q, k8.to(torch.float16), v8.to(torch.float16), bt, sl, 16, HKV)
        kd, vd = _placed(k8, k_off), _placed(v8, v_off)
        qd, btd, sld = q.cuda(), bt.cuda(), sl.cuda()
        ns, pps = _lib.plan_splits(0, len(lens), q_len, HQ, HKV, HD, promise, bt.shape[1], 0)
        assert pps == -(promise // 16), label
        ws = torch.full((_lib.workspace_bytes(len(lens), q_len, HQ, HKV, HD, ns, pps),),
                        0x7F, dtype=torch.uint8, device="cuda")
        outs = []
        for _ in range(2):
            out = torch.full_like(qd, float("nan"))
            _lib.launch_general(qd, out, kd, vd, btd, sld, None, HD ** -0.5, 1.0, ns, pps, ws,
                                torch.cuda.current_stream().cuda_stream)
            torch.cuda.synchronize()
            outs.append(out)
        assert torch.equal(outs[0], outs[1]), label
        assert_parity(outs[0], ref, label=f"{label} q{q_len} K+{k_off} V+{v_off}")
