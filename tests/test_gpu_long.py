"""Long sequences, past the BASELINE configs' 32K keys: one sequence of 256K keys
(16384 pages: the fixed plan's 128 splits of 128 pages), and ragged batches up to
512K keys (32768 pages in one block-table row) where the balanced plan's items
lie inside one sequence for hundreds of pages and pieces cross few, far-apart
sequence starts, and a uniform batch at q_len 16 whose items are paired. Each
against the float32 torch checker (pinned to the C oracle
by ``tests/test_checker_pinned.py``) on the device, a short sequence of the batch
against the float64 C oracle, and the reference's default fixed plan (512-key
chunks) against the automatic one.
"""

import sys

import pytest
import torch

from oracle import attention_c64
from small_q_attention_amd import _lib, cuda as sqa, inputs
from tests._helpers import assert_parity, compact_sequences, torch_fp32_reference

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _announce(request):
    sys.__stderr__.write(f"\n[gpu-test] {request.node.nodeid}\n")
    sys.__stderr__.flush()


CASES = [
    ("one_256k_q8", [262144], 8),
    ("ragged_200k_70k_5k_q16", [200000, 70000, 5000], 16),
    ("ragged_512k_1k_q4", [524288, 1000], 4),
    # uniform and as promised: the 64-row kernel's paired items (items of 64
    # pages, the even ones 2 pages longer) over 4096-page sequences
    ("uniform_2x64k_q16_pairs", [65536, 65536], 16),
]


@pytest.mark.parametrize("label,lens,q_len", CASES, ids=[c[0] for c in CASES])
def test_long_sequences(label, lens, q_len):
    case = inputs.Case(batch=len(lens), q_len=q_len, seq_lens=lens, seed=1900 + q_len)
    tensors = inputs.make_inputs(case, device="cuda", gen_device="cuda")
    q, k, v, bt, sl = tensors
    max_len = max(lens)
    ns, pps = _lib.plan_splits(0, len(lens), q_len, 32, 8, 128, max_len, bt.shape[1], 0)
    print(f"[long] {label}: plan {ns} splits, pages_per_split {pps}", flush=True)
    out = sqa.paged_mtp_attention(*tensors, 16, max_len)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all(), label
    assert_parity(out, torch_fp32_reference(*tensors, 16, 8), label=f"{label} vs torch fp32")
    short = min(range(len(lens)), key=lambda b: lens[b])
    cpu = compact_sequences(*tensors, [short])
    assert_parity(out[[short]], attention_c64(*cpu, 16, 8), label=f"{label} seq {short} vs C")
    if q_len <= 8:
        ref_plan = sqa.forward_v3(*tensors, 16, 512, max_len)
        assert (ref_plan.float() - out.float()).abs().max().item() <= 2e-3, label
    del tensors, q, k, v, bt, sl
    torch.cuda.empty_cache()
