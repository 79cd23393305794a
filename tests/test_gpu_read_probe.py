"""GPU check of the streaming-read probe (``sqa_read_probe`` of ``read_probe.hip``),
the measurement aid bench.py reports beside the roofline: every dword of the buffer is read exactly
once, by the thread the chunked layout assigns it to. Thread t of workgroup b
folds (xor) the 16-byte elements t, t + 256, ... of chunk b, so the sink equals
an xor-reduction of the buffer viewed as [blocks, rounds, 256, 4] dwords.
"""

import sys

import numpy as np
import pytest
import torch

import read_probe

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _announce(request):
    sys.__stderr__.write(f"\n[gpu-test] {request.node.nodeid}\n")
    sys.__stderr__.flush()


# (workgroups, 16-byte elements per workgroup): tail loop only, unrolled loop
# plus tail, one workgroup per CU.
@pytest.mark.parametrize("blocks,per_block", [(3, 256 * 5), (7, 256 * 19), (256, 256 * 16)])
def test_read_probe_reads_every_dword_once(blocks, per_block):
    g = torch.Generator().manual_seed(blocks)
    n = blocks * per_block * 4
    host = torch.randint(-2 ** 31, 2 ** 31 - 1, (n,), generator=g, dtype=torch.int64)
    host = host.to(torch.int32)
    data = host.cuda()
    sink = torch.full((blocks * 256,), -1, dtype=torch.int32, device="cuda")
    read_probe.read_probe(data, sink, blocks, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    words = host.numpy().view(np.uint32).reshape(blocks, per_block // 256, 256, 4)
    want = np.bitwise_xor.reduce(np.bitwise_xor.reduce(words, axis=3), axis=1).reshape(-1)
    assert np.array_equal(sink.cpu().numpy().view(np.uint32), want)


def test_read_probe_rejects_a_ragged_size():
    data = torch.zeros(4 * 256 + 1, dtype=torch.int32, device="cuda")
    sink = torch.zeros(256, dtype=torch.int32, device="cuda")
    with pytest.raises(RuntimeError, match="multiple"):
        read_probe.read_probe(data, sink, 1, torch.cuda.current_stream().cuda_stream)
