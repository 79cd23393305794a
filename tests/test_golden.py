"""CPU checks of the committed golden fixtures (``tests/golden/*.npz``).

The input generator must still reproduce each fixture's inputs bit for bit
(SHA-256), and all three CPU oracles must reproduce the stored outputs. The
GPU side of the same fixtures is in ``tests/test_gpu_parity.py``.
"""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import attention_c64, attention_numpy, paged_mtp_attention_reference
from small_q_attention_amd import inputs

GOLDEN = Path(__file__).resolve().parent / "golden"
FIXTURES = sorted(p.stem for p in GOLDEN.glob("*.npz"))


def load_fixture(name):
    """Returns (case, tensors on CPU, expected float32 array, stored sha)."""
    data = np.load(GOLDEN / f"{name}.npz", allow_pickle=False)
    kw = json.loads(str(data["case_json"]))
    case = inputs.Case(**kw)
    if "query" in data:
        tensors = tuple(torch.from_numpy(data[k]) for k in
                        ("query", "key_cache", "value_cache", "block_tables", "seq_lens"))
    else:
        tensors = inputs.make_inputs(case)
    return case, tensors, data["expected_f32"], str(data["input_sha256"])


def test_fixture_set_is_present():
    assert len(FIXTURES) >= 6


@pytest.mark.parametrize("name", FIXTURES)
def test_generator_reproduces_fixture_inputs(name):
    from tests.golden.make_golden import input_digest

    case, tensors, _, sha = load_fixture(name)
    assert input_digest(inputs.make_inputs(case)) == sha
    assert input_digest(tensors) == sha


@pytest.mark.parametrize("name", FIXTURES)
def test_oracles_reproduce_fixture_outputs(name):
    case, (q, k, v, bt, sl), expected, _ = load_fixture(name)
    c64 = attention_c64(q, k, v, bt, sl, case.page_size, case.num_kv_heads)
    vec = attention_numpy(q, k, v, bt, sl, case.page_size, case.num_kv_heads)
    np.testing.assert_allclose(c64, expected, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(vec, expected, rtol=1e-6, atol=1e-7)
    if min(case.seq_lens) >= case.q_len:  # the loop oracle raises otherwise (reference.py:52-53)
        loop = paged_mtp_attention_reference(q.float(), k.float(), v.float(), bt, sl,
                                             case.page_size, case.num_kv_heads)
        np.testing.assert_allclose(loop.numpy(), expected, rtol=1e-4, atol=2e-6)
    else:
        with pytest.raises(ValueError):
            paged_mtp_attention_reference(q.float(), k.float(), v.float(), bt, sl,
                                          case.page_size, case.num_kv_heads)
