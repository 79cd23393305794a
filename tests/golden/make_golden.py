"""Writes the golden fixtures under tests/golden/ (run from the repository root).

    python tests/golden/make_golden.py

Each fixture is an ``.npz`` (no pickles) holding:
* the case description (batch, q_len, seq_lens, seed, page mode) and the
  SHA-256 of the inputs that ``small_q_attention_amd.inputs.make_inputs`` draws
  for it on the CPU, so the generator itself is pinned;
* ``expected_f32``: the float64 C oracle rounded to float32 (tests round it
  to fp16 for the kernel comparison), cross-checked here against the
  vectorized numpy oracle before writing;
* for ``g1_materialized`` the input tensors themselves (one 2-page case).

The expected outputs come from this repository's oracle (``oracle/``), which
``tests/test_oracle_known_answers.py`` pins to the reference's semantics; the
reference ships no golden vectors of its own.
"""

from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import attention_c64, attention_numpy  # noqa: E402
from small_q_attention_amd import inputs  # noqa: E402

HERE = Path(__file__).resolve().parent

CASES = {
    # name: Case kwargs
    "g1_materialized": dict(batch=1, q_len=2, seq_lens=[20], page_mode="shared", seed=101),
    "g2_random_pool": dict(batch=2, q_len=4, seq_lens=[37, 50], seed=102),
    "g3_q16_spans_pages": dict(batch=1, q_len=16, seq_lens=[17], seed=103),
    "g4_ragged_edges": dict(batch=3, q_len=8, seq_lens=[8, 9, 300], seed=104),
    "g5_short_rows": dict(batch=2, q_len=2, seq_lens=[1, 2], seed=105),
    "g6_outliers": dict(batch=1, q_len=8, seq_lens=[129], seed=106, k_outlier_frac=0.05),
}


def input_digest(tensors) -> str:
    h = hashlib.sha256()
    for t in tensors:
        a = t.contiguous().numpy()
        h.update(str(a.dtype).encode())
        h.update(str(a.shape).encode())
        h.update(a.tobytes())
    return h.hexdigest()


def build(name, kw):
    case = inputs.Case(**kw)
    tensors = inputs.make_inputs(case)
    q, k, v, bt, sl = tensors
    c64 = attention_c64(q, k, v, bt, sl, case.page_size, case.num_kv_heads)
    vec = attention_numpy(q, k, v, bt, sl, case.page_size, case.num_kv_heads)
    assert np.abs(c64 - vec).max() < 1e-10, name
    payload = {
        "case_json": np.array(json.dumps(kw, sort_keys=True)),
        "input_sha256": np.array(input_digest(tensors)),
        "expected_f32": c64.astype(np.float32),
    }
    if name == "g1_materialized":
        payload.update({"query": q.numpy(), "key_cache": k.numpy(), "value_cache": v.numpy(),
                        "block_tables": bt.numpy(), "seq_lens": sl.numpy()})
    np.savez_compressed(HERE / f"{name}.npz", **payload)
    return c64


def main():
    for name, kw in CASES.items():
        build(name, kw)
        print("wrote", name)


if __name__ == "__main__":
    main()
