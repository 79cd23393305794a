"""Shared test helpers: the parity bar and two checkers.

Parity bar (the project's correctness target): fp16 output within ``|a - r| <= 2e-3 + 1e-2 * |r|``
of the oracle rounded to fp16, with max abs error reported as well, and also
measured against the unrounded float64 oracle.
"""

from __future__ import annotations

import numpy as np

TOL_ABS = 2e-3
TOL_REL = 1e-2


def parity_stats(actual, ref64, batches=None):
    """Compare a kernel output (torch fp16 or bf16, any device) with a float64 oracle
    array rounded to the output's type."""
    import torch

    a = actual.detach().float().cpu().numpy().astype(np.float64)
    r = np.asarray(ref64, dtype=np.float64)
    if batches is not None:
        a = a[list(batches)]
        r = r[list(batches)]
    if actual.dtype == torch.bfloat16:
        r16 = torch.from_numpy(r).to(torch.bfloat16).double().numpy()
    else:
        r16 = r.astype(np.float16).astype(np.float64)
    err16 = np.abs(a - r16)
    ok = bool(np.all(err16 <= TOL_ABS + TOL_REL * np.abs(r16)))
    return {
        "ok": ok,
        "finite": bool(np.all(np.isfinite(a))),
        "max_abs_vs_fp16_oracle": float(err16.max()) if err16.size else 0.0,
        "max_abs_vs_f64_oracle": float(np.abs(a - r).max()) if r.size else 0.0,
    }


def assert_parity(actual, ref64, batches=None, label=""):
    st = parity_stats(actual, ref64, batches)
    assert st["finite"], f"{label}: non-finite output"
    assert st["ok"], f"{label}: outside 2e-3 + 1e-2*|r|: {st}"
    return st


def compact_sequences(query, key_cache, value_cache, block_tables, seq_lens, batches, page_size=16):
    """CPU copies of the chosen sequences with only their pages, for the CPU oracles.

    Returns ``(q, k, v, bt, sl)`` where the block table is re-indexed into the
    compacted pool, preserving the token -> page-slot mapping.
    """
    import torch

    qs, ks, vs, rows, lens = [], [], [], [], []
    offset = 0
    max_pages = 1
    for b in batches:
        n = int(seq_lens[b])
        pages = -(-n // page_size)
        ids = block_tables[b, :pages].long()
        ks.append(key_cache.index_select(0, ids).cpu())
        vs.append(value_cache.index_select(0, ids).cpu())
        qs.append(query[b:b + 1].cpu())
        rows.append(torch.arange(offset, offset + pages, dtype=torch.int32))
        lens.append(n)
        offset += pages
        max_pages = max(max_pages, pages)
    bt = torch.zeros(len(batches), max_pages, dtype=torch.int32)
    for i, r in enumerate(rows):
        bt[i, :len(r)] = r
    k = torch.cat(ks) if offset else key_cache[:1].cpu()
    v = torch.cat(vs) if offset else value_cache[:1].cpu()
    return torch.cat(qs), k, v, bt, torch.tensor(lens, dtype=torch.int32)


def torch_fp32_reference(query, key_cache, value_cache, block_tables, seq_lens, page_size,
                         num_kv_heads, batches=None):
    """The float32 torch checker (``small_q_attention_amd.checker.attention_fp32``) on the
    tensors' device; pinned against the float64 C oracle by
    ``tests/test_checker_pinned.py``. Float64 numpy ``[B, Q, Hq, D]`` (NaN for
    skipped batches)."""
    from small_q_attention_amd.checker import attention_fp32

    return attention_fp32(query, key_cache, value_cache, block_tables, seq_lens, page_size,
                          num_kv_heads, batches)
