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
    """Same op in torch fp32 on the tensors' device (a second, fast checker).

    Float32 throughout, contiguous operands only. Rows with no visible key are 0.
    Returns a float64 numpy array ``[B, Q, Hq, D]`` (NaN for skipped batches).
    """
    import torch

    n_batch, q_len, hq, dim = query.shape
    group = hq // num_kv_heads
    out = np.full((n_batch, q_len, hq, dim), np.nan)
    for b in (range(n_batch) if batches is None else batches):
        n = int(seq_lens[b])
        if n <= 0:
            out[b] = 0
            continue
        pages = -(-n // page_size)
        ids = block_tables[b, :pages].long()
        k = key_cache.index_select(0, ids).reshape(-1, num_kv_heads, dim)[:n].float()
        v = value_cache.index_select(0, ids).reshape(-1, num_kv_heads, dim)[:n].float()
        qg = query[b].float().reshape(q_len, num_kv_heads, group, dim).permute(1, 0, 2, 3)
        qg = qg.reshape(num_kv_heads, q_len * group, dim).contiguous()
        kt = k.permute(1, 2, 0).contiguous()  # [Hkv, D, L]
        logits = torch.matmul(qg, kt) * (dim ** -0.5)  # [Hkv, Q*G, L]
        vis = n - q_len + torch.arange(q_len, device=query.device) + 1
        vis = vis.repeat_interleave(group)
        mask = torch.arange(n, device=query.device)[None, :] < vis[:, None]
        logits = logits.masked_fill(~mask[None], float("-inf"))
        w = torch.softmax(logits, dim=-1)
        w = torch.nan_to_num(w, nan=0.0)
        o = torch.matmul(w, v.permute(1, 0, 2).contiguous())  # [Hkv, Q*G, D]
        o = o.reshape(num_kv_heads, q_len, group, dim).permute(1, 0, 2, 3).reshape(q_len, hq, dim)
        out[b] = o.double().cpu().numpy()
    return out
