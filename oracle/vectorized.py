"""Vectorized numpy restatement of the reference oracle.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Same mathematics as ``/root/reference/src/small_q_attention/reference.py:46-72``
(scale ``D**-0.5``, GQA map ``qh // group``, row ``qi`` sees the first
``seq_len - q_len + qi + 1`` tokens, softmax then V), batched per sequence so
it finishes full BASELINE sizes in seconds. Computes in float64 by default;
``dtype=np.float32`` mirrors the reference's fp32 callers.
"""

from __future__ import annotations

import numpy as np


def _np(x):
    """Accept torch tensors or numpy arrays; returns a numpy view/copy on CPU."""
    if hasattr(x, "detach"):
        x = x.detach()
        if x.device.type != "cpu":
            x = x.cpu()
        return x.numpy()
    return np.asarray(x)


def gather_sequence(key_cache, value_cache, block_row, length, page_size):
    """Return the first ``length`` tokens of one sequence as ``[length, Hkv, D]``.

    Token ``t`` is read from page ``block_row[t // page_size]`` at slot
    ``t % page_size`` (``reference.py:54-59``; ``docs/kernel_design.md:19-24``).
    """
    kc, vc, row = _np(key_cache), _np(value_cache), _np(block_row)
    pages_used = -(-int(length) // page_size)
    ids = row[:pages_used].astype(np.int64)
    hkv, dim = kc.shape[2], kc.shape[3]
    k = kc[ids].reshape(-1, hkv, dim)[:length]
    v = vc[ids].reshape(-1, hkv, dim)[:length]
    return k, v


def attention_numpy(query, key_cache, value_cache, block_tables, seq_lens, page_size,
                    num_kv_heads, dtype=np.float64, batches=None):
    """Paged MTP attention; returns ``[B, Q, Hq, D]`` in ``dtype``.

    ``batches`` optionally restricts the computation to a subset of sequence
    indices (the others are left as NaN), which lets tests check a sample of
    a full-size batch. Rows whose visible-key count is <= 0 are returned as 0
    (the reference raises for them instead; callers that want the raise use
    :func:`oracle.paged_mtp_attention_reference`).
    """
    q = _np(query).astype(dtype)
    bt, sl = _np(block_tables), _np(seq_lens)
    n_batch, q_len, n_qheads, dim = q.shape
    group = n_qheads // num_kv_heads
    scale = dtype(dim ** -0.5)
    out = np.full(q.shape, np.nan, dtype=dtype)
    for b in (range(n_batch) if batches is None else batches):
        length = int(sl[b])
        if length <= 0:
            out[b] = 0
            continue
        k, v = gather_sequence(key_cache, value_cache, bt[b], length, page_size)
        k = k.astype(dtype)  # [L, Hkv, D]
        v = v.astype(dtype)
        # qg: [Hkv, Q*G, D], rows ordered (qi, g).
        qg = q[b].reshape(q_len, num_kv_heads, group, dim).transpose(1, 0, 2, 3)
        qg = qg.reshape(num_kv_heads, q_len * group, dim)
        logits = np.matmul(qg, k.transpose(1, 2, 0)) * scale  # [Hkv, Q*G, L]
        visible = length - q_len + np.arange(q_len) + 1  # [Q]
        vis_rows = np.repeat(visible, group)  # [Q*G]
        mask = np.arange(length)[None, :] < vis_rows[:, None]  # [Q*G, L]
        logits = np.where(mask[None], logits, -np.inf)
        peak = logits.max(axis=-1, keepdims=True)
        peak = np.where(np.isfinite(peak), peak, 0)
        w = np.exp(logits - peak)
        denom = w.sum(axis=-1, keepdims=True)
        o = np.matmul(w, v.transpose(1, 0, 2))  # [Hkv, Q*G, D]
        o = np.where(denom > 0, o / np.where(denom > 0, denom, 1), 0)
        o = o.reshape(num_kv_heads, q_len, group, dim).transpose(1, 0, 2, 3)
        out[b] = o.reshape(q_len, n_qheads, dim)
    return out
