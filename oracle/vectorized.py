"""Vectorized numpy restatement of the reference oracle.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Same mathematics as ``/root/reference/src/small_q_attention/reference.py:46-72``
(scale ``D**-0.5``, GQA map ``qh // group``, row ``qi`` sees the first
``seq_len - q_len + qi + 1`` tokens, softmax then V), batched per sequence so
it finishes full benchmark sizes in seconds. Computes in float64 by default;
``dtype=np.float32`` mirrors the reference's fp32 callers.
"""

from __future__ import annotations

import numpy as np


def _np(x):
    """Accept torch tensors or numpy arrays; returns a numpy view/copy on CPU
    (bfloat16, which numpy lacks, is widened exactly to float32)."""
    if hasattr(x, "detach"):
        x = x.detach()
        if x.device.type != "cpu":
            x = x.cpu()
        if str(x.dtype) in ("torch.bfloat16", "torch.float8_e4m3fn"):
            x = x.float()
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


def unpack_draft_mask(mask, q_len):
    """Packed speculative-decoding mask -> bool ``[B, Q, Q]`` (row qi sees draft token j).

    The packing is the one of the reference's FlashInfer comparisons
    (``/root/reference/scripts/run_flashinfer_baseline.py:56-85``): per row,
    ``ceil(Q / 32)`` little-endian uint32 words, bit ``j % 32`` of word ``j // 32``
    for draft token j, stored as twice as many uint16 (or as the uint32 / int32
    words themselves).
    """
    m = np.ascontiguousarray(_np(mask))
    if m.dtype in (np.uint16, np.int16):
        m = m.view(np.uint16).reshape(m.shape[:-1] + (m.shape[-1] // 2, 2))
        words = m[..., 0].astype(np.uint64) | (m[..., 1].astype(np.uint64) << np.uint64(16))
    else:
        words = m.view(np.uint32).astype(np.uint64)
    j = np.arange(q_len)
    bits = (words[..., j // 32] >> (j % 32).astype(np.uint64)) & np.uint64(1)
    return bits.astype(bool)


def attention_numpy(query, key_cache, value_cache, block_tables, seq_lens, page_size,
                    num_kv_heads, dtype=np.float64, batches=None, draft_mask=None, scale=None,
                    out_scale=1.0):
    """Paged MTP attention; returns ``[B, Q, Hq, D]`` in ``dtype``.

    ``batches`` optionally restricts the computation to a subset of sequence
    indices (the others are left as NaN), which lets tests check a sample of
    a full-size batch. Rows whose visible-key count is <= 0 are returned as 0
    (the reference raises for them instead; callers that want the raise use
    :func:`oracle.paged_mtp_attention_reference`).

    ``draft_mask`` (packed, see :func:`unpack_draft_mask`, or bool ``[B, Q, Q]``)
    replaces the causal draft chain: token ``t`` of a sequence of length ``L`` is
    seen by row qi when ``t < L - Q`` or when draft token ``j = t - (L - Q)`` is
    marked for that row. ``scale`` (default ``D**-0.5``) scales the logits,
    ``out_scale`` the output. Key and value caches may be any-stride
    ``[P, page, Hkv, D]`` views (e.g. the halves of an interleaved cache).
    """
    q = _np(query).astype(dtype)
    bt, sl = _np(block_tables), _np(seq_lens)
    n_batch, q_len, n_qheads, dim = q.shape
    group = n_qheads // num_kv_heads
    scale = dtype(dim ** -0.5) if scale is None else dtype(scale)
    if draft_mask is not None:
        dm = _np(draft_mask)
        if dm.dtype != bool:
            dm = unpack_draft_mask(dm, q_len)
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
        if draft_mask is None:
            visible = length - q_len + np.arange(q_len) + 1  # [Q]
            vis_rows = np.repeat(visible, group)  # [Q*G]
            mask = np.arange(length)[None, :] < vis_rows[:, None]  # [Q*G, L]
        else:
            t = np.arange(length)
            j = t - (length - q_len)  # draft index, < 0 before the draft block
            seen = np.where(j[None, :] < 0, True,
                            dm[b][:, np.clip(j, 0, q_len - 1)])  # [Q, L]
            mask = np.repeat(seen, group, axis=0)  # [Q*G, L]
        logits = np.where(mask[None], logits, -np.inf)
        peak = logits.max(axis=-1, keepdims=True)
        peak = np.where(np.isfinite(peak), peak, 0)
        w = np.exp(logits - peak)
        denom = w.sum(axis=-1, keepdims=True)
        o = np.matmul(w, v.transpose(1, 0, 2))  # [Hkv, Q*G, D]
        o = np.where(denom > 0, o / np.where(denom > 0, denom, 1), 0) * dtype(out_scale)
        o = o.reshape(num_kv_heads, q_len, group, dim).transpose(1, 0, 2, 3)
        out[b] = o.reshape(q_len, n_qheads, dim)
    return out
