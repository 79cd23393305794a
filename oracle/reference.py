"""Loop-faithful torch restatement of the reference oracle.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Follows ``/root/reference/src/small_q_attention/reference.py:10-74`` step by
step: validate the contract (``:34-44``), then per sequence gather the used
pages in block-table order (``:54-59``), and per draft row ``qi`` and query head
``qh`` score the visible keys (``:63,68``), take an fp32 softmax cast back to the
query dtype (``:69``) and multiply by V (``:70``).
"""

from __future__ import annotations


def paged_mtp_attention_reference(
    query,
    key_cache,
    value_cache,
    block_tables,
    seq_lens,
    page_size: int,
    num_kv_heads: int,
):
    """Causal paged attention over a uniform block of ``q_len`` draft rows.

    Args mirror ``reference.py:10-32``:
        query: ``[batch, q_len, num_query_heads, head_dim]``.
        key_cache / value_cache: ``[num_pages, page_size, num_kv_heads, head_dim]``.
        block_tables: ``[batch, max_pages]`` physical page ids.
        seq_lens: ``[batch]`` KV length including the ``q_len`` draft tokens.
        page_size: tokens per physical page.
        num_kv_heads: KV heads; query head ``qh`` reads KV head ``qh // group``.

    Returns ``[batch, q_len, num_query_heads, head_dim]`` in ``query.dtype``.
    Raises ``ValueError`` under the conditions of ``reference.py:34-44,52-53``.
    """
    import torch

    # Contract checks: reference.py:34-44.
    if query.ndim != 4:
        raise ValueError("query must be [batch, q_len, num_query_heads, head_dim]")
    n_batch, q_len, n_qheads, head_dim = query.shape
    if n_qheads % num_kv_heads:
        raise ValueError("num_query_heads must be a multiple of num_kv_heads")
    if tuple(key_cache.shape[1:]) != (page_size, num_kv_heads, head_dim):
        raise ValueError("key_cache must be [num_pages, page_size, num_kv_heads, head_dim]")
    if tuple(value_cache.shape) != tuple(key_cache.shape):
        raise ValueError("value_cache must match key_cache")
    if block_tables.shape[0] != n_batch or seq_lens.numel() != n_batch:
        raise ValueError("block_tables / seq_lens do not match the batch size")

    scale = head_dim ** -0.5  # reference.py:46
    group = n_qheads // num_kv_heads
    per_seq = []
    for b in range(n_batch):  # reference.py:50
        length = int(seq_lens[b])
        if length < q_len:  # reference.py:52-53
            raise ValueError("seq_lens[b] must be >= q_len")
        pages_used = -(-length // page_size)
        ids = block_tables[b, :pages_used].long()
        # Token t lives at page ids[t // page_size], slot t % page_size.
        k_seq = key_cache.index_select(0, ids).reshape(-1, num_kv_heads, head_dim)[:length]
        v_seq = value_cache.index_select(0, ids).reshape(-1, num_kv_heads, head_dim)[:length]
        rows = []
        for qi in range(q_len):  # reference.py:62
            visible = length - q_len + qi + 1  # reference.py:63
            heads = []
            for qh in range(n_qheads):  # reference.py:66
                kvh = qh // group  # reference.py:67
                logits = torch.matmul(k_seq[:visible, kvh], query[b, qi, qh]) * scale
                weights = torch.softmax(logits.float(), dim=0).to(query.dtype)
                heads.append(torch.matmul(weights, v_seq[:visible, kvh]))
            rows.append(torch.stack(heads))
        per_seq.append(torch.stack(rows))
    return torch.stack(per_seq)
