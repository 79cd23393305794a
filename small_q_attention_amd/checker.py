"""A float32 torch statement of the op, used only to *check* outputs.

Nothing on the op path imports this module: ``forward_vN``,
``paged_mtp_attention`` and ``decode_api`` run the HIP kernels of
``libsqa.so`` and raise if it is missing. The checker serves the matrix
runner's ``--check-correctness`` (the reference runner's flag,
``/root/reference/scripts/run_gpu_matrix.py:126-127,159-169``) and the
full-size GPU tests, where the float64 C oracle would be too slow; a CPU test
pins it against that oracle on ragged, partial-page and short-row cases.

Semantics (``/root/reference/src/small_q_attention/reference.py:46-72``): query
head ``h`` reads kv head ``h // group``; draft row ``qi`` sees tokens
``t < seq_len - q_len + qi + 1``; scale ``head_dim ** -0.5``; rows that see no
key are 0 (the reference's v2+ merge, ``csrc/small_q_attention_ext.cu:365``).
"""

from __future__ import annotations

import numpy as np


def attention_fp32(query, key_cache, value_cache, block_tables, seq_lens, page_size,
                   num_kv_heads, batches=None):
    """The op in torch float32 on the tensors' device, one sequence at a time.

    ``key_cache``/``value_cache`` are ``[P, page_size, Hkv, D]`` (any float type).
    Returns a float64 numpy array ``[B, Q, Hq, D]``; batches not in ``batches``
    (when given) are NaN.
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
        w = torch.nan_to_num(w, nan=0.0)  # rows with no visible key
        o = torch.matmul(w, v.permute(1, 0, 2).contiguous())  # [Hkv, Q*G, D]
        o = o.reshape(num_kv_heads, q_len, group, dim).permute(1, 0, 2, 3).reshape(q_len, hq, dim)
        out[b] = o.double().cpu().numpy()
    return out
