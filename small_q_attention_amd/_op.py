"""The ``sqa::paged_mtp_attention`` torch custom op over ``libsqa.so``.

Allocates the output and the split-KV workspace with torch's caching allocator
and launches on the current stream of the query's device. The fake (meta)
implementation only shapes the output, so the op traces under
``torch.compile`` / ``torch.export``; traced calls run
:func:`paged_mtp_attention_planned`, which makes the split plan at run time.
"""

from typing import Optional

import torch

from . import _lib

_KERNEL_PAGE = 16  # tokens per kernel page: the plan counts these (a cache page is 1-16 of them)


@torch.library.custom_op("sqa::paged_mtp_attention", mutates_args=())
def paged_mtp_attention(query: torch.Tensor, key_cache: torch.Tensor,
                        value_cache: torch.Tensor, block_tables: torch.Tensor,
                        seq_lens: torch.Tensor, num_splits: int,
                        pages_per_split: int) -> torch.Tensor:
    return _lib.run(query, key_cache, value_cache, block_tables, seq_lens, num_splits,
                    pages_per_split)


@torch.library.custom_op("sqa::paged_mtp_attention_planned", mutates_args=())
def paged_mtp_attention_planned(query: torch.Tensor, key_cache: torch.Tensor,
                                value_cache: torch.Tensor, block_tables: torch.Tensor,
                                seq_lens: torch.Tensor, max_seq_len: int,
                                chunk_keys: int) -> torch.Tensor:
    """:func:`paged_mtp_attention` with its split plan made at run time from the
    tensors' shapes (``_lib.plan_splits``: ``max_seq_len`` 0 plans over the whole
    block-table row, ``chunk_keys`` 0 is the automatic plan). What a traced call
    (torch.compile, torch.export) runs: the graph holds no plan, so shapes it
    leaves dynamic (the batch size of a serving loop) need no recompilation."""
    batch, q_len, hq, dim = query.shape
    num_splits, pps = _lib.plan_splits(
        query.device.index or 0, batch, q_len, hq, key_cache.shape[2], dim, max_seq_len,
        block_tables.shape[1] * (key_cache.shape[1] // _KERNEL_PAGE), chunk_keys)
    return _lib.run(query, key_cache, value_cache, block_tables, seq_lens, num_splits, pps)


@paged_mtp_attention_planned.register_fake
def _paged_mtp_attention_planned_fake(query, key_cache, value_cache, block_tables, seq_lens,
                                      max_seq_len, chunk_keys):
    return torch.empty_like(query)


@torch.library.custom_op("sqa::paged_attention_planned", mutates_args=())
def paged_attention_planned(query: torch.Tensor, k_view: torch.Tensor, v_view: torch.Tensor,
                            block_tables: torch.Tensor, seq_lens: torch.Tensor,
                            draft_mask: Optional[torch.Tensor], scale: float, out_scale: float,
                            max_seq_len: int) -> torch.Tensor:
    """The general entry (``sqa_paged_attention``: K/V as strided ``[P, page, Hkv, D]``
    views of any cache layout, fp16/bf16 queries over caches of their type or e4m3,
    packed draft words or the causal chain, softmax and output scales) with its split
    plan and workspace made at run time; ``query`` ``[B, Q, Hq, D]``. What the
    FlashInfer-shaped calls run when traced (torch.compile, torch.export)."""
    b, q_len, hq, d = query.shape
    hkv = k_view.shape[2]
    num_splits, pps = _lib.plan_splits(
        query.device.index or 0, b, q_len, hq, hkv, d, max_seq_len,
        block_tables.shape[1] * (k_view.shape[1] // _KERNEL_PAGE), 0)
    need = _lib.workspace_bytes(b, q_len, hq, hkv, d, num_splits, pps)
    workspace = torch.empty(need, dtype=torch.uint8, device=query.device) if need else None
    out = torch.empty_like(query)
    _lib.launch_general(query, out, k_view, v_view, block_tables, seq_lens, draft_mask, scale,
                        out_scale, num_splits, pps, workspace, _lib.raw_stream(query.device.index))
    return out


@paged_attention_planned.register_fake
def _paged_attention_planned_fake(query, k_view, v_view, block_tables, seq_lens, draft_mask,
                                  scale, out_scale, max_seq_len):
    return torch.empty_like(query)


@paged_mtp_attention.register_fake
def _paged_mtp_attention_fake(query, key_cache, value_cache, block_tables, seq_lens,
                              num_splits, pages_per_split):
    return torch.empty_like(query)
