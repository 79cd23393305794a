"""The ``sqa::paged_mtp_attention`` torch custom op over ``libsqa.so``.

Allocates the output and the split-KV workspace with torch's caching allocator
and launches on the current stream of the query's device. The fake (meta)
implementation only shapes the output, so the op traces under
``torch.compile`` / ``torch.export``; :func:`traced_plan` gives a traced call its split
plan.
"""

import torch

from . import _lib


@torch.library.custom_op("sqa::paged_mtp_attention", mutates_args=())
def paged_mtp_attention(query: torch.Tensor, key_cache: torch.Tensor,
                        value_cache: torch.Tensor, block_tables: torch.Tensor,
                        seq_lens: torch.Tensor, num_splits: int,
                        pages_per_split: int) -> torch.Tensor:
    return _lib.run(query, key_cache, value_cache, block_tables, seq_lens, num_splits,
                    pages_per_split)


@torch.compiler.assume_constant_result
def traced_plan(device_index: int, batch: int, q_len: int, num_query_heads: int,
                num_kv_heads: int, head_dim: int, max_seq_len: int, max_pages: int,
                chunk_keys: int):
    """``(num_splits, pages_per_split)`` of ``_lib.plan_splits`` for a call being traced:
    run while tracing (it loads the library and reads the device's CU count through
    the C ABI, which Dynamo does not trace), its result a constant of the graph; the
    plan is a pure function of these integers and the device."""
    return _lib.plan_splits(device_index, batch, q_len, num_query_heads, num_kv_heads, head_dim,
                            max_seq_len, max_pages, chunk_keys)


@paged_mtp_attention.register_fake
def _paged_mtp_attention_fake(query, key_cache, value_cache, block_tables, seq_lens,
                              num_splits, pages_per_split):
    return torch.empty_like(query)
