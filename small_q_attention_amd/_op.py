"""The ``sqa::paged_mtp_attention`` torch custom op over ``libsqa.so``.

Allocates the output and the split-KV workspace with torch's caching allocator
and launches on the current stream of the query's device. The fake (meta)
implementation only shapes the output, so the op traces under
``torch.compile`` / ``torch.export``.
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


@paged_mtp_attention.register_fake
def _paged_mtp_attention_fake(query, key_cache, value_cache, block_tables, seq_lens,
                              num_splits, pages_per_split):
    return torch.empty_like(query)
