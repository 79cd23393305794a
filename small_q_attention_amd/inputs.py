"""Deterministic synthetic inputs for the paged small-q attention op.

Shapes follow the reference contract (``/root/reference/scripts/run_gpu_matrix.py:34-60``:
Q ``[B, q_len, Hq, D]``, K/V ``[pages, page_size, Hkv, D]`` fp16, ``block_tables``
``[B, max_pages]`` int32, ``seq_lens`` ``[B]`` int32 counting the draft tokens).

Differences from the reference's runner, on purpose:

* ``gen_device="cpu"`` draws every tensor from one seeded CPU generator in fp32
  and rounds to fp16, so the same seed gives bitwise-identical inputs in this
  container and on a GPU box. ``gen_device="cuda"`` draws on the device (much
  faster for multi-GB pools; reproducible per device, not across devices).
* ``page_mode="random"`` permutes a pool twice the size of the pages in use and
  hands the first ``sum(ceil(L_b/16))`` ids out in order, so sequences land on
  scattered pages of a larger pool (the reference's ``random`` mode permutes
  only inside each request's own range). ``shared`` and ``unique`` reproduce
  the reference's modes (reversed page ids).
* ``k_outlier_frac`` multiplies K by ``k_outlier_scale`` at that fraction of
  token slots (all heads of the slot), to stress softmax stability.
"""

from __future__ import annotations

import dataclasses
from typing import List, Optional, Sequence

HQ, HKV, HEAD_DIM, PAGE_SIZE = 32, 8, 128, 16


@dataclasses.dataclass
class Case:
    batch: int
    q_len: int
    seq_lens: List[int]
    num_query_heads: int = HQ
    num_kv_heads: int = HKV
    head_dim: int = HEAD_DIM
    page_size: int = PAGE_SIZE
    page_mode: str = "random"  # random | shared | unique
    pool_factor: int = 2
    k_outlier_frac: float = 0.0
    k_outlier_scale: float = 4.0
    seed: int = 0

    @property
    def pages_per_seq(self) -> List[int]:
        return [-(-int(n) // self.page_size) for n in self.seq_lens]

    @property
    def max_pages(self) -> int:
        return max(1, max(self.pages_per_seq))

    @property
    def max_seq_len(self) -> int:
        return max(self.seq_lens)


def uniform_case(batch: int, q_len: int, kv_len: int, **kw) -> Case:
    return Case(batch=batch, q_len=q_len, seq_lens=[kv_len] * batch, **kw)


def ragged_case(batch: int, q_len: int, lo: int, hi: int, seed: int, **kw) -> Case:
    """Per-sequence lengths drawn uniformly from ``[lo, hi]`` with a seeded generator."""
    import torch

    g = torch.Generator().manual_seed(seed + 17)
    lens = torch.randint(lo, hi + 1, (batch,), generator=g).tolist()
    return Case(batch=batch, q_len=q_len, seq_lens=lens, seed=seed, **kw)


def kv_bytes(seq_lens: Sequence[int], num_kv_heads: int = HKV, head_dim: int = HEAD_DIM) -> int:
    """Algorithmic K+V bytes one call must read: ``sum_b L_b * Hkv * D * 2 (K,V) * 2 B``."""
    return int(sum(int(n) for n in seq_lens)) * num_kv_heads * head_dim * 2 * 2


def alg_bytes(case: Case) -> int:
    """KV bytes plus Q in, O out, the used block-table entries and ``seq_lens``."""
    qo = 2 * case.batch * case.q_len * case.num_query_heads * case.head_dim * 2
    return (kv_bytes(case.seq_lens, case.num_kv_heads, case.head_dim) + qo
            + 4 * sum(case.pages_per_seq) + 4 * case.batch)


def attention_flops(case: Case) -> int:
    """2 flops per multiply-add for Q.K^T and P.V over every visible key."""
    vis = 0
    for n in case.seq_lens:
        for qi in range(case.q_len):
            vis += max(0, int(n) - case.q_len + qi + 1)
    return 4 * case.num_query_heads * case.head_dim * vis


def _block_tables(torch, case: Case, generator, pool_pages: int):
    pages = case.pages_per_seq
    bt = torch.zeros(case.batch, case.max_pages, dtype=torch.int32)
    if case.page_mode == "random":
        perm = torch.randperm(pool_pages, generator=generator).to(torch.int32)
        offset = 0
        for b, n in enumerate(pages):
            bt[b, :n] = perm[offset:offset + n]
            offset += n
    elif case.page_mode == "shared":
        n = case.max_pages
        for b, nb in enumerate(pages):
            bt[b, :nb] = torch.arange(n - 1, n - 1 - nb, -1, dtype=torch.int32)
    elif case.page_mode == "unique":
        n = case.max_pages
        for b, nb in enumerate(pages):
            bt[b, :nb] = torch.arange(n - 1, n - 1 - nb, -1, dtype=torch.int32) + b * n
    else:
        raise ValueError(f"unsupported page_mode: {case.page_mode}")
    return bt


def pool_pages_for(case: Case) -> int:
    if case.page_mode == "random":
        return max(1, case.pool_factor * sum(case.pages_per_seq))
    if case.page_mode == "shared":
        return case.max_pages
    return case.max_pages * case.batch


def make_inputs(case: Case, device="cpu", gen_device: Optional[str] = None):
    """Return ``(query, key_cache, value_cache, block_tables, seq_lens)`` on ``device``.

    ``gen_device`` defaults to ``"cpu"`` (bitwise reproducible everywhere).
    """
    import torch

    gen_device = gen_device or "cpu"
    pool = pool_pages_for(case)
    qshape = (case.batch, case.q_len, case.num_query_heads, case.head_dim)
    kshape = (pool, case.page_size, case.num_kv_heads, case.head_dim)
    if gen_device == "cpu":
        g = torch.Generator().manual_seed(case.seed)
        query = torch.randn(qshape, generator=g).half()
        key = torch.randn(kshape, generator=g)
        value = torch.randn(kshape, generator=g).half()
        if case.k_outlier_frac > 0:
            hit = torch.rand(pool * case.page_size, generator=g) < case.k_outlier_frac
            key.view(pool * case.page_size, -1)[hit] *= case.k_outlier_scale
        key = key.half()
        bt = _block_tables(torch, case, g, pool)
        out = [query, key, value]
        out = [t.to(device) for t in out]
    else:
        g = torch.Generator(device=gen_device).manual_seed(case.seed)
        query = torch.randn(qshape, generator=g, device=gen_device, dtype=torch.float16)
        key = torch.randn(kshape, generator=g, device=gen_device, dtype=torch.float16)
        value = torch.randn(kshape, generator=g, device=gen_device, dtype=torch.float16)
        if case.k_outlier_frac > 0:
            hit = torch.rand(pool * case.page_size, generator=g, device=gen_device) < case.k_outlier_frac
            key.view(pool * case.page_size, -1)[hit] *= case.k_outlier_scale
        gh = torch.Generator().manual_seed(case.seed)
        bt = _block_tables(torch, case, gh, pool)
        out = [t.to(device) for t in (query, key, value)]
    seq_lens = torch.tensor([int(n) for n in case.seq_lens], dtype=torch.int32)
    return out[0], out[1], out[2], bt.to(device), seq_lens.to(device)


def baseline_configs():
    """The benchmark configurations as :class:`Case` objects (``cfg1``..``cfg5``).

    ``cfg4`` (the 36-case matrix) is expanded by :func:`matrix_cases`.
    """
    return {
        "cfg1": uniform_case(1, 2, 1024, seed=1),
        "cfg2": uniform_case(4, 4, 8192, seed=2),
        "cfg3": uniform_case(16, 8, 32768, seed=3, k_outlier_frac=0.01),
        "cfg5": ragged_case(16, 8, 1024, 32768, seed=5),
    }


def matrix_cases(q_lens=(2, 4, 8, 16), kv_lens=(1024, 8192, 32768), batches=(1, 4, 16), seed0=1000):
    """The fixed 36-case matrix (``/root/reference/configs/core_matrix.json:2-10``)."""
    cases = []
    index = 0
    for q in q_lens:
        for kv in kv_lens:
            for b in batches:
                cases.append(uniform_case(b, q, kv, seed=seed0 + index))
                index += 1
    return cases


def ceil_div(a: int, b: int) -> int:
    return -(-a // b)


__all__ = [
    "Case", "uniform_case", "ragged_case", "make_inputs", "kv_bytes", "alg_bytes",
    "attention_flops", "baseline_configs", "matrix_cases", "pool_pages_for", "ceil_div",
    "HQ", "HKV", "HEAD_DIM", "PAGE_SIZE",
]
