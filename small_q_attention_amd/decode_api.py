"""FlashInfer-shaped entry points over the gfx950 kernels.

The reference compares its kernels with four FlashInfer paths for the same op
(``/root/reference/scripts/run_flashinfer_baseline.py:99-204``,
``scripts/compare_flashinfer_paths.py:95-160``,
``scripts/probe_decode_wrapper_mtp.py``). This module offers the same call shapes,
so code written against them runs here unchanged, within the contract of this
build (fp16 or bf16 Q, K/V of the same type or OCP FP8 E4M3
(``torch.float8_e4m3fn``, K/V scales folded into ``bmm1_scale``/``bmm2_scale``),
head_dim 64, 128 or 256, pages of 16 to 256 tokens, ``q_len * Hq / Hkv <= 64``,
at most 32 at head_dim 256):

* :func:`xqa_batch_decode_with_kv_cache` — block table + seq_lens, interleaved
  ``[P, 2, 16, Hkv, D]`` ("NHD") or ``[P, 2, Hkv, 16, D]`` ("HND") cache or a
  ``(k_cache, v_cache)`` pair, packed draft mask, ``bmm1_scale`` (softmax scale)
  and ``bmm2_scale`` (output scale).
* :func:`trtllm_batch_decode_with_kv_cache` — the same with "HND" by default.
* :class:`BatchDecodeWithPagedKVCacheWrapper` / :class:`BatchPrefillWithPagedKVCacheWrapper`
  — ``plan()`` over CSR page lists (``indptr``, ``indices``, ``last_page_len``)
  once, ``run()`` per layer.

Queries are ``[B * Q, Hq, D]`` (request-major, as FlashInfer takes them) and
every request has the same ``Q`` (``q_len_per_req``, or a uniform ``qo_indptr``).
The caller's workspace buffer holds the split-KV partials, so a run allocates
only its output (none when ``out`` is given) and is graph-capturable after
``plan()``. Arguments outside the contract raise ``ValueError`` (positional
encodings, soft caps, sliding windows, sinks, custom prefill masks); behaviour
is pinned against this build's oracle, not against FlashInfer itself. Traced by
``torch.compile`` (also ``fullgraph=True``) or ``torch.export``, a call runs the
``sqa::paged_attention_planned`` custom op, which plans the splits and takes its
workspace from torch's allocator at run time.
"""

from __future__ import annotations

from typing import Optional

from . import _lib
from .cuda import _tracing
from .masks import as_words

PAGE_SIZE = 16  # tokens per kernel page; cache pages hold 16 << k of them
PAGE_SIZES = (16, 32, 64, 128, 256)
HEAD_DIMS = (64, 128, 256)


def max_rows(head_dim: int) -> int:
    """Most query rows (``q_len * Hq / Hkv``) one kv head may carry at ``head_dim``."""
    return 32 if head_dim == 256 else 64


def _kv_views(kv_cache, kv_layout: str):
    """``(k_view, v_view)``: ``[P, 16, Hkv, D]`` views of the caller's cache, no copy."""
    if isinstance(kv_cache, (tuple, list)):
        if len(kv_cache) != 2:
            raise ValueError("a split cache is a (k_cache, v_cache) pair")
        k, v = kv_cache
        if kv_layout == "HND":
            k, v = k.transpose(1, 2), v.transpose(1, 2)
        return k, v
    if kv_cache.dim() != 5 or kv_cache.shape[1] != 2:
        raise ValueError("kv_cache must be [P, 2, 16, Hkv, D] (NHD) or [P, 2, Hkv, 16, D] (HND)")
    k, v = kv_cache[:, 0], kv_cache[:, 1]
    if kv_layout == "NHD":
        return k, v
    if kv_layout == "HND":
        return k.transpose(1, 2), v.transpose(1, 2)
    raise ValueError(f"kv_layout must be 'NHD' or 'HND', got {kv_layout!r}")


def _on_device(t, device, what):
    """ValueError unless ``t`` is a GPU tensor on ``device`` (raw pointers of host or
    other-device memory must never reach a kernel)."""
    if not getattr(t, "is_cuda", False) or t.device != device:
        raise ValueError(f"{what} must be a GPU tensor on {device}")


def _check_tensors(query, k, v, num_qo_heads: Optional[int] = None):
    import torch

    if not query.is_cuda or not k.is_cuda or not v.is_cuda:
        raise ValueError("query and kv_cache must be GPU tensors")
    if k.device != query.device or v.device != query.device:
        raise ValueError("query and kv_cache must be on the same GPU")
    fp8 = getattr(torch, "float8_e4m3fn", None)
    if query.dtype not in (torch.float16, torch.bfloat16) or (
            k.dtype != query.dtype and (fp8 is None or k.dtype != fp8)):
        raise ValueError("this build supports fp16 or bf16 query with KV of the same type or "
                         "float8_e4m3fn")
    if v.dtype != k.dtype:
        raise ValueError("key and value caches must share the element type")
    if query.dim() != 3 or not query.is_contiguous():
        raise ValueError("query must be a contiguous [B * Q, Hq, D] tensor")
    if query.shape[-1] not in HEAD_DIMS or k.shape[-1] != query.shape[-1]:
        raise ValueError("this build supports head_dim 64, 128 or 256, equal for query and "
                         "kv_cache")
    if k.shape[1] not in PAGE_SIZES:
        raise ValueError("this build supports page_size 16, 32, 64, 128 or 256")
    if num_qo_heads is not None and query.shape[1] != num_qo_heads:
        raise ValueError(f"query has {query.shape[1]} heads, plan() was given {num_qo_heads}")


def _run(query, k, v, block_tables, seq_lens, max_seq_len: int, q_len: int, scale: float,
         out_scale: float, mask, workspace_buffer, out, plan=None):
    """Shared launch: ``query`` ``[B * Q, Hq, D]`` -> ``out`` of the same shape."""
    import torch

    batch = block_tables.shape[0]
    if q_len < 1 or query.shape[0] != batch * q_len:
        raise ValueError(f"query holds {query.shape[0]} rows, expected batch {batch} x "
                         f"q_len_per_req {q_len}")
    hq, hkv = query.shape[1], k.shape[2]
    if hkv == 0 or hq % hkv:
        raise ValueError("num_qo_heads must be a multiple of num_kv_heads")
    d = query.shape[-1]
    if q_len * (hq // hkv) > max_rows(d):
        raise ValueError(f"q_len_per_req * (Hq / Hkv) must be at most {max_rows(d)} at "
                         f"head_dim {d}")
    if block_tables.dtype != torch.int32 or seq_lens.dtype != torch.int32:
        raise ValueError("block_tables and seq_lens must be int32")
    # Every buffer the kernel reads or writes through a raw pointer: on the query's
    # GPU, with the layout the kernel assumes (row-major block table, one length
    # per request).
    device = query.device
    _on_device(block_tables, device, "block_tables")
    _on_device(seq_lens, device, "seq_lens")
    if block_tables.dim() != 2 or not block_tables.is_contiguous():
        raise ValueError("block_tables must be a contiguous [batch, max_pages] tensor")
    if seq_lens.dim() != 1 or seq_lens.numel() != batch or not seq_lens.is_contiguous():
        raise ValueError(f"seq_lens must be a contiguous [{batch}] tensor")
    words = None if mask is None else as_words(mask, batch, q_len)
    if words is not None:
        _on_device(words, device, "mask")
    q4 = query.view(batch, q_len, hq, d)
    if out is not None:
        _on_device(out, device, "out")
        if out.shape != query.shape or out.dtype != query.dtype or not out.is_contiguous():
            raise ValueError("out must be a contiguous tensor shaped and typed like query")
    if _tracing():
        # torch.compile / torch.export: the checks above trace as guards; the graph
        # calls a custom op that plans the splits and takes its workspace from torch's
        # allocator at run time (the caller's buffer is not used).
        from . import _op  # noqa: F401  (registers the ops)

        res = torch.ops.sqa.paged_attention_planned(q4, k, v, block_tables, seq_lens, words,
                                                     float(scale), float(out_scale),
                                                     max(int(max_seq_len), 0))
        res = res.view(query.shape)
        if out is None:
            return res
        out.copy_(res)
        return out
    if out is None:
        out = torch.empty_like(query)
    if plan is None:
        plan = _lib.plan_splits(query.device.index or 0, batch, q_len, hq, hkv, d,
                                int(max_seq_len), block_tables.shape[1] * (k.shape[1] // PAGE_SIZE),
                                0)
    ns, pps = plan
    need = _lib.workspace_bytes(batch, q_len, hq, hkv, d, ns, pps)
    ws = None
    if need:
        if workspace_buffer is None:
            ws = torch.empty(need, dtype=torch.uint8, device=query.device)
        else:
            _on_device(workspace_buffer, device, "workspace_buffer")
            have = workspace_buffer.numel() * workspace_buffer.element_size()
            if have < need or not workspace_buffer.is_contiguous():
                raise ValueError(f"workspace_buffer must be contiguous and hold at least {need} "
                                 f"bytes for this batch (has {have})")
            ws = workspace_buffer
    _lib.launch_general(q4, out.view(batch, q_len, hq, d), k, v, block_tables, seq_lens,
                        words, scale, out_scale, ns, pps, ws,
                        _lib.raw_stream(query.device.index))
    return out


def _scalar(x, name):
    if hasattr(x, "item"):
        if x.numel() != 1:
            raise ValueError(f"{name} must be a scalar")
        x = x.item()
    return float(x)


def xqa_batch_decode_with_kv_cache(query, kv_cache, workspace_buffer, block_tables, seq_lens,
                                   max_seq_len, bmm1_scale, bmm2_scale, window_left=-1,
                                   out=None, sinks=None, kv_layout="NHD", enable_pdl=None,
                                   q_len_per_req=1, mask=None):
    """Paged decode of ``q_len_per_req`` draft tokens per request.

    Call shape of ``flashinfer.decode.xqa_batch_decode_with_kv_cache`` as the
    reference uses it (``run_flashinfer_baseline.py:153-177``). ``bmm1_scale`` is
    the softmax scale, ``bmm2_scale`` multiplies the output; ``mask`` is the packed
    draft mask (``None``: causal draft chain). ``max_seq_len`` bounds every
    ``seq_lens[b]``. Returns ``out`` (``[B * Q, Hq, D]``).
    """
    if window_left not in (-1, None):
        raise ValueError("sliding windows are not supported (window_left must be -1)")
    if sinks is not None:
        raise ValueError("attention sinks are not supported")
    k, v = _kv_views(kv_cache, kv_layout)
    _check_tensors(query, k, v)
    return _run(query, k, v, block_tables, seq_lens, int(max_seq_len), int(q_len_per_req),
                _scalar(bmm1_scale, "bmm1_scale"), _scalar(bmm2_scale, "bmm2_scale"), mask,
                workspace_buffer, out)


def trtllm_batch_decode_with_kv_cache(query, kv_cache, workspace_buffer, block_tables, seq_lens,
                                      max_seq_len, bmm1_scale, bmm2_scale, window_left=-1,
                                      out=None, sinks=None, kv_layout="HND", enable_pdl=None,
                                      q_len_per_req=1, mask=None):
    """Call shape of ``flashinfer.decode.trtllm_batch_decode_with_kv_cache``
    (``run_flashinfer_baseline.py:180-204``): as :func:`xqa_batch_decode_with_kv_cache`
    with the "HND" cache layout by default."""
    return xqa_batch_decode_with_kv_cache(query, kv_cache, workspace_buffer, block_tables,
                                          seq_lens, max_seq_len, bmm1_scale, bmm2_scale,
                                          window_left, out=out, sinks=sinks, kv_layout=kv_layout,
                                          enable_pdl=enable_pdl, q_len_per_req=q_len_per_req,
                                          mask=mask)


def csr_to_block_table(indptr, indices, last_page_len, page_size: int = PAGE_SIZE):
    """CSR page lists -> ``(block_tables [B, max_pages] int32, seq_lens [B] int32)`` on the
    same device: row b lists ``indices[indptr[b]:indptr[b + 1]]`` (padded with page 0)
    and holds ``(n_b - 1) * page_size + last_page_len[b]`` tokens (0 when ``n_b == 0``).
    One host read of the longest list (plan time)."""
    import torch

    indptr = indptr.to(torch.int64)
    counts = indptr[1:] - indptr[:-1]
    if counts.numel() == 0:
        raise ValueError("indptr must hold batch + 1 entries")
    if bool((counts < 0).any()):
        raise ValueError("indptr must be non-decreasing")
    max_pages = max(1, int(counts.max()))
    j = torch.arange(max_pages, device=indptr.device)
    valid = j[None, :] < counts[:, None]
    pos = (indptr[:-1, None] + j[None, :]).clamp(max=max(indices.numel() - 1, 0))
    if indices.numel() == 0:
        block_tables = torch.zeros(counts.numel(), max_pages, dtype=torch.int32,
                                   device=indptr.device)
    else:
        block_tables = torch.where(valid, indices.to(torch.int64)[pos], 0).to(torch.int32)
    last = last_page_len.to(torch.int64)
    if bool(((counts > 0) & ((last < 1) | (last > page_size))).any()):
        raise ValueError(f"last_page_len must be in [1, {page_size}] for non-empty requests")
    seq_lens = torch.where(counts > 0, (counts - 1) * page_size + last, 0).to(torch.int32)
    return block_tables.contiguous(), seq_lens.contiguous()


def _capacity(kw, *names):
    """Length of the first FlashInfer CUDA-graph buffer given under one of ``names``."""
    for name in names:
        buf = kw.get(name)
        if buf is not None:
            return int(buf.numel())
    return None


class _PagedWrapper:
    """Plan once (CSR -> block table, split plan, workspace check), run per layer.

    With ``use_cuda_graph=True`` the plan's block table and lengths live in
    buffers fixed by the first ``plan()`` (width: the ``paged_kv_indices_buffer``
    length when given, as FlashInfer sizes its graph buffers, else the first
    plan's widest request) and every later ``plan()`` copies into them in place,
    so kernels captured in a graph read the new plan on replay. The split plan
    then covers the buffer's whole width (it may not depend on the lengths);
    a re-plan that changes the batch, heads, draft length, mask or page size, or
    needs a wider table, raises ``ValueError``.
    """

    def __init__(self, float_workspace_buffer, kv_layout="NHD", use_cuda_graph=False,
                 use_tensor_cores=False, **kw):
        if kv_layout not in ("NHD", "HND"):
            raise ValueError(f"kv_layout must be 'NHD' or 'HND', got {kv_layout!r}")
        self._workspace = float_workspace_buffer
        self._kv_layout = kv_layout
        self._planned = None
        self._use_cuda_graph = bool(use_cuda_graph)
        self._graph_width = _capacity(kw, "paged_kv_indices_buffer", "paged_kv_indices_buf")
        self._graph = None  # persistent plan state in CUDA-graph mode

    def reset_workspace_buffer(self, float_workspace_buffer, *_unused):
        self._workspace = float_workspace_buffer

    def _plan_device(self, indptr):
        """Plan data lives where the kernels run: the workspace buffer's GPU when it
        has one (CSR lists may come from the host, as FlashInfer allows)."""
        ws = self._workspace
        if ws is not None and getattr(ws, "is_cuda", False):
            return ws.device
        return indptr.device

    def _plan(self, indptr, indices, last_page_len, num_qo_heads, num_kv_heads, head_dim,
              page_size, q_len, mask_words, sm_scale, pos_encoding_mode, window_left,
              logits_soft_cap, q_data_type, kv_data_type):
        import torch

        if pos_encoding_mode not in ("NONE", None):
            raise ValueError("only pos_encoding_mode='NONE' is supported")
        if window_left not in (-1, None):
            raise ValueError("sliding windows are not supported (window_left must be -1)")
        if logits_soft_cap not in (None, 0, 0.0):
            raise ValueError("logits soft capping is not supported")
        ok = (None, torch.float16, "float16", "fp16", torch.bfloat16, "bfloat16", "bf16")
        fp8 = (getattr(torch, "float8_e4m3fn", None), "float8_e4m3fn", "e4m3")
        if q_data_type not in ok or kv_data_type not in ok + fp8:
            raise ValueError("this build supports fp16 or bf16 query and KV "
                             "(KV also float8_e4m3fn)")
        if head_dim not in HEAD_DIMS or page_size not in PAGE_SIZES:
            raise ValueError("this build supports head_dim 64, 128 or 256 and page_size 16, 32, "
                             "64, 128 or 256")
        if num_kv_heads <= 0 or num_qo_heads % num_kv_heads:
            raise ValueError("num_qo_heads must be a multiple of num_kv_heads")
        device = self._plan_device(indptr)
        block_tables, seq_lens = csr_to_block_table(indptr.to(device), indices.to(device),
                                                    last_page_len.to(device), page_size)
        if mask_words is not None:
            mask_words = mask_words.to(device)
        batch = block_tables.shape[0]
        max_seq_len = int(seq_lens.max()) if batch else 0
        shape = dict(batch=batch, q_len=q_len, hq=num_qo_heads, hkv=num_kv_heads,
                     head_dim=head_dim, page_size=page_size,
                     mask=None if mask_words is None else tuple(mask_words.shape))
        if self._use_cuda_graph:
            block_tables, seq_lens, mask_words, plan = self._graph_plan(
                shape, block_tables, seq_lens, mask_words, device)
            max_seq_len = 0
        else:
            plan = _lib.plan_splits(device.index or 0, batch, q_len, num_qo_heads, num_kv_heads,
                                    head_dim, max(max_seq_len, 1),
                                    block_tables.shape[1] * (page_size // PAGE_SIZE), 0)
        need = _lib.workspace_bytes(batch, q_len, num_qo_heads, num_kv_heads, head_dim, *plan)
        if need and self._workspace is not None:
            have = self._workspace.numel() * self._workspace.element_size()
            if have < need:
                raise ValueError(f"float_workspace_buffer holds {have} bytes, this plan needs "
                                 f"{need}")
        self._planned = dict(block_tables=block_tables, seq_lens=seq_lens, plan=plan,
                             q_len=q_len, hq=num_qo_heads, hkv=num_kv_heads,
                             max_seq_len=max_seq_len, mask_words=mask_words,
                             page_size=page_size, head_dim=head_dim,
                             scale=head_dim ** -0.5 if sm_scale is None else float(sm_scale))

    def _graph_plan(self, shape, block_tables, seq_lens, mask_words, device):
        """Copy a plan into the persistent CUDA-graph buffers (allocated by the first plan)."""
        import torch

        g = self._graph
        if g is None:
            width = max(self._graph_width or 0, block_tables.shape[1], 1)
            kernel_pages = width * (shape["page_size"] // PAGE_SIZE)
            plan = _lib.plan_splits(device.index or 0, shape["batch"], shape["q_len"],
                                    shape["hq"], shape["hkv"], shape["head_dim"], 0, kernel_pages,
                                    0)
            g = dict(shape=shape, plan=plan,
                     block_tables=torch.zeros(shape["batch"], width, dtype=torch.int32,
                                              device=device),
                     seq_lens=torch.zeros(shape["batch"], dtype=torch.int32, device=device),
                     mask=None if mask_words is None else torch.empty_like(mask_words))
            self._graph = g
        elif g["shape"] != shape:
            raise ValueError(f"use_cuda_graph=True: a re-plan must keep {g['shape']}, got {shape}")
        width = g["block_tables"].shape[1]
        if block_tables.shape[1] > width:
            raise ValueError(f"use_cuda_graph=True: this plan needs {block_tables.shape[1]} pages "
                             f"per request, the graph buffers hold {width}")
        g["block_tables"].zero_()
        g["block_tables"][:, :block_tables.shape[1]].copy_(block_tables)
        g["seq_lens"].copy_(seq_lens)
        if mask_words is not None:
            g["mask"].copy_(mask_words)
        return g["block_tables"], g["seq_lens"], g["mask"], g["plan"]

    def run(self, q, paged_kv_cache, *args, q_scale=None, k_scale=None, v_scale=None, out=None,
            lse=None, return_lse=False, enable_pdl=None, window_left=None, sinks=None, **kwargs):
        """FlashInfer's ``run`` keywords: ``q_scale`` and ``k_scale`` multiply the softmax
        scale, ``v_scale`` the output (per-tensor FP8 scales); ``enable_pdl`` is a
        launch hint and has no effect here. ``lse``/``return_lse``, sliding windows,
        sinks, extra positional arguments and unknown keywords raise ``ValueError``."""
        if args:
            raise ValueError("run() takes (q, paged_kv_cache) positionally; pass the rest "
                             "by keyword")
        if kwargs:
            raise ValueError(f"unsupported run() arguments: {sorted(kwargs)}")
        if return_lse or lse is not None:
            raise ValueError("returning the log-sum-exp (lse / return_lse) is not supported")
        if window_left not in (None, -1):
            raise ValueError("sliding windows are not supported (window_left must be -1)")
        if sinks is not None:
            raise ValueError("attention sinks are not supported")
        if self._planned is None:
            raise RuntimeError("plan() must be called before run()")
        p = self._planned
        scale = p["scale"]
        for name, x in (("q_scale", q_scale), ("k_scale", k_scale)):
            if x is not None:
                scale *= _scalar(x, name)
        out_scale = 1.0 if v_scale is None else _scalar(v_scale, "v_scale")
        k, v = _kv_views(paged_kv_cache, self._kv_layout)
        _check_tensors(q, k, v, p["hq"])
        if k.shape[2] != p["hkv"]:
            raise ValueError(f"kv_cache has {k.shape[2]} kv heads, plan() was given {p['hkv']}")
        if q.shape[-1] != p["head_dim"]:
            raise ValueError(f"query has head_dim {q.shape[-1]}, plan() was given "
                             f"{p['head_dim']}")
        if k.shape[1] != p["page_size"]:
            raise ValueError(f"kv_cache pages hold {k.shape[1]} tokens, plan() was given "
                             f"{p['page_size']}")
        return _run(q, k, v, p["block_tables"], p["seq_lens"], p["max_seq_len"], p["q_len"],
                    scale, out_scale, p["mask_words"], self._workspace, out, plan=p["plan"])

    forward = run


class BatchDecodeWithPagedKVCacheWrapper(_PagedWrapper):
    """Call shape of ``flashinfer.decode.BatchDecodeWithPagedKVCacheWrapper`` as the
    reference uses it (``compare_flashinfer_paths.py:103-118``): ``plan(indptr, indices,
    last_page_len, num_qo_heads, num_kv_heads, head_dim, page_size, ...,
    q_len_per_req=Q)`` then ``run(q, paged_kv_cache)``; ``Q`` draft rows per request
    under the causal draft chain."""

    def plan(self, indptr, indices, last_page_len, num_qo_heads, num_kv_heads, head_dim,
             page_size, pos_encoding_mode="NONE", window_left=-1, logits_soft_cap=None,
             q_data_type=None, kv_data_type=None, data_type=None, sm_scale=None,
             rope_scale=None, rope_theta=None, non_blocking=True, q_len_per_req=1, **_unused):
        self._plan(indptr, indices, last_page_len, num_qo_heads, num_kv_heads, head_dim,
                   page_size, int(q_len_per_req), None, sm_scale, pos_encoding_mode,
                   window_left, logits_soft_cap, q_data_type or data_type, kv_data_type)


class BatchPrefillWithPagedKVCacheWrapper(_PagedWrapper):
    """Call shape of ``flashinfer.prefill.BatchPrefillWithPagedKVCacheWrapper`` as the
    reference uses it (``run_flashinfer_baseline.py:121-151``) for draft blocks:
    every request has the same query length ``Q`` (``qo_indptr`` in steps of ``Q``),
    its queries are the last ``Q`` positions of its KV. ``causal=True`` gives the
    draft chain; ``causal=False`` lets every row see every token. Custom prefill
    masks are not supported (use the packed draft mask of
    :func:`xqa_batch_decode_with_kv_cache`)."""

    def plan(self, qo_indptr, paged_kv_indptr, paged_kv_indices, paged_kv_last_page_len,
             num_qo_heads, num_kv_heads, head_dim_qk, page_size, head_dim_vo=None,
             custom_mask=None, packed_custom_mask=None, causal=False, pos_encoding_mode="NONE",
             use_fp16_qk_reduction=False, sm_scale=None, window_left=-1, logits_soft_cap=None,
             rope_scale=None, rope_theta=None, q_data_type=None, kv_data_type=None,
             non_blocking=True, **_unused):
        import torch

        if custom_mask is not None or packed_custom_mask is not None:
            raise ValueError("custom prefill masks are not supported")
        if head_dim_vo not in (None, head_dim_qk):
            raise ValueError("head_dim_vo must equal head_dim_qk")
        qo = qo_indptr.to(torch.int64).cpu()
        steps = qo[1:] - qo[:-1]
        if steps.numel() == 0 or int(qo[0]) != 0 or bool((steps != steps[0]).any()):
            raise ValueError("every request must have the same query length (uniform qo_indptr)")
        q_len = int(steps[0])
        if q_len < 1:
            raise ValueError("query length must be positive")
        mask = None
        if not causal:
            from .masks import spec_dec_mask

            mask = as_words(spec_dec_mask(steps.numel(), q_len, "full",
                                          device=paged_kv_indptr.device), steps.numel(), q_len)
        self._plan(paged_kv_indptr, paged_kv_indices, paged_kv_last_page_len, num_qo_heads,
                   num_kv_heads, head_dim_qk, page_size, q_len, mask, sm_scale,
                   pos_encoding_mode, window_left, logits_soft_cap, q_data_type, kv_data_type)


__all__ = ["xqa_batch_decode_with_kv_cache", "trtllm_batch_decode_with_kv_cache",
           "BatchDecodeWithPagedKVCacheWrapper", "BatchPrefillWithPagedKVCacheWrapper",
           "csr_to_block_table"]
