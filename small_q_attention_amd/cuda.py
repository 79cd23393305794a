"""Drop-in op boundary: ``load_v0..load_v5`` and ``forward_v0..forward_v5``.

Mirrors ``/root/reference/src/small_q_attention/cuda.py`` (same names,
parameter order, defaults and exception classes) over one gfx950 library,
``libsqa.so``. Eager calls go straight to the library; under ``torch.compile``
(``fullgraph=True`` included) and ``torch.export`` the checks trace as guards and
the graph calls the ``sqa::paged_mtp_attention_planned`` torch custom op, which
plans the splits at run time (:func:`_traced_op`).
All six ``forward_vN`` run the same HIP kernels (split-KV partial kernel with
GQA and draft-row reuse, plus the log-sum-exp merge kernel); the version
number only selects which of the reference's argument checks apply.

Validation order follows the reference: ``RuntimeError`` when no GPU is
present (``cuda.py:65-66``); ``ValueError`` for inputs off the device,
non-contiguous, not fp16, an unsupported ``q_len`` or ``head_dim``
(``cuda.py:67-77``), a GQA group other than 4 for v3-v5 (``:208-209``),
``chunk_keys <= 0`` (``:149-150``) and ``token_group`` not in {2, 4}
(``:329-330``); then ``RuntimeError`` for the launcher's shape checks
(``csrc/small_q_attention_ext.cu:976-1002``).

Deliberate contract differences:
* ``q_len`` 16 is accepted (the reference allows 2, 4, 8): ``q_len * group``
  must be at most 64 rows.
* ``page_size`` must be 16, 32, 64, 128 or 256 and ``head_dim`` 128 (the reference's
  launchers take any page size, but every reference caller uses 16). The
  native entry :func:`paged_mtp_attention` also takes head_dim 64 and 256
  (at most 32 rows at 256).
* ``chunk_keys=None`` selects the automatic split plan (from the CU count).
* ``token_group`` (v5) is validated and otherwise ignored: every draft row
  already shares one K/V load.
* ``verbose`` echoes the hipcc command if the library has to be built.
"""

from __future__ import annotations

from typing import Optional

from . import _lib

SUPPORTED_Q_LENS = (2, 4, 8, 16)
HEAD_DIM = 128
HEAD_DIMS = (64, 128, 256)  # native entry
PAGE_SIZE = 16
SUPPORTED_PAGE_SIZES = (16, 32, 64, 128, 256)
MAX_ROWS = 64


def _load(verbose: bool = False):
    if _tracing():  # a traced call's custom op loads it when the graph runs (_traced_op)
        return None
    return _lib.load(verbose=bool(verbose))


class _Module:
    """What ``load_vN`` returns: the reference's extension-module attribute names."""

    def __init__(self, lib):
        self.lib = lib

    def forward(self, query, key_cache, value_cache, block_tables, seq_lens, page_size):
        return _run(query, key_cache, value_cache, block_tables, seq_lens, page_size, None, 0)

    def forward_v1(self, query, key_cache, value_cache, block_tables, seq_lens, page_size):
        return _run(query, key_cache, value_cache, block_tables, seq_lens, page_size, None, 0)

    def forward_v2(self, query, key_cache, value_cache, block_tables, seq_lens, page_size,
                   chunk_keys):
        return _run(query, key_cache, value_cache, block_tables, seq_lens, page_size,
                    chunk_keys, -1)

    def forward_v3(self, query, key_cache, value_cache, block_tables, seq_lens, page_size,
                   chunk_keys, max_seq_len):
        return _run(query, key_cache, value_cache, block_tables, seq_lens, page_size,
                    chunk_keys, max_seq_len or -1)

    forward_v4 = forward_v3

    def forward_v5(self, query, key_cache, value_cache, block_tables, seq_lens, page_size,
                   chunk_keys, token_group, max_seq_len):
        return _run(query, key_cache, value_cache, block_tables, seq_lens, page_size,
                    chunk_keys, max_seq_len or -1)


_MODULE = None


def _module(verbose):
    global _MODULE
    if _tracing():  # no module state is touched while torch.compile traces
        return _Module(None)
    if _MODULE is None or verbose:
        _MODULE = _Module(_load(verbose))
    return _MODULE


def load_v0(verbose: bool = False):
    """Load ``libsqa.so`` (building it on first use if absent)."""
    return _module(verbose)


load_v1 = load_v2 = load_v3 = load_v4 = load_v5 = load_v0


_GPU_SEEN_BY = None  # the torch.cuda.is_available function that last reported a GPU
_TORCH = None  # the torch module, once a GPU has been seen


def _gpu_present(torch) -> bool:
    """``torch.cuda.is_available()``, remembered once true (it costs ~1 us per call)."""
    global _GPU_SEEN_BY, _TORCH
    probe = torch.cuda.is_available
    if _GPU_SEEN_BY is probe:
        return True
    if probe():
        _GPU_SEEN_BY, _TORCH = probe, torch
        return True
    return False


def _check_python_contract(tag, query, key_cache, value_cache, block_tables, seq_lens,
                           gqa4: bool, allow_bf16: bool = False,
                           head_dims: tuple = (HEAD_DIM,)):
    """The reference's Python-side checks (``cuda.py:65-77,85-95,138-150,197-211``).
    ``allow_bf16`` and ``head_dims`` (native entry only) also accept Q/K/V all in
    bfloat16 and the other head dims of this build."""
    import torch

    # (While torch.compile traces, the inputs are device tensors already.)
    if not _tracing() and not _gpu_present(torch):
        raise RuntimeError(f"a ROCm GPU is required for the {tag} kernel")
    tensors = (query, key_cache, value_cache, block_tables, seq_lens)
    for t in tensors:
        if not t.is_cuda:
            raise ValueError(f"all {tag} inputs must be GPU tensors")
    device = query.device
    for t in tensors:
        if t.device != device:
            raise ValueError(f"all {tag} inputs must be on the same device")
    for t in tensors:
        if not t.is_contiguous():
            raise ValueError(f"all {tag} inputs must be contiguous")
    half = torch.float16
    if query.dtype != half or key_cache.dtype != half or value_cache.dtype != half:
        bf = torch.bfloat16
        if not (allow_bf16 and query.dtype == bf and key_cache.dtype == bf
                and value_cache.dtype == bf):
            raise ValueError(f"{tag} requires FP16 Q/K/V" + (" (or all BF16)" if allow_bf16 else ""))
    if query.ndim < 2 or query.shape[1] not in SUPPORTED_Q_LENS:
        raise ValueError(f"{tag} supports q_len 2, 4, 8 or 16")
    if query.shape[-1] not in head_dims:
        raise ValueError(f"{tag} supports head_dim " + ", ".join(map(str, head_dims)))
    if gqa4:
        if (key_cache.ndim < 3 or query.ndim < 3 or key_cache.shape[2] == 0
                or query.shape[2] % key_cache.shape[2] != 0
                or query.shape[2] // key_cache.shape[2] != 4):
            raise ValueError(f"{tag} requires a GQA group size of exactly 4 (Hq/Hkv = 32/8)")


def _check_launcher_contract(query, key_cache, value_cache, block_tables, seq_lens, page_size):
    """The launcher's checks (``csrc/small_q_attention_ext.cu:976-1002``) -> RuntimeError."""
    import torch

    if query.ndim != 4:
        raise RuntimeError("query must be [B, Q, Hq, D]")
    if key_cache.ndim != 4:
        raise RuntimeError("key_cache must be [P, page, Hkv, D]")
    if value_cache.shape != key_cache.shape:
        raise RuntimeError("value_cache shape mismatch")
    if block_tables.dtype != torch.int32 or seq_lens.dtype != torch.int32:
        raise RuntimeError("block_tables and seq_lens must be int32")
    if block_tables.ndim != 2:
        raise RuntimeError("block_tables must be [B, max_pages]")
    batch, q_len, hq, dim = query.shape
    num_pages, cache_page, hkv, kdim = key_cache.shape
    if hkv == 0 or hq % hkv != 0:
        raise RuntimeError("Hq must be divisible by Hkv")
    if kdim != dim:
        raise RuntimeError("key_cache head_dim does not match query")
    if int(page_size) != cache_page:
        raise RuntimeError("page_size argument does not match cache")
    if seq_lens.numel() != batch:
        raise RuntimeError("seq_lens batch mismatch")
    if block_tables.shape[0] != batch:
        raise RuntimeError("block_tables batch mismatch")
    if num_pages <= 0 or block_tables.shape[1] <= 0:
        raise RuntimeError("empty KV cache is not supported")
    if batch == 0:
        raise RuntimeError("batch must be positive")
    if cache_page not in SUPPORTED_PAGE_SIZES:
        raise ValueError("this build supports page_size 16, 32, 64, 128 or 256")
    rows_cap = 32 if dim == 256 else MAX_ROWS
    if q_len * (hq // hkv) > rows_cap:
        raise ValueError(f"q_len * (Hq / Hkv) must be at most {rows_cap} at head_dim {dim}")


def _run(query, key_cache, value_cache, block_tables, seq_lens, page_size,
         chunk_keys: Optional[int], max_seq_len: int):
    """Plan the split-KV grid and launch: eagerly through the library, or, while
    torch.compile / torch.export trace, through the custom op (:func:`_traced_op`).

    ``max_seq_len``: > 0 known; -1 measure with ``seq_lens.max().item()`` (a host
    sync, as the reference v2 launcher always does and v3-v5 do for 0,
    ``csrc/small_q_attention_ext.cu:1097,1173-1176``); 0 unknown, plan over the
    whole block-table row (no sync).
    """
    _check_launcher_contract(query, key_cache, value_cache, block_tables, seq_lens, page_size)
    if _tracing():
        return _traced_op(query, key_cache, value_cache, block_tables, seq_lens, chunk_keys,
                          max_seq_len)
    if max_seq_len == -1:
        max_seq_len = int(seq_lens.max().item())
        if max_seq_len <= 0:
            raise RuntimeError("seq_lens must be positive")
    batch, q_len, hq, _ = query.shape
    hkv = key_cache.shape[2]
    ck = 0 if chunk_keys is None else int(chunk_keys)
    # The plan counts 16-token kernel pages.
    kernel_pages = block_tables.shape[1] * (key_cache.shape[1] // PAGE_SIZE)
    num_splits, pps = _lib.plan_splits(query.device.index or 0, batch, q_len, hq, hkv,
                                       query.shape[-1], int(max_seq_len), kernel_pages, ck)
    # Eager: the custom op's allocation and launch without the dispatcher round trip.
    return _lib.run(query, key_cache, value_cache, block_tables, seq_lens, num_splits, pps)


def _traced_op(query, key_cache, value_cache, block_tables, seq_lens,
               chunk_keys: Optional[int], max_seq_len: int):
    """A call that torch.compile (also with ``fullgraph=True``) or torch.export is
    tracing, after the same checks, which trace as guards on dtypes and shapes: the
    graph calls the ``sqa::paged_mtp_attention_planned`` custom op, which makes the
    split plan at run time from the tensors' shapes, so a dynamic batch size needs
    no recompilation. A measured ``max_seq_len`` (-1: ``seq_lens.max().item()``, a
    host sync) plans over the whole block-table row instead, so the graph never
    synchronises; its splits differ from the measured plan's only past the
    sequences' ends (empty), which changes the merge's summation order, not which
    keys count."""
    import torch

    from . import _op  # noqa: F401  (registers the ops)

    return torch.ops.sqa.paged_mtp_attention_planned(
        query, key_cache, value_cache, block_tables, seq_lens, max(int(max_seq_len), 0),
        0 if chunk_keys is None else int(chunk_keys))


def _fast(query, key_cache, value_cache, block_tables, seq_lens, page_size, chunk_keys,
          max_seq_len: int, gqa4: bool):
    """The common valid call (fp16 Q/K/V, head dim 128, one device, contiguous, consistent
    shapes, eager, library loaded) checked in one pass, then planned and launched;
    ``None`` when anything differs, and the full checks then run (and raise as the
    reference does). Accepts exactly what those checks accept."""
    if _tracing():
        return None
    torch = _TORCH
    if torch is None or _GPU_SEEN_BY is not torch.cuda.is_available or _lib._LIB is None:
        return None
    tensor = torch.Tensor  # plain tensors only (subclasses and stand-ins take the full way)
    if not (type(query) is tensor and type(key_cache) is tensor and type(value_cache) is tensor
            and type(block_tables) is tensor and type(seq_lens) is tensor):
        return None
    f16, i32 = torch.float16, torch.int32
    if not (query.dtype is f16 and key_cache.dtype is f16 and value_cache.dtype is f16
            and block_tables.dtype is i32 and seq_lens.dtype is i32
            and query.is_cuda and key_cache.is_cuda and value_cache.is_cuda
            and block_tables.is_cuda and seq_lens.is_cuda):
        return None
    dev = query.get_device()
    if not (key_cache.get_device() == dev and value_cache.get_device() == dev
            and block_tables.get_device() == dev and seq_lens.get_device() == dev
            and query.is_contiguous() and key_cache.is_contiguous()
            and value_cache.is_contiguous() and block_tables.is_contiguous()
            and seq_lens.is_contiguous()):
        return None
    qs, ks = query.shape, key_cache.shape
    if len(qs) != 4 or len(ks) != 4 or value_cache.shape != ks or block_tables.dim() != 2:
        return None
    batch, q_len, hq, dim = qs
    num_pages, page, hkv, kdim = ks
    bt_rows, bt_cols = block_tables.shape
    if not (dim == HEAD_DIM and kdim == HEAD_DIM and q_len in SUPPORTED_Q_LENS
            and page == page_size and page in SUPPORTED_PAGE_SIZES and hkv > 0
            and hq % hkv == 0 and batch > 0 and bt_rows == batch
            and seq_lens.numel() == batch and num_pages > 0 and bt_cols > 0):
        return None
    group = hq // hkv
    if (gqa4 and group != 4) or q_len * group > MAX_ROWS:
        return None
    if chunk_keys is not None and chunk_keys <= 0:
        return None
    if max_seq_len == -1:
        max_seq_len = int(seq_lens.max().item())
        if max_seq_len <= 0:
            raise RuntimeError("seq_lens must be positive")
    num_splits, pps = _lib.plan_splits(dev, batch, q_len, hq, hkv, HEAD_DIM, int(max_seq_len),
                                       bt_cols * (page // PAGE_SIZE),
                                       0 if chunk_keys is None else int(chunk_keys))
    return _lib.run_fp16(query, key_cache, value_cache, block_tables, seq_lens, batch, q_len,
                         hq, hkv, num_pages, page, bt_cols, num_splits, pps, dev)


def _tracing() -> bool:
    import torch

    compiler = getattr(torch, "compiler", None)
    return bool(compiler is not None and compiler.is_compiling())


def paged_mtp_attention(query, key_cache, value_cache, block_tables, seq_lens,
                        page_size: int = PAGE_SIZE, max_seq_len: int = 0,
                        chunk_keys: Optional[int] = None):
    """Native entry: automatic split plan, no host sync unless ``max_seq_len < 0``.

    ``max_seq_len`` > 0 promises every ``seq_lens[b] <= max_seq_len``; 0 plans
    over the whole block-table row. Q, K and V may also all be bfloat16, and
    head_dim 64 or 256 (the ``forward_vN`` names keep the reference's fp16,
    head_dim 128 contract).
    """
    if max_seq_len >= -1:
        out = _fast(query, key_cache, value_cache, block_tables, seq_lens, page_size, chunk_keys,
                    int(max_seq_len), False)
        if out is not None:
            return out
    _check_python_contract("sqa", query, key_cache, value_cache, block_tables, seq_lens, False,
                           allow_bf16=True, head_dims=HEAD_DIMS)
    if chunk_keys is not None and chunk_keys <= 0:
        raise ValueError("chunk_keys must be positive")
    _load()
    return _run(query, key_cache, value_cache, block_tables, seq_lens, page_size, chunk_keys,
                int(max_seq_len))


def forward_v0(query, key_cache, value_cache, block_tables, seq_lens, page_size: int,
               verbose: bool = False):
    """Reference ``forward_v0`` (``cuda.py:61-78``); automatic split plan, no host sync."""
    out = _fast(query, key_cache, value_cache, block_tables, seq_lens, page_size, None, 0, False)
    if out is not None:
        return out
    _check_python_contract("v0", query, key_cache, value_cache, block_tables, seq_lens, False)
    return load_v0(verbose=verbose).forward(query, key_cache, value_cache, block_tables,
                                            seq_lens, page_size)


def forward_v1(query, key_cache, value_cache, block_tables, seq_lens, page_size: int,
               verbose: bool = False):
    """Reference ``forward_v1`` (``cuda.py:81-96``); same kernels as v0."""
    out = _fast(query, key_cache, value_cache, block_tables, seq_lens, page_size, None, 0, False)
    if out is not None:
        return out
    _check_python_contract("v1", query, key_cache, value_cache, block_tables, seq_lens, False)
    return load_v1(verbose=verbose).forward_v1(query, key_cache, value_cache, block_tables,
                                               seq_lens, page_size)


def forward_v2(query, key_cache, value_cache, block_tables, seq_lens, page_size: int,
               chunk_keys: Optional[int] = 512, verbose: bool = False):
    """Reference ``forward_v2`` (``cuda.py:120-153``): ``chunk_keys`` KV entries per split."""
    out = _fast(query, key_cache, value_cache, block_tables, seq_lens, page_size, chunk_keys, -1,
                False)
    if out is not None:
        return out
    _check_python_contract("v2", query, key_cache, value_cache, block_tables, seq_lens, False)
    if chunk_keys is not None and chunk_keys <= 0:
        raise ValueError("chunk_keys must be positive")
    return load_v2(verbose=verbose).forward_v2(query, key_cache, value_cache, block_tables,
                                               seq_lens, page_size, chunk_keys)


def forward_v3(query, key_cache, value_cache, block_tables, seq_lens, page_size: int,
               chunk_keys: Optional[int] = 512, max_seq_len: int = 0, verbose: bool = False):
    """Reference ``forward_v3`` (``cuda.py:177-214``); ``max_seq_len=0`` measures it (sync)."""
    out = _fast(query, key_cache, value_cache, block_tables, seq_lens, page_size, chunk_keys,
                max_seq_len or -1, True)
    if out is not None:
        return out
    _check_python_contract("v3", query, key_cache, value_cache, block_tables, seq_lens, True)
    if chunk_keys is not None and chunk_keys <= 0:
        raise ValueError("chunk_keys must be positive")
    return load_v3(verbose=verbose).forward_v3(query, key_cache, value_cache, block_tables,
                                               seq_lens, page_size, chunk_keys, max_seq_len)


def forward_v4(query, key_cache, value_cache, block_tables, seq_lens, page_size: int,
               chunk_keys: Optional[int] = 512, max_seq_len: int = 0, verbose: bool = False):
    """Reference ``forward_v4`` (``cuda.py:238-273``); same kernels as v3."""
    out = _fast(query, key_cache, value_cache, block_tables, seq_lens, page_size, chunk_keys,
                max_seq_len or -1, True)
    if out is not None:
        return out
    _check_python_contract("v4", query, key_cache, value_cache, block_tables, seq_lens, True)
    if chunk_keys is not None and chunk_keys <= 0:
        raise ValueError("chunk_keys must be positive")
    return load_v4(verbose=verbose).forward_v4(query, key_cache, value_cache, block_tables,
                                               seq_lens, page_size, chunk_keys, max_seq_len)


def forward_v5(query, key_cache, value_cache, block_tables, seq_lens, page_size: int,
               chunk_keys: Optional[int] = 512, token_group: int = 2, max_seq_len: int = 0,
               verbose: bool = False):
    """Reference ``forward_v5`` (``cuda.py:297-336``); ``token_group`` checked, then unused."""
    if token_group in (2, 4):
        out = _fast(query, key_cache, value_cache, block_tables, seq_lens, page_size, chunk_keys,
                    max_seq_len or -1, True)
        if out is not None:
            return out
    _check_python_contract("v5", query, key_cache, value_cache, block_tables, seq_lens, True)
    if token_group not in (2, 4):
        raise ValueError("v5 token_group must be 2 or 4")
    if chunk_keys is not None and chunk_keys <= 0:
        raise ValueError("chunk_keys must be positive")
    return load_v5(verbose=verbose).forward_v5(query, key_cache, value_cache, block_tables,
                                               seq_lens, page_size, chunk_keys, token_group,
                                               max_seq_len)


__all__ = [
    "load_v0", "load_v1", "load_v2", "load_v3", "load_v4", "load_v5",
    "forward_v0", "forward_v1", "forward_v2", "forward_v3", "forward_v4", "forward_v5",
    "paged_mtp_attention",
]
