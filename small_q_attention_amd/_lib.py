"""ctypes binding of ``libsqa.so`` (C ABI in ``include/sqa.h``) and the torch custom op.

There is no fallback: if the library is missing or fails to load, every entry
point raises ``RuntimeError``.
"""

from __future__ import annotations

import ctypes
import functools
import threading
from pathlib import Path

from . import build as _build

_LOCK = threading.Lock()
_LIB = None

SQA_OK = 0

# (name, restype, argtypes) for every symbol include/sqa.h declares.
_C = ctypes
_SIGNATURES = [
    ("sqa_plan_splits", _C.c_int,
     [_C.c_int] * 9 + [_C.POINTER(_C.c_int), _C.POINTER(_C.c_int)]),
    ("sqa_workspace_bytes", _C.c_size_t, [_C.c_int] * 7),
    ("sqa_paged_mtp_attention", _C.c_int,
     [_C.c_void_p] * 7 + [_C.c_size_t] + [_C.c_int] * 5 + [_C.c_int64] + [_C.c_int] * 4
     + [_C.c_void_p, _C.c_void_p]),
    ("sqa_paged_mtp_attention_noalloc", _C.c_int,
     [_C.c_void_p] * 6 + [_C.c_int] * 5 + [_C.c_int64] + [_C.c_int] * 4 + [_C.c_void_p]),
    ("sqa_paged_attention", _C.c_int, [_C.c_void_p]),
    ("sqa_device_cu_count", _C.c_int, [_C.c_int]),
    ("sqa_last_error", _C.c_char_p, []),
    ("sqa_version", _C.c_char_p, []),
]
EXPORTED = [name for name, _, _ in _SIGNATURES]


class KVCache(ctypes.Structure):
    """``sqa_kv_cache`` of include/sqa.h (strides in fp16 elements)."""

    _fields_ = [("k", _C.c_void_p), ("v", _C.c_void_p), ("num_pages", _C.c_int64),
                ("page_stride", _C.c_int64), ("token_stride", _C.c_int64),
                ("head_stride", _C.c_int64)]


class AttentionArgs(ctypes.Structure):
    """``sqa_attention_args`` of include/sqa.h."""

    _fields_ = [("struct_size", _C.c_size_t), ("query", _C.c_void_p), ("output", _C.c_void_p),
                ("kv", KVCache), ("block_tables", _C.c_void_p), ("seq_lens", _C.c_void_p),
                ("max_pages", _C.c_int), ("draft_mask", _C.c_void_p), ("mask_words", _C.c_int),
                ("scale", _C.c_float), ("out_scale", _C.c_float), ("batch", _C.c_int),
                ("q_len", _C.c_int), ("num_query_heads", _C.c_int), ("num_kv_heads", _C.c_int),
                ("head_dim", _C.c_int), ("page_size", _C.c_int), ("num_splits", _C.c_int),
                ("pages_per_split", _C.c_int), ("workspace", _C.c_void_p),
                ("workspace_bytes", _C.c_size_t), ("stream", _C.c_void_p),
                ("timing_events", _C.c_void_p), ("dtype", _C.c_int), ("kv_dtype", _C.c_int),
                ("flags", _C.c_int)]


DTYPE_F16, DTYPE_BF16, DTYPE_FP8_E4M3 = 0, 1, 2
FLAG_ADAPTIVE_PAIRS = 1  # SQA_FLAG_ADAPTIVE_PAIRS


def library_path() -> Path:
    return _build.LIB_PATH


def load(verbose: bool = False, build_if_missing: bool = True):
    """Load ``libsqa.so``, building it first if it is missing or was built from other
    sources (the source hash stamped into the library differs from the hash of the
    sources beside it). With ``build_if_missing=False`` either case raises
    ``RuntimeError`` instead. ``verbose`` echoes the library path and the hipcc
    command that builds it, as the reference's loaders echo their JIT build
    (``cuda.py:31-36``)."""
    global _LIB
    if verbose:
        print(f"[sqa] {_build.LIB_PATH}; build command: {' '.join(_build.build_command())}",
              flush=True)
    with _LOCK:
        if _LIB is None:
            path = _build.LIB_PATH
            want = _build.source_hash()
            have = _build.built_hash(path) if path.exists() else None
            if have != want:
                if build_if_missing:
                    _build.build(verbose=verbose)
                elif not path.exists():
                    raise RuntimeError(f"{path} is not built; run small_q_attention_amd.build")
                elif have is not None:
                    raise RuntimeError(f"{path} is stale (built from sources {have}, sources "
                                       f"now {want}); run small_q_attention_amd.build")
                # An unstamped file: loading it below fails, or its version check does.
            try:
                lib = ctypes.CDLL(str(path))
            except OSError as exc:
                raise RuntimeError(f"cannot load {path}: {exc}") from exc
            for name, res, args in _SIGNATURES:
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            version = lib.sqa_version().decode(errors="replace")
            if f"sqa-src-hash:{want}" not in version:
                raise RuntimeError(f"{path} reports '{version}', not the sources' hash {want}; "
                                   "rebuild with small_q_attention_amd.build")
            _LIB = lib
        return _LIB


def last_error(lib) -> str:
    msg = lib.sqa_last_error()
    return msg.decode() if msg else "unknown error"


@functools.lru_cache(maxsize=4096)
def plan_splits(device_index: int, batch: int, q_len: int, num_query_heads: int,
                num_kv_heads: int, head_dim: int, max_seq_len: int, max_pages: int,
                chunk_keys: int):
    """``sqa_plan_splits`` -> ``(num_splits, pages_per_split)``; memoised (the plan is a
    pure function of its arguments and the device's CU count)."""
    lib = load()
    ns, pps = ctypes.c_int(0), ctypes.c_int(0)
    rc = lib.sqa_plan_splits(device_index, batch, q_len, num_query_heads, num_kv_heads,
                             head_dim, max_seq_len, max_pages, chunk_keys, ctypes.byref(ns),
                             ctypes.byref(pps))
    if rc != SQA_OK:
        raise RuntimeError(f"sqa_plan_splits failed: {last_error(lib)}")
    return ns.value, pps.value


@functools.lru_cache(maxsize=4096)
def workspace_bytes(batch: int, q_len: int, num_query_heads: int, num_kv_heads: int,
                    head_dim: int, num_splits: int, pages_per_split: int) -> int:
    """Workspace of a plan from :func:`plan_splits` (``pages_per_split`` 0 = balanced)."""
    return int(load().sqa_workspace_bytes(batch, q_len, num_query_heads, num_kv_heads, head_dim,
                                          num_splits, pages_per_split))


def raw_stream(device_index: int) -> int:
    """Handle of torch's current stream on ``device_index`` (a ``hipStream_t`` as int)."""
    import torch

    getter = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    if getter is not None:
        return getter(device_index)
    return torch.cuda.current_stream(device_index).cuda_stream


def launch(query, key_cache, value_cache, block_tables, seq_lens, output, workspace,
           num_splits: int, pages_per_split: int, stream_handle: int, timing_events=None):
    """Call ``sqa_paged_mtp_attention`` on raw device pointers of torch tensors.

    The entry point reads fp16 elements through bare pointers, so any other
    element type (a bf16 or e4m3 cache: :func:`launch_general`) is refused here
    before the call; a 1-byte cache read as fp16 would run past its end."""
    for name, t in (("query", query), ("key_cache", key_cache), ("value_cache", value_cache),
                    ("output", output)):
        if str(t.dtype) != "torch.float16":
            raise TypeError(f"sqa_paged_mtp_attention takes fp16 tensors; {name} is {t.dtype} "
                            "(bf16 or e4m3 caches go through launch_general)")
    lib = _LIB if _LIB is not None else load()
    b, q_len, hq, d = query.shape
    ev = None
    if timing_events is not None:
        ev = (ctypes.c_void_p * 3)(*[ctypes.c_void_p(int(e)) for e in timing_events])
    ws_ptr = workspace.data_ptr() if workspace is not None else None
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    kshape = key_cache.shape
    rc = lib.sqa_paged_mtp_attention(
        query.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(),
        block_tables.data_ptr(), seq_lens.data_ptr(), output.data_ptr(),
        ws_ptr, ws_bytes, b, q_len, hq, kshape[2], d,
        kshape[0], kshape[1], block_tables.shape[1],
        num_splits, pages_per_split, stream_handle, ev)
    if rc != SQA_OK:
        raise RuntimeError(f"sqa_paged_mtp_attention failed: {last_error(lib)}")


def kv_cache(k_view, v_view) -> KVCache:
    """Describe a paged cache from two ``[num_pages, page, Hkv, D]`` views of any strides
    (separate caches, or the K / V halves of an interleaved NHD or HND cache). The head
    dimension must be contiguous and K and V must share strides."""
    if k_view.dim() != 4 or v_view.shape != k_view.shape:
        raise ValueError("K and V views must both be [num_pages, page, Hkv, D]")
    if k_view.stride() != v_view.stride() or k_view.stride(3) != 1:
        raise ValueError("K and V views must share strides with a contiguous head dimension")
    return KVCache(k_view.data_ptr(), v_view.data_ptr(), k_view.shape[0], k_view.stride(0),
                   k_view.stride(1), k_view.stride(2))


def launch_general(query, output, k_view, v_view, block_tables, seq_lens, draft_mask,
                   scale: float, out_scale: float, num_splits: int, pages_per_split: int,
                   workspace, stream_handle: int, timing_events=None, flags: int = 0):
    """Call ``sqa_paged_attention``. ``query``/``output``: contiguous ``[B, Q, Hq, D]``;
    ``k_view``/``v_view``: see :func:`kv_cache`; ``draft_mask``: ``None`` (causal draft
    chain) or a contiguous 32-bit ``[B, Q, W]`` tensor of packed draft bits; ``flags``:
    0 or :data:`FLAG_ADAPTIVE_PAIRS`."""
    lib = _LIB if _LIB is not None else load()
    b, q_len, hq, d = query.shape
    a = AttentionArgs()
    a.struct_size = ctypes.sizeof(AttentionArgs)
    a.query, a.output = query.data_ptr(), output.data_ptr()
    a.kv = kv_cache(k_view, v_view)
    a.block_tables, a.seq_lens = block_tables.data_ptr(), seq_lens.data_ptr()
    a.max_pages = block_tables.shape[1]
    if draft_mask is not None:
        a.draft_mask, a.mask_words = draft_mask.data_ptr(), draft_mask.shape[-1]
    a.scale, a.out_scale = float(scale), float(out_scale)
    a.batch, a.q_len, a.num_query_heads, a.num_kv_heads = b, q_len, hq, k_view.shape[2]
    a.head_dim, a.page_size = d, k_view.shape[1]
    a.num_splits, a.pages_per_split = num_splits, pages_per_split
    if workspace is not None:
        a.workspace = workspace.data_ptr()
        a.workspace_bytes = workspace.numel() * workspace.element_size()
    a.stream = stream_handle
    a.dtype = DTYPE_BF16 if str(query.dtype) == "torch.bfloat16" else DTYPE_F16
    a.kv_dtype = DTYPE_FP8_E4M3 if str(k_view.dtype) == "torch.float8_e4m3fn" else a.dtype
    a.flags = int(flags)
    ev = None
    if timing_events is not None:
        ev = (ctypes.c_void_p * 3)(*[ctypes.c_void_p(int(e)) for e in timing_events])
        a.timing_events = ctypes.cast(ev, ctypes.c_void_p)
    rc = lib.sqa_paged_attention(ctypes.byref(a))
    if rc != SQA_OK:
        raise RuntimeError(f"sqa_paged_attention failed: {last_error(lib)}")


def run(query, key_cache, value_cache, block_tables, seq_lens, num_splits: int,
        pages_per_split: int):
    """Allocate the output with torch's caching allocator, take a workspace from
    :func:`workspace_for`, and launch on the current stream of the query's device.
    Returns the output."""
    import torch

    out = torch.empty_like(query)
    b, q_len, hq, d = query.shape
    nbytes = workspace_bytes(b, q_len, hq, key_cache.shape[2], d, num_splits, pages_per_split)
    stream = raw_stream(query.device.index)
    ws = workspace_for(nbytes, query, query.device.index, stream) if nbytes else None
    if query.dtype == torch.float16:
        launch(query, key_cache, value_cache, block_tables, seq_lens, out, ws, num_splits,
               pages_per_split, stream)
    else:  # bf16: the general entry point carries the element type
        launch_general(query, out, key_cache, value_cache, block_tables, seq_lens, None,
                       query.shape[-1] ** -0.5, 1.0, num_splits, pages_per_split, ws, stream)
    return out


# Workspaces kept per (device, stream) for eager calls: a stream runs its calls in
# order, so one buffer serves them all and the per-call allocation is saved.
# Plans past WORKSPACE_CACHE_BYTES, and calls under graph capture (whose buffers
# belong to the graph's pool), allocate their own.
WORKSPACE_CACHE_BYTES = 64 << 20
_WORKSPACES = {}
_CUDA_STATE = None  # (current device, current stream capturing): torch's own query functions


def _cuda_state(torch):
    """The functions behind ``torch.cuda.current_device`` and
    ``torch.cuda.is_current_stream_capturing`` without their per-call
    initialisation checks (callers hold a CUDA tensor, so CUDA is initialised);
    the public ones where this torch lacks them."""
    global _CUDA_STATE
    if _CUDA_STATE is None:
        c = torch._C
        _CUDA_STATE = (getattr(c, "_cuda_getDevice", None) or torch.cuda.current_device,
                       getattr(c, "_cuda_isCurrentStreamCapturing", None)
                       or torch.cuda.is_current_stream_capturing)
    return _CUDA_STATE


def workspace_for(nbytes: int, like, device_index: int, stream_handle: int):
    """A workspace of at least ``nbytes`` for a call on ``stream_handle`` (``like``: a
    tensor on the call's device)."""
    import torch

    current_device, capturing = _CUDA_STATE or _cuda_state(torch)
    # The capture check reads the current device's stream: the cache serves only
    # calls on that device.
    if nbytes > WORKSPACE_CACHE_BYTES or device_index != current_device() or capturing():
        return torch.empty(nbytes, dtype=torch.uint8, device=like.device)
    key = (device_index, stream_handle)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=like.device)
        _WORKSPACES[key] = ws
    return ws


def run_fp16(query, key_cache, value_cache, block_tables, seq_lens, batch: int, q_len: int,
             num_query_heads: int, num_kv_heads: int, num_pages: int, page_size: int,
             max_pages: int, num_splits: int, pages_per_split: int, device_index: int):
    """:func:`run` for the fp16, head-dim-128 call whose shapes the caller has already
    checked and unpacked: the same allocation and launch with fewer Python steps."""
    import torch

    out = torch.empty_like(query)
    nbytes = workspace_bytes(batch, q_len, num_query_heads, num_kv_heads, 128, num_splits,
                             pages_per_split)
    stream = raw_stream(device_index)
    ws = workspace_for(nbytes, query, device_index, stream) if nbytes else None
    rc = _LIB.sqa_paged_mtp_attention(
        query.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(),
        block_tables.data_ptr(), seq_lens.data_ptr(), out.data_ptr(),
        ws.data_ptr() if ws is not None else None, nbytes, batch, q_len, num_query_heads,
        num_kv_heads, 128, num_pages, page_size, max_pages, num_splits, pages_per_split,
        stream, None)
    if rc != SQA_OK:
        raise RuntimeError(f"sqa_paged_mtp_attention failed: {last_error(_LIB)}")
    return out


def custom_op():
    """The ``sqa::paged_mtp_attention`` torch custom op (registered on first use)."""
    from . import _op

    return _op.paged_mtp_attention
