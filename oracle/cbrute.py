"""ctypes front end of the double-precision C brute force (``oracle/sqa_oracle.c``).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "libsqa_oracle.so"
_LIB = None


def build(verbose: bool = False) -> Path:
    """Compile ``libsqa_oracle.so`` next to its source with the committed Makefile."""
    cmd = ["make", "-C", str(_HERE), "-B", "libsqa_oracle.so"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if verbose or res.returncode:
        print(res.stdout + res.stderr)
    if res.returncode:
        raise RuntimeError("building the C oracle failed")
    return _LIB_PATH


def _load():
    global _LIB
    if _LIB is None:
        if not _LIB_PATH.exists():
            build()
        lib = ctypes.CDLL(str(_LIB_PATH))
        lib.sqa_oracle_f64.restype = ctypes.c_int
        lib.sqa_oracle_f64.argtypes = [ctypes.c_void_p] * 6 + [ctypes.c_int] * 7 + [ctypes.c_longlong]
        lib.sqa_oracle_f64_ex.restype = ctypes.c_int
        lib.sqa_oracle_f64_ex.argtypes = (
            [ctypes.c_void_p] * 3 + [ctypes.c_longlong] * 3 + [ctypes.c_void_p] * 3
            + [ctypes.c_int, ctypes.c_double, ctypes.c_double, ctypes.c_int, ctypes.c_int,
               ctypes.c_void_p]
            + [ctypes.c_int] * 7 + [ctypes.c_longlong])
        lib.sqa_oracle_half_to_double.restype = ctypes.c_double
        lib.sqa_oracle_half_to_double.argtypes = [ctypes.c_uint16]
        lib.sqa_oracle_bf16_to_double.restype = ctypes.c_double
        lib.sqa_oracle_bf16_to_double.argtypes = [ctypes.c_uint16]
        lib.sqa_oracle_fp8_to_double.restype = ctypes.c_double
        lib.sqa_oracle_fp8_to_double.argtypes = [ctypes.c_uint8]
        _LIB = lib
    return _LIB


def c_oracle_available() -> bool:
    try:
        _load()
        return True
    except (OSError, RuntimeError):
        return False


def _as_np(x, dtype):
    if hasattr(x, "detach"):
        x = x.detach()
        if x.device.type != "cpu":
            x = x.cpu()
        x = x.contiguous().numpy()
    return np.ascontiguousarray(np.asarray(x), dtype=dtype)


def _is_bf16(x):
    return hasattr(x, "dtype") and str(x.dtype) == "torch.bfloat16"


def _is_fp8(x):
    return hasattr(x, "dtype") and str(x.dtype) == "torch.float8_e4m3fn"


def _bits(x):
    """Torch fp16/bf16/e4m3 tensor -> numpy uint16 (uint8 for e4m3) bit patterns with
    the same strides; numpy fp16 arrays pass through."""
    if hasattr(x, "detach"):
        x = x.detach()
        if x.device.type != "cpu":
            x = x.cpu()
        if _is_bf16(x) or _is_fp8(x):
            import torch

            if _is_fp8(x):
                return x.view(torch.uint8).numpy()
            return x.view(torch.int16).numpy().view(np.uint16)
        x = x.numpy()
    x = np.asarray(x)
    if x.dtype not in (np.float16, np.uint16, np.uint8):
        x = x.astype(np.float16)
    return x


def _strided_half(x):
    """fp16/bf16/e4m3 ``[P, page, Hkv, D]`` view (torch or numpy, any positive strides,
    contiguous D) -> (numpy view of the bit patterns, strides in elements)."""
    x = _bits(x)
    size = x.itemsize
    if x.ndim != 4 or x.strides[3] != size or min(x.strides) <= 0:
        x = np.ascontiguousarray(x)
    return x, tuple(st // size for st in x.strides[:3])


def attention_c64(query, key_cache, value_cache, block_tables, seq_lens, page_size, num_kv_heads,
                  draft_mask=None, scale=None, out_scale=1.0):
    """fp16 inputs -> float64 ``[B, Q, Hq, D]`` output, computed in double.

    ``key_cache``/``value_cache``: ``[P, page, Hkv, D]`` with any positive strides (so the
    halves of an interleaved cache are read in place). ``draft_mask``: ``None`` (causal
    draft chain) or packed words ``[B, Q, W]`` (uint32/int32) or ``[B, Q, 2W]`` (uint16).
    ``scale`` defaults to ``D**-0.5``; ``out_scale`` multiplies the output.
    """
    lib = _load()
    bf16 = _is_bf16(query)
    kv_fp8 = _is_fp8(key_cache)
    if kv_fp8 != _is_fp8(value_cache):
        raise ValueError("key and value caches must share the element type")
    if not kv_fp8 and (bf16 != _is_bf16(key_cache) or bf16 != _is_bf16(value_cache)):
        raise ValueError("query and caches must share the element type (or caches in e4m3)")
    kv_elem = 2 if kv_fp8 else int(bf16)
    q = np.ascontiguousarray(_bits(query))
    k, kst = _strided_half(key_cache)
    v, vst = _strided_half(value_cache)
    bt = _as_np(block_tables, np.int32)
    sl = _as_np(seq_lens, np.int32)
    n_batch, q_len, n_qheads, dim = q.shape
    if k.shape[1:] != (page_size, num_kv_heads, dim) or v.shape != k.shape:
        raise ValueError("cache shape does not match page_size / num_kv_heads / head_dim")
    if kst != vst:
        v = np.ascontiguousarray(v)
        k = np.ascontiguousarray(k)
        kst = vst = tuple(st // k.itemsize for st in k.strides[:3])
    words, n_words = None, 0
    if draft_mask is not None:
        m = draft_mask
        if hasattr(m, "detach"):
            m = m.detach().cpu().numpy()
        m = np.ascontiguousarray(np.asarray(m))
        if m.dtype in (np.uint16, np.int16):
            m = m.view(np.uint16)
        words = np.ascontiguousarray(m.view(np.uint32))
        n_words = words.shape[-1]
        if words.shape[:2] != (n_batch, q_len) or n_words * 32 < q_len:
            raise ValueError("draft_mask must be [B, Q, ceil(Q / 32)] words")
    out = np.empty(q.shape, dtype=np.float64)
    ptr = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    rc = lib.sqa_oracle_f64_ex(
        ptr(q), ptr(k), ptr(v), kst[0], kst[1], kst[2], ptr(bt), ptr(sl),
        ptr(words) if words is not None else None, n_words,
        float(dim ** -0.5 if scale is None else scale), float(out_scale), int(bf16), kv_elem,
        ptr(out),
        n_batch, q_len, n_qheads, num_kv_heads, dim, page_size, bt.shape[1], k.shape[0])
    if rc == -1:
        raise IndexError("block table holds a page id outside the cache")
    if rc == -2:
        raise ValueError("a sequence needs more pages than block_tables holds")
    return out
