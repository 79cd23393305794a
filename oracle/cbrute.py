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
        lib.sqa_oracle_half_to_double.restype = ctypes.c_double
        lib.sqa_oracle_half_to_double.argtypes = [ctypes.c_uint16]
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


def attention_c64(query, key_cache, value_cache, block_tables, seq_lens, page_size, num_kv_heads):
    """fp16 inputs -> float64 ``[B, Q, Hq, D]`` output, computed in double."""
    lib = _load()
    q = _as_np(query, np.float16)
    k = _as_np(key_cache, np.float16)
    v = _as_np(value_cache, np.float16)
    bt = _as_np(block_tables, np.int32)
    sl = _as_np(seq_lens, np.int32)
    n_batch, q_len, n_qheads, dim = q.shape
    if k.shape[1:] != (page_size, num_kv_heads, dim) or v.shape != k.shape:
        raise ValueError("cache shape does not match page_size / num_kv_heads / head_dim")
    out = np.empty(q.shape, dtype=np.float64)
    ptr = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    rc = lib.sqa_oracle_f64(ptr(q), ptr(k), ptr(v), ptr(bt), ptr(sl), ptr(out),
                            n_batch, q_len, n_qheads, num_kv_heads, dim, page_size,
                            bt.shape[1], k.shape[0])
    if rc == -1:
        raise IndexError("block table holds a page id outside the cache")
    if rc == -2:
        raise ValueError("a sequence needs more pages than block_tables holds")
    return out
