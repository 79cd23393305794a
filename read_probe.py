"""The streaming-read probe bench.py reports beside the roofline (``read_probe.hip``),
built into its own library, ``libsqa_probe.so`` beside this file, with the same
hipcc flags and source-hash stamp as ``libsqa.so``. A measurement aid: nothing in
``small_q_attention_amd`` loads it.

    python read_probe.py        # build libsqa_probe.so
"""

from __future__ import annotations

import ctypes
import hashlib
import os
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent
SOURCE = ROOT / "read_probe.hip"
LIB_PATH = ROOT / "libsqa_probe.so"

_LIB = None


def _flags():
    if str(ROOT) not in sys.path:
        sys.path.insert(0, str(ROOT))
    from small_q_attention_amd import build as sqa_build

    return sqa_build


def source_hash() -> str:
    b = _flags()
    h = hashlib.sha256()
    h.update("\0".join(b.FLAGS).encode())
    h.update(b"\0" + SOURCE.name.encode() + b"\0" + SOURCE.read_bytes())
    return h.hexdigest()[:b.HASH_LEN]


def build(verbose: bool = False) -> Path:
    """Compile ``libsqa_probe.so`` (always)."""
    b = _flags()
    tmp = LIB_PATH.with_name(f"{LIB_PATH.name}.tmp{os.getpid()}")
    cmd = [b.hipcc_path(), *b.FLAGS, f'-DSQA_SOURCE_HASH="{source_hash()}"', str(SOURCE),
           "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        tmp.unlink(missing_ok=True)
        errors = [ln for ln in (res.stdout + res.stderr).splitlines()
                  if "packed-fp32-ops" not in ln and "unknown target feature" not in ln.lower()]
        raise RuntimeError("hipcc failed building libsqa_probe.so:\n" + "\n".join(errors))
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def load(build_if_missing: bool = True):
    """The probe library, built first if missing or stale (else ``RuntimeError``)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if _flags().built_hash(LIB_PATH) != source_hash():
        if not build_if_missing:
            raise RuntimeError(f"{LIB_PATH.name} is missing or stale; run `python read_probe.py`")
        build()
    lib = ctypes.CDLL(str(LIB_PATH))
    lib.sqa_read_probe.restype = ctypes.c_int
    lib.sqa_read_probe.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                   ctypes.c_int, ctypes.c_void_p]
    lib.sqa_probe_last_error.restype = ctypes.c_char_p
    lib.sqa_probe_version.restype = ctypes.c_char_p
    _LIB = lib
    return lib


def read_probe(data, sink, blocks: int, stream_handle: int, lib=None) -> None:
    """One pass of the probe over the bytes of the contiguous tensor ``data``
    (``blocks`` chunks), one folded dword per thread into ``sink`` (``blocks * 256``
    int32). Raises ``RuntimeError`` with the library's message on a bad argument."""
    lib = lib or load(build_if_missing=False)
    if not data.is_contiguous() or sink.numel() < blocks * 256:
        raise ValueError("data must be contiguous and sink hold blocks * 256 dwords")
    rc = lib.sqa_read_probe(data.data_ptr(), data.numel() * data.element_size(),
                            sink.data_ptr(), blocks, stream_handle)
    if rc != 0:
        raise RuntimeError(f"sqa_read_probe failed: {lib.sqa_probe_last_error().decode()}")


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
