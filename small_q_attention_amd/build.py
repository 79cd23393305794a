"""Builds ``libsqa.so`` (the gfx950 HIP library) in-tree with hipcc.

The reference JIT-compiles its CUDA source through
``torch.utils.cpp_extension.load`` on the first ``load_vN`` call
(``/root/reference/src/small_q_attention/cuda.py:16-37``). Here the library is
one plain shared object with a C ABI, compiled once for gfx950 by hipcc; every
``load_vN`` returns a handle to the same library.

The library carries the SHA-256 (first 16 hex digits) of its sources, headers
and compiler flags, both as the string ``sqa-src-hash:<hash>`` inside
``sqa_version()`` and as bytes of the file, so a loader can tell, before
``dlopen``, whether the library on disk was built from the sources beside it
(the reference's loaders rebuild through torch's extension cache keyed the same
way, ``cuda.py:16-37``).
"""

from __future__ import annotations

import hashlib
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO_DIR / "include"
LIB_PATH = PKG_DIR / "libsqa.so"
SOURCES = [CSRC / "sqa_kernels.hip", CSRC / "sqa_capi.hip"]
HEADERS = [CSRC / "sqa_internal.h", INCLUDE / "sqa.h"]
ARCH = "gfx950"


def hipcc_path() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; ROCm is required to build libsqa.so")


FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # Packed fp32 VALU ops are kept out of the generated code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA operands and results in VGPRs: the softmax reads every score and
    # rescales every accumulator with VALU ops, and with the default AGPR
    # form each of those costs a copy (q16: ~1500 copies per 3 pages,
    # 375 -> 334 us at KV 32K x B16).
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]
HASH_MARKER = b"sqa-src-hash:"
HASH_LEN = 16


def source_hash() -> str:
    """SHA-256 (first 16 hex digits) over the compiler flags and the name and bytes of
    every source and header the library is built from."""
    h = hashlib.sha256()
    h.update("\0".join(FLAGS).encode())
    for path in SOURCES + HEADERS:
        h.update(b"\0" + path.name.encode() + b"\0")
        h.update(path.read_bytes())
    return h.hexdigest()[:HASH_LEN]


def build_command(output: Path = LIB_PATH, src_hash: str = ""):
    return [
        hipcc_path(),
        *FLAGS,
        f'-DSQA_SOURCE_HASH="{src_hash or source_hash()}"',
        f"-I{INCLUDE}",
        f"-I{CSRC}",
        *[str(s) for s in SOURCES],
        "-o", str(output),
    ]


def built_hash(path: Path = LIB_PATH):
    """The source hash stamped into a built library, or None (missing or unstamped)."""
    try:
        data = path.read_bytes()
    except OSError:
        return None
    i = data.find(HASH_MARKER)
    if i < 0:
        return None
    stamp = data[i + len(HASH_MARKER):i + len(HASH_MARKER) + HASH_LEN]
    try:
        return stamp.decode("ascii")
    except UnicodeDecodeError:
        return None


def is_stale() -> bool:
    """True when the library is missing or was built from other sources or flags."""
    return built_hash(LIB_PATH) != source_hash()


def build(verbose: bool = False) -> Path:
    """Compile ``libsqa.so`` (always; callers decide whether a rebuild is due)."""
    tmp = LIB_PATH.with_name(f"{LIB_PATH.name}.tmp{os.getpid()}")
    cmd = build_command(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    errors = [ln for ln in (res.stdout + res.stderr).splitlines()
              if "packed-fp32-ops" not in ln and "unknown target feature" not in ln.lower()]
    if res.returncode != 0:
        tmp.unlink(missing_ok=True)
        raise RuntimeError("hipcc failed building libsqa.so:\n" + "\n".join(errors))
    if verbose and errors:
        print("\n".join(errors), flush=True)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print(LIB_PATH)
