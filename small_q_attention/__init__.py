"""Drop-in import path of the reference package (``small_q_attention``).

The reference's callers import the GPU op as ``from small_q_attention.cuda
import forward_v0, ...`` (``/root/reference/scripts/run_gpu_matrix.py:19-26``,
``scripts/build_and_test_v3.py:17``). :mod:`small_q_attention.cuda` re-exports
those names from :mod:`small_q_attention_amd.cuda`, so such callers run the
gfx950 kernels of ``libsqa.so`` unchanged.

The reference package also exports its CPU oracle
``paged_mtp_attention_reference`` (``src/small_q_attention/__init__.py:3``).
This build ships only the GPU op: the CPU restatement of that oracle is test
infrastructure in the top-level ``oracle`` package, which nothing here imports.
Asking this package for it raises ``ImportError`` with that pointer.
"""

from __future__ import annotations

__all__: list = []

_ORACLE_NAMES = ("paged_mtp_attention_reference",)


def __getattr__(name):
    if name in _ORACLE_NAMES:
        raise ImportError(
            f"{name} is the reference's CPU oracle; this package ships only the GPU op. "
            f"Its test-only restatement is oracle.{name} (the top-level oracle package).")
    raise AttributeError(f"module 'small_q_attention' has no attribute {name!r}")
