"""The reference's import path ``small_q_attention.cuda`` resolves to this build.

Every reference caller imports the op as ``from small_q_attention.cuda import
forward_vN`` (``/root/reference/scripts/run_gpu_matrix.py:19-26``,
``scripts/build_and_test_v0.py:11``, ``build_and_test_v3.py:17``,
``build_and_test_v5.py:10``). The alias must hand back the very functions of
``small_q_attention_amd.cuda`` and must not pull in the CPU oracle.
"""

import importlib
import inspect
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
NAMES = [f"forward_v{i}" for i in range(6)] + [f"load_v{i}" for i in range(6)]


def test_reference_import_lines_resolve_to_this_build():
    from small_q_attention.cuda import (  # noqa: F401  (the reference's own import lines)
        forward_v0, forward_v1, forward_v2, forward_v3, forward_v4, forward_v5)
    import small_q_attention.cuda as alias
    import small_q_attention_amd.cuda as native

    for name in NAMES:
        assert getattr(alias, name) is getattr(native, name), name


def test_alias_signatures_are_the_reference_signatures():
    """reference cuda.py:61,81,120-129,177-187,238-248,297-308."""
    import small_q_attention.cuda as alias

    assert list(inspect.signature(alias.forward_v1).parameters) == [
        "query", "key_cache", "value_cache", "block_tables", "seq_lens", "page_size", "verbose"]
    params = inspect.signature(alias.forward_v5).parameters
    assert list(params) == ["query", "key_cache", "value_cache", "block_tables", "seq_lens",
                            "page_size", "chunk_keys", "token_group", "max_seq_len", "verbose"]
    assert params["chunk_keys"].default == 512 and params["token_group"].default == 2
    assert params["max_seq_len"].default == 0


def test_alias_does_not_import_the_oracle():
    """In a fresh interpreter, importing the alias loads no module of ``oracle``."""
    code = ("import sys; import small_q_attention, small_q_attention.cuda; "
            "bad = [m for m in sys.modules if m == 'oracle' or m.startswith('oracle.')]; "
            "print(bad); sys.exit(1 if bad else 0)")
    res = subprocess.run([sys.executable, "-c", code], cwd=ROOT, capture_output=True, text=True)
    assert res.returncode == 0, res.stdout + res.stderr


def test_oracle_name_points_to_the_test_package():
    mod = importlib.import_module("small_q_attention")
    with pytest.raises(ImportError, match="oracle.paged_mtp_attention_reference"):
        mod.paged_mtp_attention_reference  # noqa: B018
    with pytest.raises(AttributeError):
        mod.no_such_name  # noqa: B018
