"""The library path has no fallback: a missing or unloadable ``libsqa.so`` raises
``RuntimeError`` (CPU checks; the loader state is restored afterwards)."""

import pytest

from small_q_attention_amd import _lib, build as _build


@pytest.fixture
def fresh_loader(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_LIB", None)
    path = tmp_path / "libsqa.so"
    monkeypatch.setattr(_build, "LIB_PATH", path)
    return path


def test_missing_library_raises(fresh_loader):
    with pytest.raises(RuntimeError, match="not built"):
        _lib.load(build_if_missing=False)


def test_unloadable_library_raises(fresh_loader):
    fresh_loader.write_bytes(b"not a shared object")
    with pytest.raises(RuntimeError, match="cannot load"):
        _lib.load(build_if_missing=False)
    # Every entry point goes through the same loader (the plan helper's cache is
    # bypassed so an earlier cached plan cannot answer instead).
    with pytest.raises(RuntimeError):
        _lib.plan_splits.__wrapped__(0, 1, 2, 32, 8, 128, 64, 4, 0)


def test_verbose_load_echoes_the_build(capsys):
    from small_q_attention_amd import cuda as sqa

    sqa.load_v3(verbose=True)
    out = capsys.readouterr().out
    assert "libsqa.so" in out and "hipcc" in out and "--offload-arch=gfx950" in out
