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


def test_unloadable_library_raises(fresh_loader, monkeypatch):
    fresh_loader.write_bytes(b"not a shared object")
    with pytest.raises(RuntimeError, match="cannot load"):
        _lib.load(build_if_missing=False)

    # Every entry point goes through the same loader (the plan helper's cache is
    # bypassed so an earlier cached plan cannot answer instead); the unstamped
    # file would be rebuilt, and a failing build surfaces as RuntimeError.
    def failing_build(verbose=False):
        raise RuntimeError("hipcc failed building libsqa.so")

    monkeypatch.setattr(_build, "build", failing_build)
    with pytest.raises(RuntimeError):
        _lib.plan_splits.__wrapped__(0, 1, 2, 32, 8, 128, 64, 4, 0)


def test_verbose_load_echoes_the_build(capsys):
    from small_q_attention_amd import cuda as sqa

    sqa.load_v3(verbose=True)
    out = capsys.readouterr().out
    assert "libsqa.so" in out and "hipcc" in out and "--offload-arch=gfx950" in out


def test_built_library_carries_the_source_hash():
    """The library on disk and the one loaded both name the hash of the sources beside them."""
    _lib.load()
    assert _build.built_hash() == _build.source_hash()
    assert f"sqa-src-hash:{_build.source_hash()}" in _lib.load().sqa_version().decode()
    assert not _build.is_stale()


def test_stale_library_raises_without_build(fresh_loader, monkeypatch):
    """A library built from other sources is refused (no silent load of old code)."""
    import shutil

    shutil.copy(_build.PKG_DIR / "libsqa.so", fresh_loader)
    monkeypatch.setattr(_build, "source_hash", lambda: "0123456789abcdef")
    with pytest.raises(RuntimeError, match="stale"):
        _lib.load(build_if_missing=False)


def test_stale_library_is_rebuilt(fresh_loader, monkeypatch):
    """With building allowed, a stale library is rebuilt before it is loaded."""
    import shutil

    shutil.copy(_build.PKG_DIR / "libsqa.so", fresh_loader)
    calls = []

    def fake_build(verbose=False):
        calls.append(verbose)
        return fresh_loader

    monkeypatch.setattr(_build, "source_hash", lambda: "0123456789abcdef")
    monkeypatch.setattr(_build, "build", fake_build)
    # The copied library still carries the real hash, so after the (stubbed)
    # rebuild the loader's own version check reports the mismatch.
    with pytest.raises(RuntimeError, match="0123456789abcdef"):
        _lib.load()
    assert calls == [False]


def test_source_edit_changes_the_hash(monkeypatch, tmp_path):
    """Touching the bytes of any source changes the hash the loader compares."""
    src = tmp_path / "sqa_kernels.hip"
    src.write_bytes(_build.SOURCES[0].read_bytes())
    monkeypatch.setattr(_build, "SOURCES", [src] + list(_build.SOURCES[1:]))
    before = _build.source_hash()
    src.write_bytes(src.read_bytes() + b"\n// edit\n")
    assert _build.source_hash() != before
