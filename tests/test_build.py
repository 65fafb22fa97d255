"""The build helper rebuilds a library that is older than its sources (CPU only)."""
import os
import shutil

import pytest


def test_stale_library_is_rebuilt(tmp_path, monkeypatch):
    from exactinfer_amd import build as B
    # work on a copy of the package tree so the real library is never touched
    pkg = tmp_path / "exactinfer_amd"
    shutil.copytree(B.PKG, pkg, ignore=shutil.ignore_patterns("__pycache__", "*.so"))
    shutil.copytree(B.ROOT / "include", tmp_path / "include")
    monkeypatch.setattr(B, "PKG", pkg)
    monkeypatch.setattr(B, "ROOT", tmp_path)
    monkeypatch.setattr(B, "CSRC", pkg / "csrc")
    monkeypatch.setattr(B, "LIB", pkg / "libei_attn.so")
    calls = []
    monkeypatch.setattr(B, "build", lambda verbose=False: calls.append(1) or B.LIB.write_bytes(b"built") or B.LIB)
    assert B.is_stale()  # absent
    B.ensure_built()
    assert len(calls) == 1 and not B.is_stale()
    B.ensure_built()
    assert len(calls) == 1  # up to date: no rebuild
    # a source edited after the build makes the library stale
    src = pkg / "csrc" / "decode.hip"
    t = B.LIB.stat().st_mtime + 10
    os.utime(src, (t, t))
    assert B.is_stale()
    B.ensure_built()
    assert len(calls) == 2
    # so does the ABI header
    os.utime(B.LIB, (t + 10, t + 10))
    hdr = tmp_path / "include" / "ei_attn.h"
    os.utime(hdr, (t + 20, t + 20))
    assert B.is_stale()


def test_real_library_is_current():
    """The library the tests load was built after every source it is built from."""
    from exactinfer_amd import build as B
    if not B.LIB.exists():
        pytest.skip("library not built")
    assert not B.is_stale(), "libei_attn.so is older than a source: run __graft_entry__.build()"
