"""Stale-build detection for libnanokv.so, on the host.

The build bakes a fingerprint of the sources, headers, flags and target
into nkv_build_id(); the loader recomputes it from the files on disk and
refuses a library built from other ones (the reference's extension build
is named after such a fingerprint, nanovllm/layers/paged_kv/loader.py:47-112,
and its tests check that the fingerprint follows the sources, flags and arch
list, tests/test_paged_kv_extension_loader.py:12-32).  The rebuild test runs
hipcc on a copy of the sources (~40 s)."""
from __future__ import annotations

import shutil
from pathlib import Path

import pytest

from nanokv import _lib
from nanokv import build as nkv_build


def _copy_sources(tmp_path: Path) -> tuple[Path, Path]:
    src = tmp_path / "csrc"
    inc = tmp_path / "include"
    shutil.copytree(nkv_build.SOURCE_DIR, src, ignore=shutil.ignore_patterns("*.o", "*.so"))
    inc.mkdir()
    shutil.copy(nkv_build.INCLUDE_DIR / "nanokv.h", inc / "nanokv.h")
    return src, inc


def test_loaded_library_reports_the_sources_it_was_built_from():
    assert _lib.build_id() == nkv_build.build_id()
    assert _lib.build_id().endswith("-default")


def test_fingerprint_follows_sources_flags_and_arch(tmp_path, monkeypatch):
    src, inc = _copy_sources(tmp_path)
    base = nkv_build.source_fingerprint(src, inc)
    assert base == nkv_build.source_fingerprint()          # a copy fingerprints the same
    (src / "nkv_store.hip").write_text((src / "nkv_store.hip").read_text() + "\n// edited\n")
    edited = nkv_build.source_fingerprint(src, inc)
    assert edited != base
    (inc / "nanokv.h").write_text((inc / "nanokv.h").read_text() + "\n")
    assert nkv_build.source_fingerprint(src, inc) not in (base, edited)
    monkeypatch.setattr(nkv_build, "HIPCC_FLAGS", nkv_build.HIPCC_FLAGS[:1] + ("-O2",)
                        + nkv_build.HIPCC_FLAGS[2:])
    assert nkv_build.source_fingerprint() != base
    monkeypatch.undo()
    monkeypatch.setattr(nkv_build, "OFFLOAD_ARCH", "gfx942")
    assert nkv_build.source_fingerprint() != base
    monkeypatch.undo()
    assert nkv_build.config_tag(None) == "default"
    assert nkv_build.config_tag({"NKV_GATHER_UNROLL": 2}) != nkv_build.config_tag({"NKV_GATHER_UNROLL": 4})


def test_verify_rules(tmp_path):
    src, inc = _copy_sources(tmp_path)
    sources = nkv_build.source_fingerprint(src, inc)
    lib = Path("libnanokv.so")
    _lib.verify_build_id(f"{sources}-default", lib, override=False, source_dir=src, include_dir=inc)
    # an override may carry other launch-shape defines, the in-tree library may not
    _lib.verify_build_id(f"{sources}-1a2b3c4d", lib, override=True, source_dir=src, include_dir=inc)
    with pytest.raises(RuntimeError, match="stale"):
        _lib.verify_build_id(f"{sources}-1a2b3c4d", lib, override=False, source_dir=src, include_dir=inc)
    for found in ("0123456789abcdef-default", "unfingerprinted"):
        for override in (False, True):
            with pytest.raises(RuntimeError, match="stale") as raised:
                _lib.verify_build_id(found, lib, override=override, source_dir=src, include_dir=inc)
            assert found in str(raised.value) and sources in str(raised.value)
    # no sources to compare against: nothing to refuse
    _lib.verify_build_id("unfingerprinted", lib, override=False, source_dir=tmp_path / "none",
                         include_dir=inc)


@pytest.mark.timeout(600)
def test_edit_without_rebuild_is_refused_and_build_clears_it(tmp_path):
    src, inc = _copy_sources(tmp_path)
    # the in-tree library against unedited sources loads
    _lib.open_library(nkv_build.LIBRARY_PATH, source_dir=src, include_dir=inc)
    hip = src / "nkv_gather.hip"
    hip.write_text(hip.read_text() + "\n// an edit that was never compiled\n")
    with pytest.raises(RuntimeError, match="stale") as raised:
        _lib.open_library(nkv_build.LIBRARY_PATH, source_dir=src, include_dir=inc)
    assert nkv_build.build_id() in str(raised.value)
    assert nkv_build.build_id(source_dir=src, include_dir=inc) in str(raised.value)
    rebuilt = nkv_build.build(output=tmp_path / "libnanokv.so", source_dir=src, include_dir=inc)
    library = _lib.open_library(rebuilt, source_dir=src, include_dir=inc)
    assert library.nkv_build_id().decode() == nkv_build.build_id(source_dir=src, include_dir=inc)
