"""Built libraries carry the id of the sources they were built from
(build.py source_id, ft_build_id): a source edit without a rebuild makes
build.built() false, so tests, smoke() and bench.py rebuild instead of
loading a stale library."""

import ctypes
import os

import build as ftbuild


def test_every_library_carries_the_source_id(ft):
    sid = ftbuild.source_id()
    assert len(sid) == 16 and int(sid, 16) >= 0
    for p in (ftbuild.LIB_AMD, ftbuild.LIB_MARISA, ftbuild.PYMOD):
        assert ftbuild.built_id(p) == sid, p
    assert ftbuild.built()
    assert ft.build_id() == sid
    lib = ctypes.CDLL(ftbuild.LIB_AMD)
    lib.ft_build_id.restype = ctypes.c_char_p
    assert lib.ft_build_id() == sid.encode()


def test_a_source_edit_makes_the_build_stale(monkeypatch, tmp_path):
    files = ftbuild._source_files()
    assert any(f.endswith("tbs_kernel.hip") for f in files)
    assert any(f.endswith("flashtrie_amd.h") for f in files)
    assert any(f.endswith("build.py") for f in files)
    sid = ftbuild.source_id()
    # the same files with one byte changed in a copy of the kernel source
    kern = next(f for f in files if f.endswith("tbs_kernel.hip"))
    edited = tmp_path / "tbs_kernel.hip"
    edited.write_bytes(open(kern, "rb").read() + b"\n")
    real_relpath = os.path.relpath

    def relpath(p, start=None):
        return real_relpath(kern if p == str(edited) else p, start)

    monkeypatch.setattr(ftbuild, "_source_files",
                        lambda: [str(edited) if f == kern else f for f in files])
    monkeypatch.setattr(ftbuild.os.path, "relpath", relpath)
    assert ftbuild.source_id() != sid
    assert not ftbuild.built()


def test_missing_library_is_not_built(monkeypatch, tmp_path):
    monkeypatch.setattr(ftbuild, "LIB_MARISA", str(tmp_path / "absent.so"))
    assert ftbuild.built_id(ftbuild.LIB_MARISA) is None
    assert not ftbuild.built()
