"""The C-ABI library loads and exports every entry point include/dizo_amd.h
declares, with a ctypes signature for each (no GPU calls)."""
import os
import re

import pytest

from dizo_amd import _lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    text = open(os.path.join(ROOT, "include", "dizo_amd.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dz_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_functions()
    assert "dz_perturb" in names and "dz_project" in names
    assert len(names) >= 16


def test_library_exports_every_declared_symbol():
    lib = L.load()
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} not exported by {L.lib_path()}"


def test_ctypes_signatures_cover_header():
    assert sorted(L.SIGNATURES) == declared_functions()


def test_header_constants_match_binding():
    text = open(os.path.join(ROOT, "include", "dizo_amd.h")).read()
    consts = dict(re.findall(r"#define (DZ_[A-Z0-9_]+) \(?(-?\d+)u?\)?", text))
    for name in ("DZ_DTYPE_F32", "DZ_DTYPE_F16", "DZ_DTYPE_BF16", "DZ_PROJ_SUMSQ", "DZ_PROJ_APPLY",
                 "DZ_PROJ_REVERSE", "DZ_PROJ_REVERSE_SUMSQ", "DZ_STREAM_PARAM", "DZ_STREAM_GAMMA",
                 "DZ_STREAM_INIT"):
        assert int(consts[name]) == getattr(L, name), name


def test_version_and_errors_without_gpu():
    lib = L.load()
    assert lib.dz_version() >= 100
    with pytest.raises(L.DzError, match="unknown dtype"):
        L.call("dz_normal_table", 7, None, 32768)
    with pytest.raises(L.DzError, match="32768"):
        import ctypes
        buf = (ctypes.c_uint16 * 10)()
        L.call("dz_normal_table", 1, ctypes.cast(buf, ctypes.c_void_p), 10)
