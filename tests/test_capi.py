"""The C ABI library loads and exports every symbol include/*.h declares (CPU only:
no compute call is made)."""
import ctypes
import glob
import os
import re

import pytest

from conftest import ROOT

import forgedb


def declared_symbols():
    names = []
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        names += re.findall(r"FDB_API\s+[\w\s\*]+?\b(fdb_\w+)\s*\(", text)
    return sorted(set(names))


def test_header_declares_the_python_symbol_table():
    assert set(declared_symbols()) == set(forgedb.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    if not os.path.exists(forgedb.LIB_PATH):
        pytest.fail(f"library not built: {forgedb.LIB_PATH}")
    lib = ctypes.CDLL(forgedb.LIB_PATH)
    missing = [n for n in declared_symbols() if not hasattr(lib, n)]
    assert not missing, missing


def test_version_and_last_error_are_callable_without_a_device():
    lib = forgedb.load_library()
    assert b"gfx950" in lib.fdb_version()
    assert isinstance(lib.fdb_last_error(), bytes)


def test_null_handle_is_an_error_not_a_crash():
    lib = forgedb.load_library()
    d = forgedb._Desc()
    assert lib.fdb_ivfpq_describe(None, ctypes.byref(d)) == -1
    assert b"null" in lib.fdb_last_error()
    assert lib.fdb_ivfpq_nprobe(None) == 0
    lib.fdb_ivfpq_set_nprobe(None, 3)  # no-op
    lib.fdb_ivfpq_destroy(None)


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    monkeypatch.setattr(forgedb, "_lib_handle", None)
    with pytest.raises(RuntimeError, match="not found"):
        forgedb.load_library(str(tmp_path / "nope.so"))
