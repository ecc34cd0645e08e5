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


def test_load_errors_are_reported_before_any_device_work(tmp_path):
    """Persistable::load error paths (persistence/mod.rs:77-94): the file is
    mapped, its header and CRC checked and its payload decoded on the host, so
    every malformed file fails with its status before a device is needed."""
    import struct
    import zlib

    def fdb(index_type, payload, magic=b"FORGEDB\0", version=1, crc=None):
        crc = zlib.crc32(payload) if crc is None else crc
        return magic + struct.pack("<IIII", version, index_type, 0, crc) + payload

    payload = b"\x05" * 40  # a bincode length far beyond the payload
    cases = {
        "missing": (None, "Io"),
        "dir": ("dir", "Io"),
        "empty": (b"", "InvalidFormat"),
        "short": (b"FORGEDB\0\x01", "InvalidFormat"),
        "magic": (fdb(1, payload, magic=b"FORGEDX\0"), "InvalidFormat"),
        "version": (fdb(1, payload, version=2), "InvalidFormat"),
        "crc": (fdb(1, payload, crc=zlib.crc32(payload) ^ 1), "ChecksumMismatch"),
        "payload": (fdb(1, payload), "InvalidFormat"),
        "type": (fdb(4, payload), "InvalidFormat"),
    }
    for name, (content, kind) in cases.items():
        p = tmp_path / name
        if content == "dir":
            p.mkdir()
        elif content is not None:
            p.write_bytes(content)
        with pytest.raises(forgedb.ForgeDbError) as e:
            forgedb.IVFPQIndex.load(str(p))
        assert e.value.kind == kind, (name, e.value)
    # the brute-force loader on an IVF-PQ file and on a bad checksum
    (tmp_path / "bf").write_bytes(fdb(1, payload))
    with pytest.raises(forgedb.ForgeDbError) as e:
        forgedb.BruteForceIndex.load(str(tmp_path / "bf"))
    assert e.value.kind == "InvalidFormat"
    (tmp_path / "bf").write_bytes(fdb(4, payload, crc=7))
    with pytest.raises(forgedb.ForgeDbError) as e:
        forgedb.BruteForceIndex.load(str(tmp_path / "bf"))
    assert e.value.kind == "ChecksumMismatch"
