"""The library's host-side .fdb codec (forge-db_amd/csrc/fdb_format.cpp) on the
CPU: partial original_vectors, stored fields kept as stored, and malformed
sizes rejected before any allocation.  A small driver is compiled with g++
against the codec's source."""
import os
import struct
import subprocess
import zlib

import numpy as np
import pytest

from conftest import ROOT
from test_ivfpq_gpu import _bincode_ivfpq, _bincode_vector, _fdb_file

CSRC = os.path.join(ROOT, "forge-db_amd", "csrc")


@pytest.fixture(scope="module")
def probe(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("probe") / "fdb_format_probe")
    subprocess.run(["g++", "-O1", "-std=c++17", "-I", CSRC, "-I", os.path.join(ROOT, "include"),
                    os.path.join(ROOT, "tests", "fdb_format_probe.cpp"), os.path.join(CSRC, "fdb_format.cpp"),
                    "-o", exe], check=True)

    def run(*paths):
        out = subprocess.run([exe, *map(str, paths)], check=True, capture_output=True, text=True).stdout
        return dict(line.split(" ", 1) for line in out.strip().splitlines())
    return run


def _art(rng, nlist=3, dim=4, M=2, n=6):
    off = np.array([0, 2, 2, n], np.uint64)
    return dict(centroids=rng.standard_normal((nlist, dim)).astype(np.float32),
                codebooks=rng.standard_normal((M, 256, dim // M)).astype(np.float32),
                list_offsets=off, ids=np.array([10, 3, 7, 42, 1, 3], np.uint64)[:n],
                codes=rng.integers(0, 256, (n, M), dtype=np.uint8))


def test_partial_originals_load_and_save_back(probe, tmp_path):
    # ids 10, 7 and 42 have records; 3 (held twice) and 1 have none, as after
    # the reference's delete (ivf_pq.rs:1786-1799) and save; one extra record
    # of an id no list holds; two records of 7 (the later one wins)
    rng = np.random.default_rng(1)
    art = _art(rng)
    v = rng.standard_normal((6, 4)).astype(np.float32)
    recs = [(10, v[0]), (7, v[1]), (99, v[2]), (42, v[3]), (7, v[4])]
    src = tmp_path / "in.fdb"
    src.write_bytes(_fdb_file(1, _bincode_ivfpq(art, 99, 2, 0, originals=recs)))
    out = probe(src, tmp_path / "out.fdb")
    assert out["status"] == "0"
    fields = out["nlist"].split()
    kv = dict(zip(["nlist"] + fields[1::2], [fields[0]] + fields[2::2]))
    assert kv == {"nlist": "3", "dim": "4", "M": "2", "n": "6", "nprobe": "99", "metric": "2",
                  "rerank_factor": "0", "originals": "1"}
    # list order ids 10 3 | - | 7 42 1 3
    assert out["orig_ok"] == "101100"
    # written back: the same fields, one record per id with a vector (7 with
    # the later vector; 99 is not kept), in any order
    raw = (tmp_path / "out.fdb").read_bytes()
    assert raw[:8] == b"FORGEDB\0" and struct.unpack_from("<I", raw, 20)[0] == zlib.crc32(raw[24:])
    payload = raw[24:]
    head = _bincode_ivfpq(art, 99, 2, 0)[:-9]
    assert payload[:len(head)] == head
    rest = payload[len(head):]
    rec = 16 + 16
    assert rest[0] == 1 and struct.unpack_from("<Q", rest, 1)[0] == 3
    got = {rest[9 + r * rec:9 + (r + 1) * rec] for r in range(3)}
    assert got == {_bincode_vector(10, v[0]), _bincode_vector(7, v[4]), _bincode_vector(42, v[3])}
    assert struct.unpack_from("<Q", rest, 9 + 3 * rec)[0] == 0 and len(rest) == 9 + 3 * rec + 8


def test_no_originals_roundtrip_is_byte_exact(probe, tmp_path):
    rng = np.random.default_rng(2)
    art = _art(rng)
    src = tmp_path / "in.fdb"
    data = _fdb_file(1, _bincode_ivfpq(art, 7, 0, 3))
    src.write_bytes(data)
    out = probe(src, tmp_path / "out.fdb")
    assert out["status"] == "0" and out["orig_ok"] == ""
    assert (tmp_path / "out.fdb").read_bytes() == data


@pytest.mark.parametrize("case", ["centroids", "codebooks", "originals"])
def test_sizes_are_checked_before_allocating(probe, tmp_path, case):
    """A small file whose lengths claim far more data than it holds fails as
    InvalidFormat (-7), without reserving memory for the claimed sizes."""
    if case == "centroids":
        # nlist 65,536 centroids of dimension 262,144 in a 1 MB payload
        payload = struct.pack("<QQQ", 65536, 0, 262144) + b"\0" * (1 << 20)
    elif case == "codebooks":
        # one centroid of dimension 200,000, then M = 1 codebook of 256
        # codewords of that dimension (205 MB) that the file does not hold
        dim = 200_000
        payload = (struct.pack("<QQQ", 1, 0, dim) + b"\0" * (4 * dim) + struct.pack("<Q", 1)
                   + struct.pack("<Q", 256) + b"\0" * 64)
    else:
        rng = np.random.default_rng(4)
        art = _art(rng)
        full = _bincode_ivfpq(art, 1, 0, 1, originals=[(10, np.zeros(4, np.float32))])
        at = len(full) - 8 - (16 + 16) - 8  # the record count
        payload = full[:at] + struct.pack("<Q", 1 << 36) + full[at + 8:]
    p = tmp_path / "bad.fdb"
    p.write_bytes(_fdb_file(1, payload))
    out = probe(p)
    assert out["status"].split()[0] == "-7", out
