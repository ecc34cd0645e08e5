"""IVF-PQ parity: the HIP path (through the C ABI) against the oracle on the
same artifacts and queries.

Bar: probed lists and PQ codes bit-exact; distances bit-exact (the kernels
reproduce the reference's summation orders, which is stricter than the
1e-4 relative tolerance allowed); ids identical, with exact distance ties
ordered by list position on both sides (the reference leaves that order to
its BinaryHeap, so this is one of the orders it can return).
"""
import os
import struct
import tempfile
import zlib

import numpy as np
import pytest

import refcpu

from forgedb import COARSE_EXACT, COARSE_SCREEN, DistanceMetric, ForgeDbError, IVFPQIndex, datagen

pytestmark = pytest.mark.gpu


def gpu_index(art, metric=DistanceMetric.Euclidean):
    return IVFPQIndex.from_artifacts(art["centroids"], art["codebooks"], art["list_offsets"],
                                     art["ids"], art["codes"], metric)


def check_batch(gx, ox, queries, k, label):
    gi, gd, gc = gx.batch_search_arrays(queries, k)
    oi, od, oc = ox.batch_search(queries, k)
    assert np.array_equal(gc, oc.astype(np.uint32)), f"{label}: counts differ"
    for q in range(len(queries)):
        c = int(oc[q])
        assert np.array_equal(gd[q, :c], od[q, :c]), f"{label} q{q}: distances {gd[q,:c]} vs {od[q,:c]}"
        # both sides order exact distance ties by list position
        assert np.array_equal(gi[q, :c], oi[q, :c]), f"{label} q{q}: ids {gi[q,:c]} vs {oi[q,:c]}"
        assert np.all(gi[q, c:] == np.iinfo(np.uint64).max)
        assert np.all(np.isinf(gd[q, c:]))


@pytest.mark.parametrize("mode", [COARSE_EXACT, COARSE_SCREEN], ids=["exact", "screen"])
def test_probe_parity_bit_exact(small_ivfpq, mode):
    print(f"probe parity: 64 queries, nlist 64, nprobe 1/16/48/64, coarse mode {mode}", flush=True)
    gx = gpu_index(small_ivfpq["art"])
    gx.set_coarse_mode(mode)
    ox = small_ivfpq["oracle"]
    for nprobe in (1, 16, 48, 64):
        lists, d = gx.probe(small_ivfpq["queries"], nprobe)
        for q, qv in enumerate(small_ivfpq["queries"]):
            ol, odist = ox.probes(qv, nprobe)
            assert np.array_equal(d[q], odist), (nprobe, q)
            assert np.array_equal(lists[q], ol), (nprobe, q)


@pytest.mark.parametrize("nlist,dim,nq", [(300, 40, 2100), (1100, 128, 33), (4096, 96, 700)])
def test_probe_parity_centroid_parts(nlist, dim, nq):
    """Batches too small to fill the GPU split the centroids into parts whose
    lists are merged; twins placed in other parts make exact ties across them."""
    print(f"probe parity with centroid parts: nlist {nlist}, dim {dim}, {nq} queries", flush=True)
    rng = np.random.default_rng(nlist + dim)
    M = 4
    cen = rng.standard_normal((nlist, dim)).astype(np.float32)
    half = nlist // 2
    cen[half:half + nlist // 4] = cen[:nlist // 4]  # twins: ties resolve to the lower list id
    cb = rng.standard_normal((M, 256, dim // M)).astype(np.float32)
    offsets = np.arange(nlist + 1, dtype=np.uint64)
    ids = np.arange(nlist, dtype=np.uint64)
    codes = rng.integers(0, 256, (nlist, M), dtype=np.uint8)
    gx = gpu_index(dict(centroids=cen, codebooks=cb, list_offsets=offsets, ids=ids, codes=codes))
    ox = refcpu.IvfPq.create(cen, cb, offsets, ids, codes)
    queries = (cen[rng.integers(0, nlist, nq)] + 0.3 * rng.standard_normal((nq, dim))).astype(np.float32)
    queries[::7] = cen[rng.integers(0, nlist // 4, len(queries[::7]))]  # exactly on a twin
    for nprobe in (1, 16, 100, min(nlist, 1024)):  # nprobe is limited to 1024
        lists, d = gx.probe(queries, nprobe)
        for q in range(nq):
            ol, od = ox.probes(queries[q], nprobe)
            assert np.array_equal(d[q], od), (nprobe, q)
            assert np.array_equal(lists[q], ol), (nprobe, q)


@pytest.mark.parametrize("nlist,dim,nq,nprobes", [(2048, 37, 100, (17, 32, 33, 64)), (1024, 128, 65, (2, 16)),
                                                  (4096, 96, 300, (64,)), (512, 12, 50, (8, 16)),
                                                  (640, 20, 97, (1, 20))])
def test_probe_parity_screened_shapes(nlist, dim, nq, nprobes):
    """Coarse selection at list counts the matrix-core screening serves
    (nprobe <= 64 and at most one probe per 32 lists): dimensions off the
    8- and 4-float grids, a last tile of fewer than 32 queries, twins, and
    rows the screening hands to the exact kernel (values past fp16's reach
    once scaled, and zero)."""
    print(f"screened probe parity: nlist {nlist}, dim {dim}, {nq} queries, nprobe {nprobes}", flush=True)
    rng = np.random.default_rng(nlist * 7 + dim)
    M = 1
    cen = (rng.standard_normal((nlist, dim)) * 3.0).astype(np.float32)
    cen[nlist // 2:nlist // 2 + 16] = cen[:16]  # twins
    cb = rng.standard_normal((M, 256, dim)).astype(np.float32)
    offsets = np.arange(nlist + 1, dtype=np.uint64)
    ids = np.arange(nlist, dtype=np.uint64)
    codes = rng.integers(0, 256, (nlist, M), dtype=np.uint8)
    gx = gpu_index(dict(centroids=cen, codebooks=cb, list_offsets=offsets, ids=ids, codes=codes))
    ox = refcpu.IvfPq.create(cen, cb, offsets, ids, codes)
    queries = (cen[rng.integers(0, nlist, nq)] + 0.5 * rng.standard_normal((nq, dim))).astype(np.float32)
    queries[3] = cen[5]                # on a twin
    queries[4] *= np.float32(1e19)     # |q|^2 past fp32
    queries[5] *= np.float32(1e-33)    # scale exponent out of range
    queries[6] = 0.0
    for nprobe in nprobes:
        lists, d = gx.probe(queries, nprobe)
        for q in range(nq):
            ol, od = ox.probes(queries[q], nprobe)
            assert np.array_equal(d[q], od), (nprobe, q)
            assert np.array_equal(lists[q], ol), (nprobe, q)


@pytest.mark.parametrize("nprobe,k", [(1, 10), (8, 10), (16, 1), (16, 64), (16, 65), (16, 100),
                                      (64, 10), (5, 256), (3, 1000)])
def test_batch_search_parity(small_ivfpq, nprobe, k):
    print(f"batch parity nprobe={nprobe} k={k}", flush=True)
    gx = gpu_index(small_ivfpq["art"])
    ox = small_ivfpq["oracle"]
    gx.set_nprobe(nprobe)
    ox.set_nprobe(nprobe)
    assert gx.nprobe() == ox.nprobe()
    check_batch(gx, ox, small_ivfpq["queries"], k, f"np{nprobe} k{k}")


def test_single_search_parity(small_ivfpq):
    print("single search parity (groups-of-4 ADC order)", flush=True)
    gx = gpu_index(small_ivfpq["art"])
    ox = small_ivfpq["oracle"]
    for nprobe in (0, 1, 16):
        gx.set_nprobe(nprobe)
        ox.set_nprobe(nprobe)
        for qv in small_ivfpq["queries"][:16]:
            g = gx.search(qv, 10)
            oi, od = ox.search(qv, 10)
            assert len(g) == len(oi)
            gi = np.array([x[0] for x in g], np.uint64)
            gd = np.array([x[1] for x in g], np.float32)
            assert np.array_equal(gd, od)
            assert np.array_equal(gi, oi)


@pytest.mark.parametrize("dim,M,nlist", [(96, 32, 32), (128, 8, 16), (16, 4, 8), (48, 12, 12),
                                         (20, 5, 6), (64, 64, 8)])
def test_shapes_parity(dim, M, nlist):
    print(f"shape parity dim={dim} M={M} nlist={nlist}", flush=True)
    base = datagen.gaussian_mixture(dim + M, 99, 4000, dim, ncomp=32, centre_std=2.0)
    ox = refcpu.IvfPq.build(base, nlist=nlist, M=M, seed=1)
    gx = gpu_index(ox.export())
    q = datagen.gaussian_mixture(dim + M + 1, 99, 24, dim, ncomp=32, centre_std=2.0)
    for nprobe, k in ((1, 5), (3, 10), (nlist, 50)):
        gx.set_nprobe(nprobe)
        ox.set_nprobe(nprobe)
        check_batch(gx, ox, q, k, f"d{dim} M{M} np{nprobe}")


def test_edges(small_ivfpq):
    print("edge cases: nprobe 0, k 0, k > candidates, empty lists", flush=True)
    art = dict(small_ivfpq["art"])
    gx = gpu_index(art)
    q = small_ivfpq["queries"][:4]
    gx.set_nprobe(0)
    assert gx.nprobe() == 0
    assert gx.search(q[0], 10) == []           # search probes no list
    ids, d, c = gx.batch_search_arrays(q, 10)  # batch_search probes one
    assert np.all(c == 10)
    gx.set_nprobe(10_000)
    assert gx.nprobe() == 64                   # clamped to nlist
    ids, d, c = gx.batch_search_arrays(q, 0)
    assert ids.shape == (4, 0) and np.all(c == 0)
    assert gx.batch_search([], 5) == []
    # an index where most lists are empty and k exceeds the candidates
    off = np.zeros(65, np.uint64)
    off[5:] = 7
    off[40:] = 12
    small = dict(centroids=art["centroids"], codebooks=art["codebooks"], list_offsets=off,
                 ids=art["ids"][:12], codes=art["codes"][:12])
    gx2 = gpu_index(small)
    ox2 = refcpu.IvfPq.create(small["centroids"], small["codebooks"], off, small["ids"], small["codes"])
    for nprobe in (1, 30, 64):
        gx2.set_nprobe(nprobe)
        ox2.set_nprobe(nprobe)
        check_batch(gx2, ox2, small_ivfpq["queries"], 20, f"sparse np{nprobe}")


def test_errors(small_ivfpq):
    print("error statuses", flush=True)
    gx = gpu_index(small_ivfpq["art"])
    q = small_ivfpq["queries"][:3].copy()
    with pytest.raises(ForgeDbError) as e:
        gx.batch_search_arrays(q[:, :100], 5)
    assert e.value.kind == "DimensionMismatch"
    q[1, 7] = np.nan
    gx.set_nprobe(4)
    with pytest.raises(ForgeDbError) as e:
        gx.batch_search_arrays(q, 5)
    assert e.value.kind == "NaN"
    # the handle stays usable
    gx.batch_search_arrays(small_ivfpq["queries"][:3], 5)
    with pytest.raises(ForgeDbError) as e:
        IVFPQIndex.from_artifacts(np.zeros((4, 10), np.float32), np.zeros((3, 256, 3), np.float32),
                                  np.zeros(5, np.uint64), np.zeros(0, np.uint64),
                                  np.zeros((0, 3), np.uint8))
    assert e.value.kind == "InvalidArgument"


def test_encode_parity(small_ivfpq):
    print("encode parity", flush=True)
    gx = gpu_index(small_ivfpq["art"])
    art = small_ivfpq["art"]
    rng = np.random.default_rng(0)
    resid = (small_ivfpq["base"][:512] - art["centroids"][rng.integers(0, 64, 512)]).astype(np.float32)
    codes = gx.encode(resid)
    for i in range(0, 512, 7):
        assert np.array_equal(codes[i], refcpu.pq_encode(art["codebooks"], resid[i]))


@pytest.mark.parametrize("n,dim,nlist,M", [(3000, 16, 8, 4), (5000, 32, 100, 8), (2000, 96, 70, 32)])
def test_build_parity(n, dim, nlist, M):
    """GPU build (k-means, assignment, PQ training, encode) equals the oracle's
    seeded restatement of IVFPQIndex::build bit for bit."""
    print(f"build parity n={n} dim={dim} nlist={nlist} M={M}", flush=True)
    x = datagen.gaussian_mixture(n + dim, 5, n, dim, ncomp=40, centre_std=2.0)
    ox = refcpu.IvfPq.build(x, nlist=nlist, M=M, seed=11)
    gx = IVFPQIndex.build(x, nlist, M, seed=11)
    o, g = ox.export(), gx.export()
    for key in ("centroids", "codebooks", "list_offsets", "ids", "codes"):
        assert np.array_equal(o[key], g[key]), key


def test_rerank_parity(small_ivfpq):
    print("rerank parity", flush=True)
    art = small_ivfpq["art"]
    base = small_ivfpq["base"]
    orig = base[art["ids"].astype(np.int64)]
    gx = gpu_index(art)
    ox = refcpu.IvfPq.create(art["centroids"], art["codebooks"], art["list_offsets"], art["ids"],
                             art["codes"])
    gx.enable_reranking(orig, 4)
    ox.enable_reranking(orig, 4)
    assert gx.describe()["reranking"] == 1
    for nprobe in (4, 16):
        gx.set_nprobe(nprobe)
        ox.set_nprobe(nprobe)
        check_batch(gx, ox, small_ivfpq["queries"], 10, f"rerank np{nprobe}")


def test_save_load_roundtrip(small_ivfpq):
    print("save/load roundtrip", flush=True)
    gx = gpu_index(small_ivfpq["art"])
    gx.set_nprobe(9)
    with tempfile.TemporaryDirectory() as d:
        p = os.path.join(d, "ix.fdb")
        gx.save(p)
        lx = IVFPQIndex.load(p)
        assert lx.nprobe() == 9
        a, b = gx.export(), lx.export()
        for key in a:
            assert np.array_equal(a[key], b[key]), key
        q = small_ivfpq["queries"]
        ga = gx.batch_search_arrays(q, 10)
        gb = lx.batch_search_arrays(q, 10)
        for x, y in zip(ga, gb):
            assert np.array_equal(x, y)
        raw = bytearray(open(p, "rb").read())
        raw[100] ^= 0xFF
        open(p, "wb").write(bytes(raw))
        with pytest.raises(ForgeDbError) as e:
            IVFPQIndex.load(p)
        assert e.value.kind == "ChecksumMismatch"


def _bincode_vector(vid, data):
    """SerializableVector {id: u64, data: Vec<f32>} (ivf_pq.rs:198-202)."""
    data = np.ascontiguousarray(data, dtype="<f4")
    return struct.pack("<QQ", vid, data.size) + data.tobytes()


def _bincode_ivfpq(art, nprobe, metric, rerank_factor, originals=None):
    """An independent writer of SerializableIVFPQ (ivf_pq.rs:318-327) in
    bincode 1.3's default encoding (`bincode::serialize`, ivf_pq.rs:1972):
    fixed-width little-endian integers, usize as u64, Vec as a u64 length then
    its elements, a unit enum variant as its u32 index, Option as a u8 tag
    (0 = None, 1 = Some) then the value, struct fields in declaration order.
    Centroid and codebook vectors carry their k-means cluster index as id
    (kmeans.rs:183)."""
    cen, cb = art["centroids"], art["codebooks"]
    off, ids, codes = art["list_offsets"], art["ids"], art["codes"]
    nlist, dim = cen.shape
    M, ncb, dsub = cb.shape
    out = [struct.pack("<Q", nlist)]
    out += [_bincode_vector(c, cen[c]) for c in range(nlist)]
    # SerializablePQ {codebooks: Vec<Vec<SerializableVector>>, n_subvectors, subvector_dim, dim}
    out.append(struct.pack("<Q", M))
    for m in range(M):
        out.append(struct.pack("<Q", ncb))
        out += [_bincode_vector(j, cb[m, j]) for j in range(ncb)]
    out.append(struct.pack("<QQQ", M, dsub, dim))
    # partitions: Vec<SerializablePartition {ids: Vec<u64>, codes: Vec<Vec<u8>>}>
    out.append(struct.pack("<Q", nlist))
    for l in range(nlist):
        s, e = int(off[l]), int(off[l + 1])
        out.append(struct.pack("<Q", e - s) + ids[s:e].astype("<u8").tobytes())
        out.append(struct.pack("<Q", e - s))
        out += [struct.pack("<Q", M) + codes[i].tobytes() for i in range(s, e)]
    out.append(struct.pack("<QI", nprobe, metric))
    if originals is None:
        out.append(b"\x00")
    else:
        out.append(b"\x01" + struct.pack("<Q", len(originals)))
        out += [_bincode_vector(i, v) for i, v in originals]
    out.append(struct.pack("<Q", rerank_factor))
    return b"".join(out)


def _fdb_file(index_type, payload):
    """[MAGIC 8B][VERSION u32][INDEX_TYPE u32][FLAGS u32][CHECKSUM u32]
    (persistence/format.rs:79), CRC-32 (IEEE) of the payload."""
    return b"FORGEDB\0" + struct.pack("<IIII", 1, index_type, 0, zlib.crc32(payload)) + payload


def test_save_bincode_bytes():
    """The IVF-PQ payload byte for byte against the independent writer above,
    with an empty list, a non-default metric and both Option states; then the
    reader loads the independently written file."""
    print("IVF-PQ bincode bytes", flush=True)
    rng = np.random.default_rng(7)
    nlist, dim, M = 3, 4, 2
    art = dict(centroids=rng.standard_normal((nlist, dim)).astype(np.float32),
               codebooks=rng.standard_normal((M, 256, dim // M)).astype(np.float32),
               list_offsets=np.array([0, 2, 2, 5], np.uint64),
               ids=np.array([10, 3, 7, 42, 1], np.uint64),
               codes=rng.integers(0, 256, (5, M), dtype=np.uint8))
    gx = gpu_index(art, DistanceMetric.Cosine)
    gx.set_nprobe(2)
    with tempfile.TemporaryDirectory() as d:
        p = os.path.join(d, "ix.fdb")
        gx.save(p)
        raw = open(p, "rb").read()
        want = _bincode_ivfpq(art, nprobe=2, metric=int(DistanceMetric.Cosine), rerank_factor=1)
        assert raw == _fdb_file(1, want)

        # original_vectors comes from a HashMap's values() (ivf_pq.rs:1905-1910), so its
        # record order is unspecified: compare the records as a set, everything else exactly
        orig = rng.standard_normal((5, dim)).astype(np.float32)
        gx.enable_reranking(orig, 3)
        gx.save(p)
        payload = open(p, "rb").read()[24:]
        head = _bincode_ivfpq(art, 2, int(DistanceMetric.Cosine), 3)[:-9]
        assert payload[:len(head)] == head
        rest = payload[len(head):]
        assert rest[0] == 1 and struct.unpack_from("<Q", rest, 1)[0] == 5
        rec = 8 + 8 + 4 * dim
        got = {rest[9 + r * rec: 9 + (r + 1) * rec] for r in range(5)}
        assert got == {_bincode_vector(int(i), v) for i, v in zip(art["ids"], orig)}
        assert len(rest) == 9 + 5 * rec + 8
        assert struct.unpack_from("<Q", rest, 9 + 5 * rec)[0] == 3

        # the reader on a file written independently
        open(p, "wb").write(_fdb_file(1, want))
        lx = IVFPQIndex.load(p)
        assert lx.nprobe() == 2
        ex = lx.export()
        for key in art:
            assert np.array_equal(ex[key], art[key]), key


@pytest.mark.parametrize("shape", ["16x8", "32x3"])
def test_fast_lut_within_tolerance(small_ivfpq, shape):
    """Fast LUTs compute |cb|^2 - 2<r, cb> + |r|^2: distances within 1e-4
    relative of the oracle (the north_star bound), ids equal except where
    distances tie within that tolerance."""
    print(f"fast LUT tolerance {shape}", flush=True)
    from conftest import tie_aware_match
    from forgedb import LUT_FAST
    if shape == "16x8":
        art, ox, q = small_ivfpq["art"], small_ivfpq["oracle"], small_ivfpq["queries"]
    else:
        base, q = datagen.workload("ivfpq_large", n=20_000, nq=48)
        ox = refcpu.IvfPq.build(base, nlist=64, M=32, seed=2)
        art = ox.export()
    gx = gpu_index(art)
    gx.set_lut_mode(LUT_FAST)
    assert gx.lut_mode() == LUT_FAST
    worst = 0.0
    for nprobe, k in ((1, 10), (8, 10), (16, 100)):
        gx.set_nprobe(nprobe)
        ox.set_nprobe(nprobe)
        gi, gd, gc = gx.batch_search_arrays(q, k)
        oi, od, oc = ox.batch_search(q, k)
        assert np.array_equal(gc, oc.astype(np.uint32))
        for t in range(len(q)):
            c = int(oc[t])
            rel = np.abs(gd[t, :c].astype(np.float64) - od[t, :c]) / np.maximum(np.abs(od[t, :c]), 1e-30)
            worst = max(worst, float(rel.max()))
            ok, msg = tie_aware_match(gi[t, :c], gd[t, :c], oi[t, :c], od[t, :c], rel=1e-4)
            assert ok, f"np{nprobe} k{k} q{t}: {msg}"
    print(f"worst relative distance error {worst:.3g}")
    assert worst < 1e-4


def test_fast_lut_unsupported_shape():
    base = datagen.gaussian_mixture(3, 4, 3000, 16, ncomp=8)
    ox = refcpu.IvfPq.build(base, nlist=8, M=4, seed=0)
    gx = gpu_index(ox.export())
    with pytest.raises(ForgeDbError) as e:
        gx.set_lut_mode(1)
    assert e.value.kind == "Unsupported"
    assert gx.lut_mode() == 0


# ---- tombstones, insert, compact, filtered search ------------------------------
def fresh_pair(small_ivfpq, rerank=False):
    art = small_ivfpq["art"]
    gx = gpu_index(art)
    ox = refcpu.IvfPq.create(art["centroids"], art["codebooks"], art["list_offsets"], art["ids"],
                             art["codes"])
    if rerank:
        orig = small_ivfpq["base"][art["ids"].astype(np.int64)]
        gx.enable_reranking(orig, 4)
        ox.enable_reranking(orig, 4)
    return gx, ox


def check_single(gx, ox, queries, k, label):
    for q, qv in enumerate(queries):
        got = gx.search(qv, k)
        oi, od = ox.search(qv, k)
        assert [i for i, _ in got] == oi.tolist(), f"{label} q{q}"
        assert np.array_equal(np.array([d for _, d in got], np.float32), od), f"{label} q{q}"


def test_tombstone_parity(small_ivfpq):
    print("delete -> search parity (batch and single)", flush=True)
    gx, ox = fresh_pair(small_ivfpq)
    q = small_ivfpq["queries"]
    gx.set_nprobe(16)
    ox.set_nprobe(16)
    # the ids nearest to the first queries, so deleting them changes results
    gi, _, _ = gx.batch_search_arrays(q[:8], 5)
    victims = sorted(set(int(x) for x in gi.ravel()))[:20] + [10 ** 12]
    for v in victims:
        assert gx.delete(v) == ox.delete(v), v
    assert gx.num_tombstones() == ox.num_tombstones() == 20
    assert len(gx) == 20_000 - 20 and gx.len_with_tombstones() == 20_000
    check_batch(gx, ox, q, 10, "tombstones")
    check_single(gx, ox, q[:16], 10, "tombstones single")
    gx.compact()
    ox.compact()
    a, b = gx.export(), ox.export()
    for key in ("list_offsets", "ids", "codes"):
        assert np.array_equal(a[key], b[key]), key
    assert gx.num_tombstones() == 0 and len(gx) == 20_000 - 20
    check_batch(gx, ox, q, 10, "compacted")


def test_insert_parity(small_ivfpq):
    print("insert_batch parity (assignment, codes, searches, un-tombstoning)", flush=True)
    gx, ox = fresh_pair(small_ivfpq)
    q = small_ivfpq["queries"]
    rng = np.random.default_rng(6)
    new = np.clip(q[:40] + rng.normal(0, 3, q[:40].shape), 0, 255).astype(np.float32)
    ids = np.arange(500_000, 500_040, dtype=np.uint64)
    assert gx.delete(3) and ox.delete(3)
    ids[7] = 3  # re-inserting a deleted id lifts that list's tombstone
    gx.insert_batch(new, ids)
    ox.insert(new, ids)
    a, b = gx.export(), ox.export()
    for key in ("list_offsets", "ids", "codes"):
        assert np.array_equal(a[key], b[key]), key
    assert gx.num_tombstones() == ox.num_tombstones()
    for nprobe in (4, 16):
        gx.set_nprobe(nprobe)
        ox.set_nprobe(nprobe)
        check_batch(gx, ox, q, 10, f"inserted np{nprobe}")


@pytest.mark.parametrize("rerank", [False, True], ids=["adc", "rerank"])
def test_search_filtered_parity(small_ivfpq, rerank):
    print(f"search_filtered parity rerank={rerank}", flush=True)
    gx, ox = fresh_pair(small_ivfpq, rerank)
    q = small_ivfpq["queries"][:24]
    rng = np.random.default_rng(9)
    for nprobe, n_allowed in ((16, 3000), (4, 200), (64, 50), (0, 3000), (8, 0)):
        gx.set_nprobe(nprobe)
        ox.set_nprobe(nprobe)
        allowed = rng.choice(20_000, n_allowed, replace=False).astype(np.uint64)
        if n_allowed:
            assert gx.delete(int(allowed[0])) == ox.delete(int(allowed[0]))
        k = 5 if rerank else 10
        gi, gd, gc = gx.search_filtered_arrays(q, k, allowed)
        for j, qv in enumerate(q):
            oi, od = ox.search_filtered(qv, k, allowed)
            label = f"filtered np{nprobe} n{n_allowed} q{j}"
            assert int(gc[j]) == len(oi), label
            assert gi[j, :len(oi)].tolist() == oi.tolist(), label
            assert np.array_equal(gd[j, :len(oi)], od), label
        assert gx.search_filtered(q[0], k, allowed) == [(int(i), float(d)) for i, d in
                                                         zip(*ox.search_filtered(q[0], k, allowed))]


@pytest.mark.parametrize("nprobe,k", [(1, 10), (16, 100), (48, 10)])
def test_batch_search_screened_coarse(small_ivfpq, nprobe, k):
    print(f"batch parity with screened coarse selection nprobe={nprobe} k={k}", flush=True)
    gx = gpu_index(small_ivfpq["art"])
    gx.set_coarse_mode(COARSE_SCREEN)
    ox = small_ivfpq["oracle"]
    gx.set_nprobe(nprobe)
    ox.set_nprobe(nprobe)
    check_batch(gx, ox, small_ivfpq["queries"], k, f"screened coarse np{nprobe} k{k}")
    check_single(gx, ox, small_ivfpq["queries"][:8], k, f"screened coarse single np{nprobe}")


def test_screened_coarse_duplicate_centroids(small_ivfpq):
    print("screened coarse selection with duplicated centroids (exact ties)", flush=True)
    art = dict(small_ivfpq["art"])
    cen = art["centroids"].copy()
    cen[32:] = cen[:32]  # every centroid has a twin: ties resolve to the lower list id
    art["centroids"] = cen
    ox = refcpu.IvfPq.create(cen, art["codebooks"], art["list_offsets"], art["ids"], art["codes"])
    for mode in (COARSE_EXACT, COARSE_SCREEN):
        gx = gpu_index(art)
        gx.set_coarse_mode(mode)
        for nprobe in (3, 16, 40):
            lists, d = gx.probe(small_ivfpq["queries"], nprobe)
            for q, qv in enumerate(small_ivfpq["queries"]):
                ol, od = ox.probes(qv, nprobe)
                assert np.array_equal(lists[q], ol) and np.array_equal(d[q], od), (mode, nprobe, q)
