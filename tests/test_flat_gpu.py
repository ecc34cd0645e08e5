"""Brute force and IVF (full vectors): the HIP path through the C ABI against
the oracle on the same rows and queries.

Bar: distances bit-exact for all five metrics (each kernel reproduces the
metric's AVX2 operation order); ids identical, exact distance ties ordered by
row (brute force: the earlier row, as scan_range's strict-< replacement
keeps it) or by list-order position (IVF).
"""
import os
import struct
import tempfile
import zlib

import numpy as np
import pytest

import refcpu

from forgedb import (BF_EXACT, BF_SCREEN, BF_SCREEN_F32, COARSE_SCREEN, IVF_AUTO, IVF_EXACT, IVF_SCREEN_LISTS,
                     BruteForceIndex, DistanceMetric, ForgeDbError, IVFIndex, datagen)

pytestmark = pytest.mark.gpu

METRICS = list(DistanceMetric)
NO_ID = np.iinfo(np.uint64).max


def check_rows(gi, gd, gc, oi, od, oc, label):
    assert np.array_equal(gc, oc.astype(np.uint32)), f"{label}: counts {gc} vs {oc}"
    for q in range(len(gc)):
        c = int(oc[q])
        assert np.array_equal(gd[q, :c], od[q, :c]), f"{label} q{q}: {gd[q, :c]} vs {od[q, :c]}"
        assert np.array_equal(gi[q, :c], oi[q, :c]), f"{label} q{q}: ids {gi[q, :c]} vs {oi[q, :c]}"
        assert np.all(gi[q, c:] == NO_ID) and np.all(np.isinf(gd[q, c:]))


MODES = [BF_EXACT, BF_SCREEN, BF_SCREEN_F32]
MODE_IDS = ["exact", "screen", "screen_f32"]


def bf_pair(rows, ids, metric, queries, k, mode=BF_EXACT, index=None):
    g = index or BruteForceIndex.from_arrays(rows, ids, metric)
    g.set_search_mode(mode)
    out = g.batch_search_arrays(queries, k)
    ref = refcpu.bf_batch_search(rows, ids, int(metric), queries, k)
    return out, ref


@pytest.fixture(scope="module")
def bf_small():
    base, queries = datagen.workload("bf_small")  # 10k x 128 U[0,1), 100 queries
    return base, queries, np.arange(len(base), dtype=np.uint64)


@pytest.mark.parametrize("mode", MODES, ids=MODE_IDS)
@pytest.mark.parametrize("metric", METRICS, ids=[m.name for m in METRICS])
def test_bf_small_parity(bf_small, metric, mode):
    print(f"bf 10k x 128, 100 queries, k 10, {metric.name}, mode {mode}", flush=True)
    base, queries, ids = bf_small
    (gi, gd, gc), (oi, od, oc) = bf_pair(base, ids, metric, queries, 10, mode)
    check_rows(gi, gd, gc, oi, od, oc, metric.name)


@pytest.mark.parametrize("mode", MODES, ids=MODE_IDS)
@pytest.mark.parametrize("metric", [DistanceMetric.Cosine, DistanceMetric.DotProduct,
                                    DistanceMetric.Euclidean])
def test_bf_normalised_parity(metric, mode):
    print(f"bf normalised 60k x 128, 200 queries, k 100, {metric.name}, mode {mode}", flush=True)
    base, queries = datagen.workload("bf_norm", n=60_000, nq=200)
    ids = np.arange(len(base), dtype=np.uint64) * 3 + 7
    g = BruteForceIndex.from_arrays(base, ids, metric)
    (gi, gd, gc), (oi, od, oc) = bf_pair(base, ids, metric, queries, 100, mode, index=g)
    check_rows(gi, gd, gc, oi, od, oc, metric.name)
    if mode != BF_EXACT:
        fb = g.last_fallbacks()
        print(f"  screening fallbacks: {fb} of 200", flush=True)
        assert fb < 20  # the screen decides nearly every query by itself
        assert g.last_search_path() == (2 if mode == BF_SCREEN else 1)


def test_bf_screen_fallback_on_near_ties():
    print("bf screening: near-tied rows force the exact rescan", flush=True)
    dim = 64
    q = np.zeros(dim, np.float32)
    q[0] = 1.0
    ids = np.arange(4000, dtype=np.uint64)
    for metric in (DistanceMetric.Cosine, DistanceMetric.DotProduct, DistanceMetric.EuclideanSquared):
        # 300 rows within 1e-4 of scale * q: their distances to q differ by
        # far less than the screening error bound
        rng = np.random.default_rng(12)
        rows = rng.standard_normal((4000, dim)).astype(np.float32)
        scale = 10.0 if metric == DistanceMetric.DotProduct else 1.0
        near = np.tile(q * scale, (300, 1))
        near[np.arange(300), rng.integers(1, dim, 300)] = rng.uniform(-1e-4, 1e-4, 300)
        rows[rng.choice(4000, 300, replace=False)] = near
        queries = np.stack([q, rows[5]])
        g = BruteForceIndex.from_arrays(rows, ids, metric)
        for mode in (BF_SCREEN, BF_SCREEN_F32):
            (gi, gd, gc), (oi, od, oc) = bf_pair(rows, ids, metric, queries, 20, mode, index=g)
            check_rows(gi, gd, gc, oi, od, oc, f"near ties {metric.name} mode {mode}")
            assert g.last_fallbacks() >= 1, (metric.name, mode)


@pytest.mark.parametrize("dim,n,nq,k", [(1, 300, 5, 4), (7, 1000, 17, 64), (8, 513, 3, 65),
                                        (13, 2000, 33, 1), (100, 777, 20, 1000),
                                        (130, 3000, 16, 256), (96, 50, 4, 100),
                                        (2048, 600, 3, 5)])
def test_bf_shapes(dim, n, nq, k):
    print(f"bf shape dim={dim} n={n} nq={nq} k={k}", flush=True)
    rng = np.random.default_rng(dim * 1000 + n)
    rows = rng.standard_normal((n, dim)).astype(np.float32)
    queries = rng.standard_normal((nq, dim)).astype(np.float32)
    ids = rng.permutation(n).astype(np.uint64)
    for metric in METRICS:
        g = BruteForceIndex.from_arrays(rows, ids, metric)
        for mode in MODES:
            (gi, gd, gc), (oi, od, oc) = bf_pair(rows, ids, metric, queries, k, mode, index=g)
            check_rows(gi, gd, gc, oi, od, oc, f"dim{dim} {metric.name} mode {mode}")


@pytest.mark.parametrize("n,dim,nq,k", [(100, 32, 40, 10), (1025, 64, 70, 48), (40_000, 32, 300, 100),
                                        (3000, 96, 16500, 1), (2047, 200, 33, 112)])
def test_bf_fp16_screen_sizes(n, dim, nq, k):
    """Row counts for one, two and three threshold stages, a query batch
    over two passes, the largest k, a dimension padded to whole k-steps."""
    print(f"bf fp16 screening n={n} dim={dim} nq={nq} k={k}", flush=True)
    rng = np.random.default_rng(n + dim)
    rows = rng.standard_normal((n, dim)).astype(np.float32)
    queries = rng.standard_normal((nq, dim)).astype(np.float32)
    ids = rng.permutation(n).astype(np.uint64)
    for metric in (DistanceMetric.Cosine, DistanceMetric.DotProduct, DistanceMetric.Euclidean,
                   DistanceMetric.EuclideanSquared):
        g = BruteForceIndex.from_arrays(rows, ids, metric)
        (gi, gd, gc), (oi, od, oc) = bf_pair(rows, ids, metric, queries, k, BF_SCREEN, index=g)
        check_rows(gi, gd, gc, oi, od, oc, f"fp16 n{n} {metric.name}")
        assert g.last_search_path() == 2, metric.name
        assert g.last_fallbacks() <= max(2, nq // 20), metric.name


def test_bf_fp16_screen_edges():
    """Rows or queries that fp16 cannot carry: the search still matches the
    oracle, through the fp32 screen (rows) or the exact rescan (queries)."""
    print("bf fp16 screening edge cases", flush=True)
    rng = np.random.default_rng(5)
    n, dim = 3000, 64
    base = rng.standard_normal((n, dim)).astype(np.float32)
    ids = np.arange(n, dtype=np.uint64)
    queries = rng.standard_normal((40, dim)).astype(np.float32)

    def run(rows, qs, metric, k=10):
        g = BruteForceIndex.from_arrays(rows, ids, metric)
        (gi, gd, gc), (oi, od, oc) = bf_pair(rows, ids, metric, qs, k, BF_SCREEN, index=g)
        check_rows(gi, gd, gc, oi, od, oc, f"edge {metric.name}")
        return g

    # a zero row: cosine distance 0 to every query (the reference's zero
    # denominator), so fp16 screening is off for the index
    rows = base.copy()
    rows[17] = 0.0
    assert run(rows, queries, DistanceMetric.Cosine).last_search_path() == 1
    # a zero query under cosine: rescanned exactly, the others screened
    qs = queries.copy()
    qs[3] = 0.0
    g = run(base, qs, DistanceMetric.Cosine)
    assert g.last_search_path() == 2 and g.last_fallbacks() >= 1
    # components beyond the fp16 range are scaled into it (rows as a whole,
    # each query on its own)
    rows = base.copy()
    rows[100, 5] = 1e6
    assert run(rows, queries, DistanceMetric.DotProduct).last_search_path() == 2
    qs = queries.copy()
    qs[7, 0] = 3e5
    assert run(base, qs, DistanceMetric.DotProduct).last_search_path() == 2
    # a row scale the power-of-two scaling does not cover: fp32 screening
    rows = base.copy()
    rows[100, 5] = 1e35
    assert run(rows, queries, DistanceMetric.DotProduct).last_search_path() == 1
    # small and large scales are carried by the power-of-two scaling
    for scale in (1e-6, 1e3):
        for metric in (DistanceMetric.EuclideanSquared, DistanceMetric.DotProduct, DistanceMetric.Cosine):
            g = run(base * np.float32(scale), queries * np.float32(scale), metric)
            assert g.last_search_path() == 2, (scale, metric.name)
            assert g.last_fallbacks() <= 2, (scale, metric.name)
    # near the float underflow the bound's floor sends queries to the exact
    # scan, and cosine rows with denormal norms keep the index off fp16
    for metric in (DistanceMetric.EuclideanSquared, DistanceMetric.DotProduct, DistanceMetric.Cosine):
        run(base * np.float32(1e-20), queries * np.float32(1e-20), metric)


def test_bf_ties_keep_the_earlier_row():
    print("bf exact ties", flush=True)
    rng = np.random.default_rng(4)
    uniq = rng.integers(0, 3, (40, 16)).astype(np.float32)
    rows = uniq[rng.integers(0, 40, 5000)]  # many duplicate rows
    queries = uniq[:10]
    ids = np.arange(5000, dtype=np.uint64)
    for metric in METRICS:
        g = BruteForceIndex.from_arrays(rows, ids, metric)
        for mode in MODES:
            (gi, gd, gc), (oi, od, oc) = bf_pair(rows, ids, metric, queries, 50, mode, index=g)
            check_rows(gi, gd, gc, oi, od, oc, f"ties {metric.name} mode {mode}")


def test_bf_single_search_and_kat():
    print("bf single search + brute_force.rs KAT", flush=True)
    # brute_force.rs:434-455: rows [i;4], i = 0..9, remove id 5, query [5;4]
    g = BruteForceIndex(DistanceMetric.Euclidean)
    for i in range(10):
        g.add(i, [float(i)] * 4)
    assert len(g) == 10 and g.dimension() == 4
    assert g.remove(5) and not g.remove(5)
    res = g.search([5.0] * 4, 10)
    assert len(res) == 9 and 5 not in [i for i, _ in res]
    assert res[0][1] == pytest.approx(2.0)
    rows, ids = g.export()
    assert ids.tolist() == [0, 1, 2, 3, 4, 9, 6, 7, 8]  # swap_remove moved the last row
    oid, od = refcpu.bf_search(rows, ids, 0, np.full(4, 5.0, np.float32), 10)
    assert [i for i, _ in res] == oid.tolist() and [d for _, d in res] == od.tolist()
    # add after a search re-uploads
    g.add(100, [5.0] * 4)
    assert g.search([5.0] * 4, 1) == [(100, 0.0)]


def test_bf_edges_and_errors():
    print("bf edges", flush=True)
    g = BruteForceIndex(DistanceMetric.Cosine)
    assert g.search([1.0, 2.0], 3) == [] and g.dimension() == 0
    rows = np.array([[0, 0, 0], [1, 0, 0], [0, 2, 0]], np.float32)
    g.add_batch(rows)
    # zero vector: cosine distance 0 (simd.rs:511-516)
    assert g.search([0.0, 0.0, 0.0], 3) == [(0, 0.0), (1, 0.0), (2, 0.0)]
    assert g.search([1.0, 0.0, 0.0], 0) == []
    ids, d, c = g.batch_search_arrays(np.zeros((0, 3), np.float32), 5)
    assert ids.shape == (0, 5)
    with pytest.raises(ForgeDbError) as e:
        g.search([1.0, 2.0], 3)
    assert e.value.kind == "DimensionMismatch"
    with pytest.raises(ForgeDbError) as e:
        g.add_batch(np.ones((2, 4), np.float32))
    assert e.value.kind == "DimensionMismatch"
    with pytest.raises(ForgeDbError):
        BruteForceIndex(7)
    res = g.search([1.0, 1.0, 0.0], 10)
    assert len(res) == 3


def test_bf_save_load_bytes():
    print("bf save/load", flush=True)
    rng = np.random.default_rng(2)
    rows = rng.standard_normal((257, 9)).astype(np.float32)
    ids = rng.permutation(257).astype(np.uint64) + 1000
    g = BruteForceIndex.from_arrays(rows, ids, DistanceMetric.Manhattan)
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "bf.fdb")
        g.save(path)
        raw = open(path, "rb").read()
        # brute_force.rs:278-320 payload, persistence/format.rs header
        payload = bytes([4]) + struct.pack("<QQ", 257, 9) + ids.tobytes() + rows.tobytes()
        header = b"FORGEDB\0" + struct.pack("<IIII", 1, 4, 0, zlib.crc32(payload))
        assert raw == header + payload
        h = BruteForceIndex.load(path)
        assert h.metric == DistanceMetric.Manhattan and len(h) == 257
        q = rng.standard_normal((5, 9)).astype(np.float32)
        a, b = g.batch_search_arrays(q, 7), h.batch_search_arrays(q, 7)
        assert all(np.array_equal(x, y) for x, y in zip(a, b))
        bad = bytearray(raw)
        bad[-1] ^= 1
        open(path, "wb").write(bytes(bad))
        with pytest.raises(ForgeDbError) as e:
            BruteForceIndex.load(path)
        assert e.value.kind == "ChecksumMismatch"


# ---- IVF ----------------------------------------------------------------------
@pytest.fixture(scope="module")
def ivf_small():
    """Gaussian-mixture rows (dim 96), 128 lists built by the oracle."""
    base, queries = datagen.workload("ivf_flat", n=24_000, nq=64)
    cen, off, order = refcpu.ivf_build(base, 128, seed=5)
    return dict(base=base, queries=queries, cen=cen, off=off, ids=order.astype(np.uint64),
                rows=base[order])


IVF_SCREENED = (DistanceMetric.Euclidean, DistanceMetric.EuclideanSquared, DistanceMetric.Manhattan)


def ivf_pair(s, metric, nprobe, k, queries=None, coarse=None, mode=IVF_AUTO):
    q = s["queries"] if queries is None else queries
    g = IVFIndex.from_artifacts(s["cen"], s["off"], s["ids"], s["rows"], metric)
    g.set_search_mode(mode)
    if coarse is not None:
        g.set_coarse_mode(coarse)
    g.set_nprobe(nprobe)
    out = g.batch_search_arrays(q, k)
    ref = refcpu.ivf_batch_search(s["cen"], s["off"], s["ids"], s["rows"], int(metric), g.nprobe(),
                                  q, k)
    return g, out, ref


@pytest.mark.parametrize("mode", [IVF_AUTO, IVF_EXACT], ids=["auto", "exact"])
@pytest.mark.parametrize("metric", METRICS, ids=[m.name for m in METRICS])
@pytest.mark.parametrize("nprobe,k", [(1, 10), (8, 100), (32, 100), (128, 7)])
def test_ivf_parity(ivf_small, metric, nprobe, k, mode):
    print(f"ivf 24k x 96, nlist 128, nprobe {nprobe}, k {k}, {metric.name}, mode {mode}", flush=True)
    g, (gi, gd, gc), (oi, od, oc) = ivf_pair(ivf_small, metric, nprobe, k, mode=mode)
    check_rows(gi, gd, gc, oi, od, oc, f"{metric.name} nprobe {nprobe}")
    screened = mode == IVF_AUTO and metric in IVF_SCREENED
    assert g.last_search_path() == (2 if screened else 0)
    if screened:
        fb = g.last_fallbacks()
        print(f"  fp16 screening: {fb} of 64 queries rescanned", flush=True)
        assert fb <= 6


def test_ivf_fp16_screen_edges(ivf_small):
    """Near-equal rows, a query beyond the rows' scale, an odd dimension and
    lists shorter than the candidate count: results match the oracle, and
    the queries the bound cannot settle are rescanned."""
    print("ivf fp16 screening edge cases", flush=True)
    rng = np.random.default_rng(21)
    s = dict(ivf_small)
    # 200 copies (within 1e-4) of each of 3 rows of the first list
    rows = s["rows"].copy()
    n0 = int(s["off"][1])
    for t in range(3):
        src = rows[t].copy()
        pos = rng.choice(np.arange(3, n0), min(200, n0 - 3) // 3, replace=False)
        rows[pos] = src + rng.uniform(-1e-4, 1e-4, (len(pos), rows.shape[1])).astype(np.float32)
    s["rows"] = rows
    q = np.concatenate([rows[:3] + 1e-3, s["queries"][:5]]).astype(np.float32)
    q[4, 7] = 1e6  # far beyond the rows' scale: rescanned exactly
    for metric in IVF_SCREENED:
        g, (gi, gd, gc), (oi, od, oc) = ivf_pair(s, metric, 4, 100, queries=q)
        check_rows(gi, gd, gc, oi, od, oc, f"near ties {metric.name}")
        assert g.last_search_path() == 2 and g.last_fallbacks() >= 1, metric.name
    # an odd number of dimension pairs, short lists (every scanned row a
    # candidate); a dimension the exact rescoring does not take (37) scans
    # exactly
    for dim, path in ((44, 2), (37, 0)):
        base = rng.standard_normal((3000, dim)).astype(np.float32)
        cen, off, order = refcpu.ivf_build(base, 64, seed=2)
        s2 = dict(cen=cen, off=off, ids=order.astype(np.uint64), rows=base[order],
                  queries=rng.standard_normal((50, dim)).astype(np.float32))
        for metric in IVF_SCREENED:
            for nprobe, k in ((1, 100), (6, 30), (64, 112)):
                g, (gi, gd, gc), (oi, od, oc) = ivf_pair(s2, metric, nprobe, k)
                check_rows(gi, gd, gc, oi, od, oc, f"dim {dim} {metric.name} nprobe {nprobe}")
                assert g.last_search_path() == path


@pytest.mark.parametrize("metric", [DistanceMetric.Euclidean, DistanceMetric.EuclideanSquared],
                         ids=["l2", "l2sq"])
@pytest.mark.parametrize("nprobe,k", [(2, 10), (8, 100), (32, 100), (128, 7), (16, 300)])
def test_ivf_parity_list_screen(ivf_small, metric, nprobe, k):
    """List screening on the matrix cores (IVF_SCREEN_LISTS forces it at this
    size): bit-identical to the oracle, ties by list position."""
    print(f"ivf list screening, nprobe {nprobe}, k {k}, {metric.name}", flush=True)
    g, (gi, gd, gc), (oi, od, oc) = ivf_pair(ivf_small, metric, nprobe, k, mode=IVF_SCREEN_LISTS)
    check_rows(gi, gd, gc, oi, od, oc, f"list screen {metric.name} nprobe {nprobe} k {k}")
    assert g.last_search_path() == 3
    fb = g.last_fallbacks()
    print(f"  {fb} of 64 queries rescanned", flush=True)
    assert fb <= 2


def test_ivf_list_screen_edges(ivf_small):
    """List screening with near-equal rows (square roots that tie), a query
    far beyond the rows' scale (rescanned exactly), and dimensions off the
    16-float grid (44, 37: no 16-byte row loads, 20)."""
    print("ivf list screening edge cases", flush=True)
    rng = np.random.default_rng(33)
    s = dict(ivf_small)
    rows = s["rows"].copy()
    n0 = int(s["off"][1])
    for t in range(3):
        src = rows[t].copy()
        pos = rng.choice(np.arange(3, n0), min(200, n0 - 3) // 3, replace=False)
        rows[pos] = src + rng.uniform(-1e-4, 1e-4, (len(pos), rows.shape[1])).astype(np.float32)
    rows[n0 + 1] = rows[n0]  # exact duplicates: ties resolve to the lower list position
    s["rows"] = rows
    q = np.concatenate([rows[:3] + 1e-3, rows[n0:n0 + 1], s["queries"][:5]]).astype(np.float32)
    q[5, 7] = 1e30  # beyond fp16 once scaled: rescanned exactly
    for metric in (DistanceMetric.Euclidean, DistanceMetric.EuclideanSquared):
        g, (gi, gd, gc), (oi, od, oc) = ivf_pair(s, metric, 4, 100, queries=q, mode=IVF_SCREEN_LISTS)
        check_rows(gi, gd, gc, oi, od, oc, f"list screen near ties {metric.name}")
        assert g.last_search_path() == 3 and g.last_fallbacks() >= 1, metric.name
    for dim in (44, 37, 20):
        base = rng.standard_normal((3000, dim)).astype(np.float32)
        cen, off, order = refcpu.ivf_build(base, 64, seed=2)
        s2 = dict(cen=cen, off=off, ids=order.astype(np.uint64), rows=base[order],
                  queries=rng.standard_normal((50, dim)).astype(np.float32))
        for metric in (DistanceMetric.Euclidean, DistanceMetric.EuclideanSquared):
            for nprobe, k in ((2, 100), (6, 30), (64, 112)):
                g, (gi, gd, gc), (oi, od, oc) = ivf_pair(s2, metric, nprobe, k, mode=IVF_SCREEN_LISTS)
                check_rows(gi, gd, gc, oi, od, oc, f"list screen dim {dim} {metric.name} nprobe {nprobe}")
                assert g.last_search_path() == 3


@pytest.mark.parametrize("metric", [DistanceMetric.Euclidean, DistanceMetric.Manhattan])
def test_ivf_parity_screened_coarse(ivf_small, metric):
    print(f"ivf with screened coarse selection, {metric.name}", flush=True)
    for nprobe, k in ((1, 10), (32, 100), (100, 5)):
        _, (gi, gd, gc), (oi, od, oc) = ivf_pair(ivf_small, metric, nprobe, k, coarse=COARSE_SCREEN)
        check_rows(gi, gd, gc, oi, od, oc, f"screened coarse {metric.name} nprobe {nprobe}")


def test_ivf_single_search_nprobe_rules(ivf_small):
    print("ivf single search, nprobe 0 / clamp", flush=True)
    g, (gi, gd, gc), _ = ivf_pair(ivf_small, DistanceMetric.Euclidean, 4, 20)
    for q in range(5):
        res = g.search(ivf_small["queries"][q], 20)
        assert [i for i, _ in res] == gi[q, :gc[q]].tolist()
        assert [d for _, d in res] == gd[q, :gc[q]].tolist()
    g.set_nprobe(0)  # take(0): no lists (ivf.rs:175)
    assert g.search(ivf_small["queries"][0], 5) == []
    assert np.all(g.batch_search_arrays(ivf_small["queries"][:3], 5)[2] == 0)
    g.set_nprobe(10_000)  # ivf.rs:125-127
    assert g.nprobe() == 128
    assert g.num_partitions() == 128 and len(g) == 24_000 and g.dimension() == 96
    with pytest.raises(ForgeDbError) as e:
        g.search(np.ones(95, np.float32), 3)
    assert e.value.kind == "DimensionMismatch"


def test_ivf_ragged_lists_and_ties():
    print("ivf ragged lists, empty lists, ties", flush=True)
    rng = np.random.default_rng(9)
    uniq = rng.integers(-2, 3, (30, 11)).astype(np.float32)
    rows = uniq[rng.integers(0, 30, 3001)]
    cen = rng.standard_normal((17, 11)).astype(np.float32) * 2
    cen[5] = 1000.0  # an empty list
    lens = np.bincount(rng.integers(0, 16, 3001), minlength=17)
    lens[5], lens[16] = 0, lens[5] + lens[16]
    off = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint64)
    s = dict(cen=cen, off=off, ids=np.arange(3001, dtype=np.uint64)[::-1].copy(), rows=rows,
             queries=uniq[:12])
    for metric in METRICS:
        for nprobe, k in ((3, 40), (17, 300)):
            _, (gi, gd, gc), (oi, od, oc) = ivf_pair(s, metric, nprobe, k)
            check_rows(gi, gd, gc, oi, od, oc, f"ragged {metric.name} {nprobe}")


def test_ivf_build_parity():
    print("ivf build 12k x 96, nlist 64 vs the oracle", flush=True)
    base, queries = datagen.workload("ivf_flat", n=12_000, nq=16)
    g = IVFIndex.build(base, 64, DistanceMetric.Manhattan, seed=21)
    art = g.export()
    cen, off, order = refcpu.ivf_build(base, 64, seed=21)
    assert np.array_equal(art["centroids"], cen)
    assert np.array_equal(art["list_offsets"], off)
    assert np.array_equal(art["ids"], order)
    assert np.array_equal(art["rows"], base[order])
    g.set_nprobe(6)
    gi, gd, gc = g.batch_search_arrays(queries, 10)
    oi, od, oc = refcpu.ivf_batch_search(cen, off, order, base[order], 4, 6, queries, 10)
    check_rows(gi, gd, gc, oi, od, oc, "built")
