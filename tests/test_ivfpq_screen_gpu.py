"""IVF-PQ screening (IVFPQ_SCREEN / IVFPQ_AUTO): half-precision products on
the matrix cores pick candidates, which are rescored in the reference's
order.  Its results must equal the table scan's bit for bit: compared here
with the oracle on the same artifacts, and with IVFPQ_EXACT on the same GPU
index, across shapes, k, nprobe, both ADC orders and the cases that force
the exact fallback (huge residuals, candidate overflow)."""
import numpy as np
import pytest

import refcpu

from forgedb import (IVFPQ_AUTO, IVFPQ_EXACT, IVFPQ_SCREEN, IVFPQ_SCREEN_SORTED, DistanceMetric, ForgeDbError,
                     IVFPQIndex, datagen)

pytestmark = pytest.mark.gpu

NO_ID = np.iinfo(np.uint64).max


def gpu_index(art):
    return IVFPQIndex.from_artifacts(art["centroids"], art["codebooks"], art["list_offsets"], art["ids"],
                                     art["codes"], DistanceMetric.Euclidean)


def same(a, b, label):
    (gi, gd, gc), (oi, od, oc) = a, b
    assert np.array_equal(gc, np.asarray(oc).astype(np.uint32)), f"{label}: counts differ"
    for q in range(len(gc)):
        c = int(oc[q])
        assert np.array_equal(gd[q, :c], od[q, :c]), f"{label} q{q}: distances {gd[q, :c]} vs {od[q, :c]}"
        assert np.array_equal(gi[q, :c], oi[q, :c]), f"{label} q{q}: ids differ"
        assert np.all(gi[q, c:] == NO_ID)


def screened(gx, queries, k, label, mode=IVFPQ_SCREEN):
    gx.set_search_mode(mode)
    out = gx.batch_search_arrays(queries, k)
    assert gx.last_search_path() == 2, label
    fb, cand = gx.last_screen_stats()
    print(f"  {label}: {fb} of {len(queries)} rescanned, {cand / max(len(queries), 1):.0f} candidates per query",
          flush=True)
    return out, fb


@pytest.mark.parametrize("nprobe,k", [(2, 10), (8, 10), (16, 1), (16, 64), (16, 65), (16, 100), (64, 10),
                                      (5, 256), (3, 1000)])
def test_screen_parity(small_ivfpq, nprobe, k):
    print(f"screened batch parity nprobe={nprobe} k={k} (20k x 128, nlist 64, M 16)", flush=True)
    gx = gpu_index(small_ivfpq["art"])
    ox = small_ivfpq["oracle"]
    gx.set_nprobe(nprobe)
    ox.set_nprobe(nprobe)
    q = small_ivfpq["queries"]
    got, _ = screened(gx, q, k, f"np{nprobe} k{k}")
    same(got, ox.batch_search(q, k), f"screen np{nprobe} k{k} vs oracle")
    gx.set_search_mode(IVFPQ_EXACT)
    same(got, gx.batch_search_arrays(q, k), f"screen np{nprobe} k{k} vs table scan")
    assert gx.last_search_path() == 0


@pytest.mark.parametrize("nprobe,k", [(2, 10), (16, 10), (16, 100), (64, 1000)])
def test_screen_sorted_schedule(small_ivfpq, nprobe, k):
    """The work schedule of large indexes (tiles ordered by size, taken from
    per-XCD counters by a grid of resident workgroups) on the small index:
    the same results as the table scan and the oracle."""
    print(f"screened batch, sorted tiles, nprobe={nprobe} k={k} (20k x 128, nlist 64, M 16)", flush=True)
    gx = gpu_index(small_ivfpq["art"])
    ox = small_ivfpq["oracle"]
    gx.set_nprobe(nprobe)
    ox.set_nprobe(nprobe)
    q = small_ivfpq["queries"]
    got, _ = screened(gx, q, k, f"sorted np{nprobe} k{k}", IVFPQ_SCREEN_SORTED)
    same(got, ox.batch_search(q, k), f"sorted np{nprobe} k{k} vs oracle")
    gx.set_search_mode(IVFPQ_SCREEN)
    same(got, gx.batch_search_arrays(q, k), f"sorted np{nprobe} k{k} vs static tiles")


@pytest.mark.parametrize("dim,M", [(96, 32), (128, 16), (20, 5)])
def test_screen_sorted_skewed_lists(dim, M):
    """Sorted tiles on skewed lists: most vectors in one list (several
    64-block chunks and pair tiles), many lists holding a few codes or none,
    so the size keys span their whole range and fewer tiles than workgroups
    exist for some stages."""
    print(f"sorted tiles, skewed lists dim={dim} M={M}", flush=True)
    rng = np.random.default_rng(dim + M)
    nlist = 48
    centres = rng.normal(0.0, 6.0, size=(nlist, dim)).astype(np.float32)
    # 70% of the points around centre 0, the rest spread thinly over a few
    # centres; lists 40.. get nothing beyond what k-means gives them
    n = 9000
    pick = np.where(rng.random(n) < 0.7, 0, rng.integers(1, 12, size=n))
    base = (centres[pick] + rng.normal(0.0, 1.0, size=(n, dim))).astype(np.float32)
    ox = refcpu.IvfPq.build(base, nlist=nlist, M=M, seed=2)
    gx = gpu_index(ox.export())
    q = (centres[np.where(rng.random(300) < 0.8, 0, rng.integers(0, nlist, size=300))]
         + rng.normal(0.0, 1.0, size=(300, dim))).astype(np.float32)
    for nprobe, k in ((2, 10), (8, 100), (nlist, 7)):
        gx.set_nprobe(nprobe)
        ox.set_nprobe(nprobe)
        got, _ = screened(gx, q, k, f"skewed d{dim} np{nprobe}", IVFPQ_SCREEN_SORTED)
        same(got, ox.batch_search(q, k), f"skewed sorted d{dim} M{M} np{nprobe} k{k} vs oracle")
        gx.set_search_mode(IVFPQ_EXACT)
        same(got, gx.batch_search_arrays(q, k), f"skewed sorted d{dim} M{M} np{nprobe} k{k} vs table scan")


@pytest.mark.parametrize("dim,M,nlist", [(96, 32, 32), (128, 8, 16), (16, 4, 8), (48, 12, 12), (20, 5, 6),
                                         (64, 64, 8), (40, 8, 10), (256, 32, 16), (24, 3, 8), (256, 64, 128)])
def test_screen_shapes(dim, M, nlist):
    """(256, 64, 128) probes 128 lists of 256 dims: residuals beyond the
    rescoring's LDS cache, recomputed per candidate."""
    print(f"screened shape parity dim={dim} M={M} nlist={nlist}", flush=True)
    base = datagen.gaussian_mixture(dim + M, 99, 4000, dim, ncomp=32, centre_std=2.0)
    ox = refcpu.IvfPq.build(base, nlist=nlist, M=M, seed=1)
    gx = gpu_index(ox.export())
    q = datagen.gaussian_mixture(dim + M + 1, 99, 40, dim, ncomp=32, centre_std=2.0)
    for nprobe, k in ((2, 5), (3, 10), (nlist, 50)):
        gx.set_nprobe(nprobe)
        ox.set_nprobe(nprobe)
        got, _ = screened(gx, q, k, f"d{dim} M{M} np{nprobe}")
        same(got, ox.batch_search(q, k), f"d{dim} M{M} np{nprobe} k{k}")


def test_screen_single_search(small_ivfpq):
    print("screened single search (groups-of-4 ADC order)", flush=True)
    gx = gpu_index(small_ivfpq["art"])
    gx.set_search_mode(IVFPQ_SCREEN)
    ox = small_ivfpq["oracle"]
    for nprobe in (2, 16):
        gx.set_nprobe(nprobe)
        ox.set_nprobe(nprobe)
        for qv in small_ivfpq["queries"][:16]:
            g = gx.search(qv, 10)
            assert gx.last_search_path() == 2
            oi, od = ox.search(qv, 10)
            assert [x[0] for x in g] == oi.tolist()
            assert np.array_equal(np.array([x[1] for x in g], np.float32), od)


def test_screen_edges(small_ivfpq):
    print("screening edge cases: a query on a centroid, scaled queries, a residual beyond half precision, "
          "first lists shorter than k, candidate overflow", flush=True)
    art = small_ivfpq["art"]
    gx = gpu_index(art)
    ox = small_ivfpq["oracle"]
    q = small_ivfpq["queries"][:24].copy()
    q[0] = art["centroids"][5]          # zero residual for its first probe
    q[1] = q[1] * 1.0e4                 # large but in range after scaling
    q[2] = art["centroids"][7] + 1e-3   # tiny first residual
    gx.set_nprobe(16)
    ox.set_nprobe(16)
    got, _ = screened(gx, q, 10, "scaled queries")
    same(got, ox.batch_search(q, 10), "edges vs oracle")
    # a component of 1e36: the residual's scale is out of reach, rescanned exactly
    big = q.copy()
    big[3, 0] = 1.0e36
    got, fb = screened(gx, big, 10, "1e36 component")
    assert fb >= 1
    gx.set_search_mode(IVFPQ_EXACT)
    same(got, gx.batch_search_arrays(big, 10), "1e36 vs table scan")
    # k above the first list's length: d_k is infinite, every code is a candidate
    gx.set_nprobe(2)
    ox.set_nprobe(2)
    got, _ = screened(gx, q, 700, "k 700 over two lists")
    same(got, ox.batch_search(q, 700), "k 700 vs oracle")
    # a query far from every code: all 64 lists qualify, the candidates overflow
    far = q.copy()
    far[4] = 1.0e3
    gx.set_nprobe(64)
    ox.set_nprobe(64)
    got, fb = screened(gx, far, 10, "far query over 64 lists")
    same(got, ox.batch_search(far, 10), "far query vs oracle")


def test_screen_nan_query(small_ivfpq):
    print("screening with a NaN query raises as the table scan does", flush=True)
    gx = gpu_index(small_ivfpq["art"])
    gx.set_search_mode(IVFPQ_SCREEN)
    gx.set_nprobe(16)
    q = small_ivfpq["queries"][:8].copy()
    q[3, 5] = np.nan
    with pytest.raises(ForgeDbError):
        gx.batch_search_arrays(q, 10)
    # the next batch is clean
    gx.batch_search_arrays(small_ivfpq["queries"][:8], 10)


def test_screen_after_changes(small_ivfpq):
    print("screening after insert, delete and compact (decoded lists rebuilt)", flush=True)
    art = small_ivfpq["art"]
    gx = gpu_index(art)
    gx.set_nprobe(16)
    q = small_ivfpq["queries"]
    rng = np.random.default_rng(5)
    extra = small_ivfpq["base"][:500] + rng.standard_normal((500, 128)).astype(np.float32)
    gx.insert_batch(extra, np.arange(10**6, 10**6 + 500, dtype=np.uint64))
    got, _ = screened(gx, q, 20, "after insert")
    gx.set_search_mode(IVFPQ_EXACT)
    same(got, gx.batch_search_arrays(q, 20), "after insert")
    for i in range(0, 400, 3):
        gx.delete(int(art["ids"][i]))
    gx.set_search_mode(IVFPQ_SCREEN)
    gx.batch_search_arrays(q, 20)
    assert gx.last_search_path() == 0  # tombstones: the table scan skips them
    gx.compact()
    got, _ = screened(gx, q, 20, "after compact")
    gx.set_search_mode(IVFPQ_EXACT)
    same(got, gx.batch_search_arrays(q, 20), "after compact")


def test_screen_auto_mode(small_ivfpq):
    print("automatic mode: small batches take the table scan", flush=True)
    gx = gpu_index(small_ivfpq["art"])
    gx.set_nprobe(16)
    gx.set_search_mode(IVFPQ_AUTO)
    gx.batch_search_arrays(small_ivfpq["queries"], 10)
    assert gx.last_search_path() == 0  # 64 queries x ~5k codes is below the threshold


def test_screen_several_slices(small_ivfpq):
    """k = 100 holds 16,384 queries per slice: 20,000 queries take two
    slices, whose statistics add up and whose results equal the table
    scan's."""
    print("screening in two slices (20,000 queries, k 100)", flush=True)
    gx = gpu_index(small_ivfpq["art"])
    gx.set_nprobe(8)
    rng = np.random.default_rng(11)
    base = small_ivfpq["base"]
    q = (base[rng.integers(0, len(base), 20_000)] + rng.normal(0, 4, (20_000, base.shape[1]))).astype(np.float32)
    got, fb = screened(gx, q, 100, "two slices")
    _, cand = gx.last_screen_stats()
    assert cand >= 100 * (len(q) - fb)  # every query settled by screening rescored at least k candidates
    gx.set_search_mode(IVFPQ_EXACT)
    same(got, gx.batch_search_arrays(q, 100), "two slices vs table scan")
    # a second batch of one slice reports its own counts
    gx.set_search_mode(IVFPQ_SCREEN)
    gx.batch_search_arrays(q[:500], 100)
    fb2, cand2 = gx.last_screen_stats()
    assert fb2 <= 500 and 0 < cand2 < cand
