"""Parity at the benchmark sizes.

Every workload bench.py measures, at its full size:
- the GPU index against the oracle on a subset of the queries: bit-exact
  distances, identical ids (ties by list position or row);
- for the screened paths (brute force, IVF and IVF-PQ), the screened result
  against the GPU's exact scan on many more queries: bit-exact, since
  screening only chooses which rows are rescored exactly.

The two IVF-PQ workloads (1M x 128 and 10M x 96) take the index the GPU
built; the oracle searches the exported artifacts.  One test per workload;
each prints its configuration first.
"""
import numpy as np
import pytest

import refcpu

from forgedb import (BF_EXACT, BF_SCREEN, IVF_AUTO, IVF_EXACT, IVFPQ_AUTO, IVFPQ_EXACT, IVFPQ_SCREEN, BruteForceIndex,
                     DistanceMetric, IVFIndex, IVFPQIndex, datagen)

pytestmark = pytest.mark.gpu

NO_ID = np.iinfo(np.uint64).max


def same(a, b, label):
    (gi, gd, gc), (oi, od, oc) = a, b
    assert np.array_equal(gc, oc.astype(np.uint32)), f"{label}: counts differ"
    for q in range(len(gc)):
        c = int(oc[q])
        assert np.array_equal(gd[q, :c], od[q, :c]), f"{label} q{q}: distances differ"
        assert np.array_equal(gi[q, :c], oi[q, :c]), f"{label} q{q}: ids differ"
        assert np.all(gi[q, c:] == NO_ID)


def ivfpq_check(name, nlist, M, nprobe, k, n_oracle):
    base, queries = datagen.workload(name)
    gx = IVFPQIndex.build(base, nlist, M, seed=1)
    gx.set_nprobe(nprobe)
    art = gx.export()
    ox = refcpu.IvfPq.create(art["centroids"], art["codebooks"], art["list_offsets"], art["ids"], art["codes"])
    ox.set_nprobe(nprobe)
    q = queries[:n_oracle]
    # the oracle's subset through both the screened and the table-scan paths
    for mode in (IVFPQ_SCREEN, IVFPQ_EXACT):
        gx.set_search_mode(mode)
        same(gx.batch_search_arrays(q, k), ox.batch_search(q, k, parallel=True, nthreads=16), f"{name} mode {mode}")
    # the whole batch screened (the automatic choice at this size) against the table scan
    gx.set_search_mode(IVFPQ_AUTO)
    screened = gx.batch_search_arrays(queries, k)
    assert gx.last_search_path() == 2
    fb, cand = gx.last_screen_stats()
    print(f"  screened: {fb} of {len(queries)} rescanned, {cand / len(queries):.0f} candidates per query", flush=True)
    gx.set_search_mode(IVFPQ_EXACT)
    gi, gd, gc = gx.batch_search_arrays(queries, k)
    assert np.all(gc == k) and np.all(np.diff(gd, axis=1) >= 0)
    same(screened, (gi, gd, gc), f"{name} screened vs table scan")


def test_ivfpq_1m_x128():
    print("IVF-PQ 1M x 128 integer mixture, nlist 1024, M 16x8, nprobe 16, k 10: GPU build, 2000 queries "
          "against the oracle (screened and table scan), 10000 screened against the table scan", flush=True)
    ivfpq_check("ivfpq_int", 1024, 16, 16, 10, 2000)


def test_ivfpq_10m_x96():
    print("IVF-PQ 10M x 96 mixture, nlist 4096, M 32x3, nprobe 64, k 100: GPU build, 100 queries against "
          "the oracle (screened and table scan), 10000 screened against the table scan", flush=True)
    ivfpq_check("ivfpq_large", 4096, 32, 64, 100, 100)


@pytest.mark.parametrize("metric", [DistanceMetric.DotProduct, DistanceMetric.Cosine], ids=["dot", "cosine"])
def test_bf_1m_x128(metric):
    print(f"brute force 1M x 128 normalised, k 100, {metric.name}: fp16 screening against the "
          "exact scan on 2000 queries, 30 against the oracle", flush=True)
    base, queries = datagen.workload("bf_norm", nq=2000)
    g = BruteForceIndex.from_arrays(base, None, metric)
    g.set_search_mode(BF_SCREEN)
    screened = g.batch_search_arrays(queries, 100)
    # Euclidean: list screening on the matrix cores; Manhattan: per-query fp16 screening
    assert g.last_search_path() == (3 if metric == DistanceMetric.Euclidean else 2)
    print(f"  exact rescans: {g.last_fallbacks()} of 2000", flush=True)
    g.set_search_mode(BF_EXACT)
    same(screened, g.batch_search_arrays(queries, 100), f"bf {metric.name} screened vs exact")
    ids = np.arange(len(base), dtype=np.uint64)
    q = queries[:30]
    same(tuple(x[:30] for x in screened), refcpu.bf_batch_search(base, ids, int(metric), q, 100, 16),
         f"bf {metric.name} vs oracle")


@pytest.mark.parametrize("metric", [DistanceMetric.Euclidean, DistanceMetric.Manhattan], ids=["l2", "l1"])
def test_ivf_1m_x96(metric):
    print(f"IVF 1M x 96 mixture, nlist 4096, nprobe 32, k 100, {metric.name}: fp16 screening "
          "against the exact scan on 10000 queries, 300 against the oracle", flush=True)
    base, queries = datagen.workload("ivf_flat")
    g = IVFIndex.build(base, 4096, metric, seed=1)
    g.set_nprobe(32)
    screened = g.batch_search_arrays(queries, 100)
    # Euclidean: list screening on the matrix cores; Manhattan: per-query fp16 screening
    assert g.last_search_path() == (3 if metric == DistanceMetric.Euclidean else 2)
    print(f"  exact rescans: {g.last_fallbacks()} of 10000", flush=True)
    g.set_search_mode(IVF_EXACT)
    same(screened, g.batch_search_arrays(queries, 100), f"ivf {metric.name} screened vs exact")
    g.set_search_mode(IVF_AUTO)
    art = g.export()
    q = queries[:300]
    ref = refcpu.ivf_batch_search(art["centroids"], art["list_offsets"], art["ids"], art["rows"], int(metric), 32,
                                  q, 100, 16)
    same(tuple(x[:300] for x in screened), ref, f"ivf {metric.name} vs oracle")
