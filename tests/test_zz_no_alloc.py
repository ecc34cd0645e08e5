"""fdb_ivfpq_batch_search_device_noalloc: no counterpart in the reference; the
variant of fdb_ivfpq_batch_search_device for callers that cannot allocate
device memory.  Through the C ABI, its results equal the existing entry
point's bit for bit (ids, distances, counts) on two calls in a row, the
second with fewer queries (the static scratch keeps the first call's
contents), and the oracle's on a sample of queries."""
import numpy as np
import pytest

import refcpu
from forgedb import IVFPQ_EXACT, IVFPQ_SCREEN, ForgeDbError, IVFPQIndex, datagen
from test_threads_gpu import _Hip

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def setup():
    base, queries = datagen.workload("ivfpq_int", n=60_000, nq=3000)
    ox = refcpu.IvfPq.build(base, nlist=128, M=16, seed=6)
    art = ox.export()
    gx = IVFPQIndex.from_artifacts(art["centroids"], art["codebooks"], art["list_offsets"], art["ids"],
                                   art["codes"])
    return base, queries, ox, art, gx


def _run(h, fn, dq, nq, k, stream):
    """fn enqueues on `stream`; the results are copied back after the
    stream has finished (a plain hipMemcpy does not wait for a non-blocking
    stream)."""
    ids, d, c = h.malloc(nq * max(k, 1) * 8), h.malloc(nq * max(k, 1) * 4), h.malloc(nq * 4)
    try:
        fn(dq, nq, k, ids, d, c, stream=stream)
        h.ok(h.L.hipStreamSynchronize(stream))
        return (h.to_host(ids, (nq, max(k, 1)), np.uint64)[:, :k], h.to_host(d, (nq, max(k, 1)), np.float32)[:, :k],
                h.to_host(c, (nq,), np.uint32))
    finally:
        for p in (ids, d, c):
            h.L.hipFree(p)


@pytest.mark.parametrize("mode", [IVFPQ_EXACT, IVFPQ_SCREEN], ids=["table", "screen"])
def test_noalloc_equals_batch_search_device(setup, mode):
    base, queries, ox, art, gx = setup
    print(f"no-allocation batch search vs batch_search_device, mode {mode}", flush=True)
    h = _Hip()
    s = h.stream()
    k = 10
    gx.set_search_mode(mode)
    try:
        for npb in (24, 128):  # 128 = nlist: every list, no coarse selection
            gx.set_nprobe(npb)
            ox.set_nprobe(npb)
            for nq in (3000, 700):  # the second call is smaller
                dq = h.to_dev(np.ascontiguousarray(queries[:nq]))
                try:
                    want = _run(h, gx.batch_search_device, dq, nq, k, s)
                    gx.sync(s)
                    got = _run(h, gx.batch_search_device_noalloc, dq, nq, k, s)
                    gx.sync(s)
                finally:
                    h.L.hipFree(dq)
                assert np.array_equal(got[2], want[2]), (npb, nq)
                assert np.array_equal(got[1], want[1]), (npb, nq)
                assert np.array_equal(got[0], want[0]), (npb, nq)
                oi, od, oc = ox.batch_search(queries[:40], k)
                assert np.array_equal(got[2][:40], oc.astype(np.uint32))
                assert np.array_equal(got[1][:40], od) and np.array_equal(got[0][:40], oi)
        # k = 0: no results
        dq = h.to_dev(np.ascontiguousarray(queries[:5]))
        try:
            got = _run(h, gx.batch_search_device_noalloc, dq, 5, 0, s)
            gx.sync(s)
        finally:
            h.L.hipFree(dq)
        assert np.all(got[2] == 0)
    finally:
        h.L.hipStreamDestroy(s)
        gx.set_search_mode(0)


def test_noalloc_rejects_what_it_does_not_serve(setup):
    """Checked on the host before any device work."""
    base, queries, ox, art, gx = setup
    print("no-allocation batch search: rejections", flush=True)
    gx.set_nprobe(16)
    # more probe entries than the scratch holds (2^21)
    with pytest.raises(ForgeDbError) as e:
        gx.batch_search_device_noalloc(0, (1 << 21) // 16 + 1, 10, 0, 0, 0)
    assert e.value.kind == "Unsupported"
    # an index with reranking
    rx = IVFPQIndex.from_artifacts(art["centroids"], art["codebooks"], art["list_offsets"], art["ids"],
                                   art["codes"])
    rx.enable_reranking(base[art["ids"].astype(np.int64)], 2)
    with pytest.raises(ForgeDbError) as e:
        rx.batch_search_device_noalloc(0, 4, 10, 0, 0, 0)
    assert e.value.kind == "Unsupported"
