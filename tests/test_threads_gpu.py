"""Concurrent use of one handle (include/forgedb_hip.h threading contract;
the reference's IVFPQIndex is Send + Sync, ivf_pq.rs:363, searches take
&self and set_nprobe is a relaxed atomic store, :524-527; tests/stress.rs:11-157
searches from several threads).  ctypes releases the GIL during each call."""
import ctypes as C
import threading

import numpy as np
import pytest

import refcpu
from forgedb import IVFPQ_SCREEN, IVFPQIndex, datagen

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def index_and_queries():
    base, queries = datagen.workload("ivfpq_int", n=40_000, nq=600)
    ox = refcpu.IvfPq.build(base, nlist=64, M=16, seed=4)
    art = ox.export()
    return art, queries


def _gpu(art):
    return IVFPQIndex.from_artifacts(art["centroids"], art["codebooks"], art["list_offsets"], art["ids"],
                                     art["codes"])


def test_searches_from_threads_while_nprobe_changes(index_and_queries):
    print("8 search threads + 1 set_nprobe thread on one handle", flush=True)
    art, queries = index_and_queries
    gx = _gpu(art)
    k = 10
    serial = {}
    for npb in (8, 16):
        gx.set_nprobe(npb)
        ids, d, c = gx.batch_search_arrays(queries, k)
        single = [gx.search(q, k) for q in queries[:40]]
        serial[npb] = (ids.copy(), d.copy(), c.copy(), single)
    stop = threading.Event()
    errors = []

    def flipper():
        i = 0
        while not stop.is_set():
            gx.set_nprobe(8 if i % 2 else 16)
            i += 1
            stop.wait(0.0005)

    def worker(t):
        rng = np.random.default_rng(t)
        try:
            for it in range(25):
                if errors:
                    return
                if (t + it) % 3 == 0:
                    qi = int(rng.integers(0, 40))
                    got = gx.search(queries[qi], k)
                    if all(got != serial[n][3][qi] for n in (8, 16)):
                        errors.append(f"thread {t} search q{qi}: {got}")
                else:
                    lo = int(rng.integers(0, 500))
                    hi = lo + int(rng.integers(1, 100))
                    ids, d, c = gx.batch_search_arrays(queries[lo:hi], k)
                    ok = any(np.array_equal(ids, serial[n][0][lo:hi]) and np.array_equal(d, serial[n][1][lo:hi])
                             and np.array_equal(c, serial[n][2][lo:hi]) for n in (8, 16))
                    if not ok:
                        errors.append(f"thread {t} batch [{lo}, {hi})")
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append(f"thread {t}: {e!r}")

    fl = threading.Thread(target=flipper)
    fl.start()
    ws = [threading.Thread(target=worker, args=(t,)) for t in range(8)]
    for w in ws:
        w.start()
    for w in ws:
        w.join(timeout=100)
    stop.set()
    fl.join(timeout=10)
    assert not any(w.is_alive() for w in ws), "a search thread did not finish"
    assert not errors, errors[:5]


class _Hip:
    """The HIP runtime through ctypes: device buffers and streams for the
    device-pointer entry points."""

    def __init__(self):
        self.L = C.CDLL("libamdhip64.so")
        self.L.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        self.L.hipFree.argtypes = [C.c_void_p]
        self.L.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        self.L.hipStreamCreateWithFlags.argtypes = [C.POINTER(C.c_void_p), C.c_uint]
        self.L.hipStreamSynchronize.argtypes = [C.c_void_p]
        self.L.hipStreamDestroy.argtypes = [C.c_void_p]

    def ok(self, rc):
        assert rc == 0, f"HIP error {rc}"

    def malloc(self, n):
        p = C.c_void_p()
        self.ok(self.L.hipMalloc(C.byref(p), n))
        return p.value

    def to_dev(self, a):
        a = np.ascontiguousarray(a)
        p = self.malloc(a.nbytes)
        self.ok(self.L.hipMemcpy(p, a.ctypes.data, a.nbytes, 1))
        return p

    def to_host(self, p, shape, dtype):
        out = np.empty(shape, dtype)
        self.ok(self.L.hipMemcpy(out.ctypes.data, p, out.nbytes, 2))
        return out

    def stream(self):
        s = C.c_void_p()
        self.ok(self.L.hipStreamCreateWithFlags(C.byref(s), 1))
        return s.value


@pytest.mark.parametrize("screen", [False, True], ids=["table", "screen"])
def test_two_streams_on_one_handle(index_and_queries, screen):
    """Calls on two streams, enqueued back to back without waits, use the
    handle's scratch in turn: each result equals the serial one."""
    print(f"two streams, screening={screen}", flush=True)
    art, queries = index_and_queries
    gx = _gpu(art)
    if screen:
        gx.set_search_mode(IVFPQ_SCREEN)
    gx.set_nprobe(12)
    k = 10
    batches = [np.ascontiguousarray(queries[:230]), np.ascontiguousarray(queries[230:600])]
    want = [gx.batch_search_arrays(b, k) for b in batches]
    h = _Hip()
    streams = [h.stream(), h.stream()]
    dq = [h.to_dev(b) for b in batches]
    outs = [(h.malloc(len(b) * k * 8), h.malloc(len(b) * k * 4), h.malloc(len(b) * 4)) for b in batches]
    try:
        for rep in range(12):
            for i in (0, 1) if rep % 2 == 0 else (1, 0):
                gx.batch_search_device(dq[i], len(batches[i]), k, *outs[i], stream=streams[i])
            for i in (0, 1):
                gx.sync(streams[i])
                ids = h.to_host(outs[i][0], (len(batches[i]), k), np.uint64)
                d = h.to_host(outs[i][1], (len(batches[i]), k), np.float32)
                c = h.to_host(outs[i][2], (len(batches[i]),), np.uint32)
                assert np.array_equal(c, want[i][2]), (rep, i)
                assert np.array_equal(d, want[i][1]), (rep, i)
                assert np.array_equal(ids, want[i][0]), (rep, i)
    finally:
        for p in dq + [x for o in outs for x in o]:
            h.L.hipFree(p)
        for s in streams:
            h.L.hipStreamDestroy(s)
