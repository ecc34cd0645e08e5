"""ctypes binding of the oracle (oracle/lib/librefcpu.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() as
the checker, and by bench.py's cpu_baseline leg.  The shipped library never
uses it.  Function-by-function reference citations are in refcpu.h.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "lib", "librefcpu.so")
_P = C.c_void_p
_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB):
        build()
    L = C.CDLL(LIB)
    f32, u64, i32, sz = C.c_float, C.c_uint64, C.c_int, C.c_size_t
    for name in ("fdbo_l2sq", "fdbo_l2", "fdbo_dot", "fdbo_cosine", "fdbo_l1", "fdbo_scalar_l2sq",
                 "fdbo_scalar_dot", "fdbo_scalar_cosine", "fdbo_scalar_l1"):
        getattr(L, name).argtypes = [_P, _P, sz]
        getattr(L, name).restype = f32
    L.fdbo_metric.argtypes = [i32, _P, _P, sz]
    L.fdbo_metric.restype = f32
    L.fdbo_pq_lut.argtypes = [_P, i32, i32, _P, _P]
    L.fdbo_pq_lut.restype = None
    for name in ("fdbo_adc_lanes8", "fdbo_adc_groups4", "fdbo_adc_seq"):
        getattr(L, name).argtypes = [_P, _P, i32]
        getattr(L, name).restype = f32
    L.fdbo_adc_batch4.argtypes = [_P, _P, i32, _P]
    L.fdbo_adc_batch4.restype = None
    L.fdbo_pq_encode.argtypes = [_P, i32, i32, _P, _P]
    L.fdbo_pq_encode.restype = None
    L.fdbo_splitmix64_at.argtypes = [u64, u64]
    L.fdbo_splitmix64_at.restype = u64
    L.fdbo_shuffle_indices.argtypes = [u64, _P, u64]
    L.fdbo_shuffle_indices.restype = None
    L.fdbo_kmeans_fit.argtypes = [_P, u64, i32, i32, i32, u64, _P]
    L.fdbo_kmeans_fit.restype = i32
    L.fdbo_ivfpq_create.argtypes = [_P, i32, i32, _P, i32, _P, _P, _P]
    L.fdbo_ivfpq_create.restype = _P
    L.fdbo_ivfpq_build.argtypes = [_P, u64, i32, i32, i32, u64, i32]
    L.fdbo_ivfpq_build.restype = _P
    L.fdbo_ivfpq_destroy.argtypes = [_P]
    L.fdbo_ivfpq_destroy.restype = None
    L.fdbo_ivfpq_shape.argtypes = [_P, _P, _P, _P, _P]
    L.fdbo_ivfpq_shape.restype = None
    L.fdbo_ivfpq_export.argtypes = [_P, _P, _P, _P, _P, _P]
    L.fdbo_ivfpq_export.restype = None
    L.fdbo_ivfpq_set_nprobe.argtypes = [_P, u64]
    L.fdbo_ivfpq_set_nprobe.restype = None
    L.fdbo_ivfpq_nprobe.argtypes = [_P]
    L.fdbo_ivfpq_nprobe.restype = u64
    L.fdbo_ivfpq_enable_reranking.argtypes = [_P, _P, u64]
    L.fdbo_ivfpq_enable_reranking.restype = None
    L.fdbo_ivfpq_set_originals.argtypes = [_P, _P, _P, u64, u64]
    L.fdbo_ivfpq_set_originals.restype = None
    L.fdbo_ivfpq_probes.argtypes = [_P, _P, u64, _P, _P]
    L.fdbo_ivfpq_probes.restype = i32
    L.fdbo_ivfpq_search.argtypes = [_P, _P, i32, _P, _P]
    L.fdbo_ivfpq_search.restype = i32
    L.fdbo_ivfpq_batch_search.argtypes = [_P, _P, u64, i32, _P, _P, _P]
    L.fdbo_ivfpq_batch_search.restype = None
    L.fdbo_ivfpq_batch_search_parallel.argtypes = [_P, _P, u64, i32, i32, _P, _P, _P]
    L.fdbo_ivfpq_batch_search_parallel.restype = None
    L.fdbo_bf_search.argtypes = [_P, _P, u64, i32, i32, _P, i32, _P, _P]
    L.fdbo_bf_search.restype = i32
    L.fdbo_bf_search_parallel.argtypes = [_P, _P, u64, i32, i32, _P, i32, _P, _P]
    L.fdbo_bf_search_parallel.restype = i32
    L.fdbo_bf_batch_search.argtypes = [_P, _P, u64, i32, i32, _P, u64, i32, i32, _P, _P, _P]
    L.fdbo_bf_batch_search.restype = None
    L.fdbo_ivf_probes.argtypes = [_P, i32, i32, _P, u64, _P]
    L.fdbo_ivf_probes.restype = i32
    L.fdbo_ivf_search.argtypes = [_P, i32, i32, _P, _P, _P, i32, u64, _P, i32, _P, _P]
    L.fdbo_ivf_search.restype = i32
    L.fdbo_ivf_batch_search.argtypes = [_P, i32, i32, _P, _P, _P, i32, u64, _P, u64, i32, i32,
                                        _P, _P, _P]
    L.fdbo_ivf_batch_search.restype = None
    L.fdbo_ivf_build.argtypes = [_P, u64, i32, i32, u64, i32, _P, _P, _P]
    L.fdbo_ivf_build.restype = i32
    L.fdbo_ivfpq_search_filtered.argtypes = [_P, _P, i32, _P, u64, _P, _P]
    L.fdbo_ivfpq_search_filtered.restype = i32
    L.fdbo_ivfpq_delete.argtypes = [_P, u64]
    L.fdbo_ivfpq_delete.restype = i32
    L.fdbo_ivfpq_num_tombstones.argtypes = [_P]
    L.fdbo_ivfpq_num_tombstones.restype = u64
    L.fdbo_ivfpq_insert.argtypes = [_P, _P, _P, u64]
    L.fdbo_ivfpq_insert.restype = None
    L.fdbo_ivfpq_compact.argtypes = [_P]
    L.fdbo_ivfpq_compact.restype = None
    _lib = L
    return L


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


def _f(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- distances -------------------------------------------------------------
def dist(name: str, a, b) -> float:
    a, b = _f(a), _f(b)
    return float(getattr(lib(), "fdbo_" + name)(_p(a), _p(b), a.shape[0]))


def metric(m: int, a, b) -> float:
    a, b = _f(a), _f(b)
    return float(lib().fdbo_metric(int(m), _p(a), _p(b), a.shape[0]))


def pq_lut(codebooks, r) -> np.ndarray:
    cb, r = _f(codebooks), _f(r)
    M, _, dsub = cb.shape
    out = np.empty((M, 256), np.float32)
    lib().fdbo_pq_lut(_p(cb), M, dsub, _p(r), _p(out))
    return out


def adc(order: str, lut, code) -> float:
    lut = _f(lut)
    code = np.ascontiguousarray(code, np.uint8)
    return float(getattr(lib(), "fdbo_adc_" + order)(_p(lut), _p(code), code.shape[0]))


def adc_batch4(luts, code) -> np.ndarray:
    luts = [_f(t) for t in luts]
    ptrs = (C.c_void_p * 4)(*[t.ctypes.data for t in luts])
    code = np.ascontiguousarray(code, np.uint8)
    out = np.empty(4, np.float32)
    lib().fdbo_adc_batch4(C.cast(ptrs, C.c_void_p), _p(code), code.shape[0], _p(out))
    return out


def pq_encode(codebooks, x) -> np.ndarray:
    cb, x = _f(codebooks), _f(x)
    M, _, dsub = cb.shape
    out = np.empty(M, np.uint8)
    lib().fdbo_pq_encode(_p(cb), M, dsub, _p(x), _p(out))
    return out


def kmeans_fit(data, k: int, max_iters: int, seed: int) -> np.ndarray:
    d = _f(data)
    out = np.empty((k, d.shape[1]), np.float32)
    rc = lib().fdbo_kmeans_fit(_p(d), d.shape[0], d.shape[1], k, max_iters, seed, _p(out))
    if rc:
        raise ValueError("k-means needs at least k rows")
    return out


def shuffle_indices(seed: int, n: int) -> np.ndarray:
    idx = np.arange(n, dtype=np.uint64)
    lib().fdbo_shuffle_indices(seed, _p(idx), n)
    return idx


# ---- IVF-PQ ------------------------------------------------------------------
class IvfPq:
    """The oracle's IVFPQIndex (ivf_pq.rs), same artifacts as the GPU index."""

    def __init__(self, handle):
        if not handle:
            raise ValueError("oracle rejected the index arguments")
        self.h = C.c_void_p(handle)
        L = lib()
        nl, dm, M, n = C.c_int(), C.c_int(), C.c_int(), C.c_uint64()
        L.fdbo_ivfpq_shape(self.h, C.byref(nl), C.byref(dm), C.byref(M), C.byref(n))
        self.nlist, self.dim, self.M, self.n = nl.value, dm.value, M.value, n.value

    @classmethod
    def create(cls, centroids, codebooks, list_offsets, ids, codes):
        c, cb = _f(centroids), _f(codebooks)
        off = np.ascontiguousarray(list_offsets, np.uint64)
        idv = np.ascontiguousarray(ids, np.uint64)
        cod = np.ascontiguousarray(codes, np.uint8)
        return cls(lib().fdbo_ivfpq_create(_p(c), c.shape[0], c.shape[1], _p(cb), cb.shape[0],
                                           _p(off), _p(idv), _p(cod)))

    @classmethod
    def build(cls, vectors, nlist: int, M: int, seed: int, nthreads: int = 0):
        v = _f(vectors)
        return cls(lib().fdbo_ivfpq_build(_p(v), v.shape[0], v.shape[1], nlist, M, seed, nthreads))

    def __del__(self):
        try:
            lib().fdbo_ivfpq_destroy(self.h)
        except Exception:
            pass

    def _reshape(self):
        nl, dm, M, n = C.c_int(), C.c_int(), C.c_int(), C.c_uint64()
        lib().fdbo_ivfpq_shape(self.h, C.byref(nl), C.byref(dm), C.byref(M), C.byref(n))
        self.n = n.value

    def export(self) -> dict:
        self._reshape()  # insert / compact change the entry count
        dsub = self.dim // self.M
        out = dict(centroids=np.empty((self.nlist, self.dim), np.float32),
                   codebooks=np.empty((self.M, 256, dsub), np.float32),
                   list_offsets=np.empty(self.nlist + 1, np.uint64),
                   ids=np.empty(self.n, np.uint64), codes=np.empty((self.n, self.M), np.uint8))
        lib().fdbo_ivfpq_export(self.h, _p(out["centroids"]), _p(out["codebooks"]),
                                _p(out["list_offsets"]), _p(out["ids"]), _p(out["codes"]))
        return out

    def set_nprobe(self, n: int):
        lib().fdbo_ivfpq_set_nprobe(self.h, n)

    def nprobe(self) -> int:
        return int(lib().fdbo_ivfpq_nprobe(self.h))

    def enable_reranking(self, vectors_list_order, factor: int):
        v = _f(vectors_list_order)
        lib().fdbo_ivfpq_enable_reranking(self.h, _p(v), factor)

    def set_originals(self, ids, vectors, factor: int):
        """original_vectors as a loaded file holds them: (id, vector) records."""
        idv = np.ascontiguousarray(ids, np.uint64)
        v = _f(np.asarray(vectors, np.float32).reshape(len(idv), self.dim))
        lib().fdbo_ivfpq_set_originals(self.h, _p(idv), _p(v), len(idv), factor)

    def probes(self, q, nprobe: int):
        q = _f(q)
        lists = np.empty(max(nprobe, 1), np.int32)
        d = np.empty(max(nprobe, 1), np.float32)
        cnt = lib().fdbo_ivfpq_probes(self.h, _p(q), nprobe, _p(lists), _p(d))
        return lists[:cnt], d[:cnt]

    def search(self, q, k: int):
        q = _f(q)
        ids = np.empty(max(k, 1), np.uint64)
        d = np.empty(max(k, 1), np.float32)
        cnt = lib().fdbo_ivfpq_search(self.h, _p(q), k, _p(ids), _p(d))
        return ids[:cnt], d[:cnt]

    def search_filtered(self, q, k: int, allowed_ids):
        q = _f(q)
        allow = np.ascontiguousarray(allowed_ids, np.uint64)
        ids = np.empty(max(k * 4 * 64, 1), np.uint64)
        d = np.empty(max(k * 4 * 64, 1), np.float32)
        cnt = lib().fdbo_ivfpq_search_filtered(self.h, _p(q), k, _p(allow), allow.shape[0], _p(ids),
                                               _p(d))
        return ids[:cnt], d[:cnt]

    def delete(self, vector_id: int) -> bool:
        return bool(lib().fdbo_ivfpq_delete(self.h, int(vector_id)))

    def num_tombstones(self) -> int:
        return int(lib().fdbo_ivfpq_num_tombstones(self.h))

    def insert(self, vectors, ids):
        v = _f(vectors)
        idv = np.ascontiguousarray(ids, np.uint64)
        lib().fdbo_ivfpq_insert(self.h, _p(v), _p(idv), v.shape[0])

    def compact(self):
        lib().fdbo_ivfpq_compact(self.h)

    def batch_search(self, queries, k: int, parallel: bool = False, nthreads: int = 0):
        q = _f(queries)
        nq = q.shape[0]
        ids = np.full((nq, max(k, 1)), np.iinfo(np.uint64).max, np.uint64)
        d = np.full((nq, max(k, 1)), np.inf, np.float32)
        cnt = np.zeros(nq, np.int32)
        if parallel:
            lib().fdbo_ivfpq_batch_search_parallel(self.h, _p(q), nq, k, nthreads, _p(ids), _p(d),
                                                   _p(cnt))
        else:
            lib().fdbo_ivfpq_batch_search(self.h, _p(q), nq, k, _p(ids), _p(d), _p(cnt))
        return ids[:, :k], d[:, :k], cnt


# ---- brute force / IVF-flat ---------------------------------------------------
def bf_search(data, ids, metric_id: int, q, k: int, parallel: bool = False):
    d, q = _f(data), _f(q)
    idv = np.ascontiguousarray(ids, np.uint64)
    oid = np.empty(max(k, 1), np.uint64)
    od = np.empty(max(k, 1), np.float32)
    fn = lib().fdbo_bf_search_parallel if parallel else lib().fdbo_bf_search
    cnt = fn(_p(d), _p(idv), d.shape[0], d.shape[1], metric_id, _p(q), k, _p(oid), _p(od))
    return oid[:cnt], od[:cnt]


def bf_batch_search(data, ids, metric_id: int, queries, k: int, nthreads: int = 0):
    d, q = _f(data), _f(queries)
    idv = np.ascontiguousarray(ids, np.uint64)
    nq = q.shape[0]
    oid = np.full((nq, max(k, 1)), np.iinfo(np.uint64).max, np.uint64)
    od = np.full((nq, max(k, 1)), np.inf, np.float32)
    cnt = np.zeros(nq, np.int32)
    lib().fdbo_bf_batch_search(_p(d), _p(idv), d.shape[0], d.shape[1], metric_id, _p(q), nq, k,
                               nthreads, _p(oid), _p(od), _p(cnt))
    return oid[:, :k], od[:, :k], cnt


def ivf_probes(centroids, q, nprobe: int):
    c, q = _f(centroids), _f(q)
    out = np.empty(max(nprobe, 1), np.int32)
    cnt = lib().fdbo_ivf_probes(_p(c), c.shape[0], c.shape[1], _p(q), nprobe, _p(out))
    return out[:cnt]


def ivf_batch_search(centroids, list_offsets, ids, rows, metric_id: int, nprobe: int, queries,
                     k: int, nthreads: int = 0):
    c, r, q = _f(centroids), _f(rows), _f(queries)
    off = np.ascontiguousarray(list_offsets, np.uint64)
    idv = np.ascontiguousarray(ids, np.uint64)
    nq = q.shape[0]
    oid = np.full((nq, max(k, 1)), np.iinfo(np.uint64).max, np.uint64)
    od = np.full((nq, max(k, 1)), np.inf, np.float32)
    cnt = np.zeros(nq, np.int32)
    lib().fdbo_ivf_batch_search(_p(c), c.shape[0], c.shape[1], _p(off), _p(idv), _p(r), metric_id,
                                nprobe, _p(q), nq, k, nthreads, _p(oid), _p(od), _p(cnt))
    return oid[:, :k], od[:, :k], cnt


def splitmix64_at(seed: int, i: int) -> int:
    return int(lib().fdbo_splitmix64_at(seed, i))


def ivf_build(vectors, nlist: int, seed: int, nthreads: int = 0):
    """IVFIndex::build restated: (centroids, list_offsets, order) where order
    holds the input row of each list-order position."""
    v = _f(vectors)
    n, dim = v.shape
    cen = np.empty((nlist, dim), np.float32)
    off = np.empty(nlist + 1, np.uint64)
    order = np.empty(n, np.uint64)
    if lib().fdbo_ivf_build(_p(v), n, dim, nlist, seed, nthreads, _p(cen), _p(off), _p(order)):
        raise ValueError("IVF build needs n >= nlist > 0")
    return cen, off, order
