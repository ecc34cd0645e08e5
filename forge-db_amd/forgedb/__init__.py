"""forgedb — Python mirror of forge-db's query-path API on MI355X.

Thin ctypes layer over ``lib/libforgedb_hip.so`` (the C ABI declared in
``include/forgedb_hip.h``).  Names, argument meaning and error behaviour follow
the reference's Rust API:

* ``IVFPQIndex``  — src/index/ivf_pq.rs: ``build``, ``set_nprobe``/``nprobe``,
  ``search``, ``batch_search``, ``batch_search_parallel``, ``save``/``load``,
  ``enable_reranking``.
* ``BruteForceIndex`` — src/index/brute_force.rs: ``new``/``add``/``remove``,
  ``search``, ``search_parallel``, ``batch_search``, ``save``/``load``.
* ``IVFIndex`` — src/index/ivf.rs: ``build``, ``set_nprobe``/``nprobe``,
  ``search``, ``search_parallel``, ``batch_search``, ``batch_search_optimized``.
* ``DistanceMetric`` — src/distance/mod.rs:17-32.

There is no CPU fallback: when the HIP library is absent, importing works but
every constructor raises ``RuntimeError``.
"""
from __future__ import annotations

import ctypes as C
import enum
import os
from typing import List, Optional, Sequence, Tuple

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_HERE), "lib", "libforgedb_hip.so")

__all__ = [
    "DistanceMetric", "ForgeDbError", "IVFPQIndex", "BruteForceIndex", "IVFIndex",
    "IVFPQ_AUTO", "IVFPQ_EXACT", "IVFPQ_SCREEN", "IVFPQ_SCREEN_SORTED",
    "load_library", "LIB_PATH",
    "EXPORTED_SYMBOLS",
]

# every symbol declared in include/forgedb_hip.h
EXPORTED_SYMBOLS = (
    "fdb_last_error", "fdb_version",
    "fdb_ivfpq_create", "fdb_ivfpq_build", "fdb_ivfpq_load", "fdb_ivfpq_save",
    "fdb_ivfpq_destroy", "fdb_ivfpq_set_nprobe", "fdb_ivfpq_nprobe",
    "fdb_ivfpq_describe", "fdb_ivfpq_export", "fdb_ivfpq_enable_reranking",
    "fdb_ivfpq_search", "fdb_ivfpq_batch_search", "fdb_ivfpq_batch_search_device",
    "fdb_ivfpq_batch_search_device_noalloc",
    "fdb_ivfpq_sync", "fdb_ivfpq_probe", "fdb_ivfpq_encode",
    "fdb_ivfpq_batch_search_device_timed", "fdb_ivfpq_set_lut_mode", "fdb_ivfpq_lut_mode",
    "fdb_ivfpq_search_filtered", "fdb_ivfpq_delete", "fdb_ivfpq_insert", "fdb_ivfpq_compact",
    "fdb_ivfpq_len", "fdb_ivfpq_num_tombstones", "fdb_ivfpq_set_coarse_mode", "fdb_ivf_set_coarse_mode",
    "fdb_ivf_set_search_mode", "fdb_ivf_last_fallbacks", "fdb_ivf_last_search_path",
    "fdb_ivf_last_screen_kernel_ms",
    "fdb_ivfpq_set_search_mode", "fdb_ivfpq_last_screen_stats", "fdb_ivfpq_last_search_path",
    "fdb_ivfpq_last_screen_kernel_ms",
    "fdb_bf_create", "fdb_bf_add", "fdb_bf_remove", "fdb_bf_len", "fdb_bf_dimension",
    "fdb_bf_metric", "fdb_bf_load", "fdb_bf_save", "fdb_bf_destroy", "fdb_bf_export",
    "fdb_bf_search", "fdb_bf_batch_search", "fdb_bf_batch_search_device",
    "fdb_bf_set_search_mode", "fdb_bf_last_fallbacks", "fdb_bf_last_search_path",
    "fdb_ivf_create", "fdb_ivf_build", "fdb_ivf_destroy", "fdb_ivf_set_nprobe", "fdb_ivf_nprobe",
    "fdb_ivf_len", "fdb_ivf_num_partitions", "fdb_ivf_dimension", "fdb_ivf_export",
    "fdb_ivf_search", "fdb_ivf_batch_search", "fdb_ivf_batch_search_device", "fdb_ivf_sync",
    "fdb_ivf_probe",
)

LUT_EXACT, LUT_FAST = 0, 1
BF_AUTO, BF_EXACT, BF_SCREEN, BF_SCREEN_F32 = 0, 1, 2, 3
IVF_AUTO, IVF_EXACT, IVF_SCREEN_LISTS = 0, 1, 2
IVFPQ_AUTO, IVFPQ_EXACT, IVFPQ_SCREEN, IVFPQ_SCREEN_SORTED = 0, 1, 2, 3
COARSE_AUTO, COARSE_EXACT, COARSE_SCREEN = 0, 1, 2


class DistanceMetric(enum.IntEnum):
    """src/distance/mod.rs:17-32 (ordinals as the brute-force metric byte)."""
    Euclidean = 0
    EuclideanSquared = 1
    Cosine = 2
    DotProduct = 3
    Manhattan = 4


STATUS_NAMES = {
    0: "Ok", -1: "InvalidArgument", -2: "DimensionMismatch", -3: "NaN",
    -4: "OutOfMemory", -5: "Hip", -6: "Io", -7: "InvalidFormat",
    -8: "ChecksumMismatch", -9: "Unsupported", -10: "NoDevice",
}


class ForgeDbError(RuntimeError):
    """A nonzero fdb_status; ``.status`` holds the code, ``.kind`` its name."""

    def __init__(self, status: int, message: str):
        self.status = status
        self.kind = STATUS_NAMES.get(status, str(status))
        super().__init__(f"{self.kind}: {message}")


class _Desc(C.Structure):
    _fields_ = [("nlist", C.c_uint32), ("dim", C.c_uint32), ("n_subvectors", C.c_uint32),
                ("subvector_dim", C.c_uint32), ("n_vectors", C.c_uint64),
                ("metric", C.c_uint32), ("reranking", C.c_uint32),
                ("rerank_factor", C.c_uint64)]


_lib_handle = None
_P = C.c_void_p


def load_library(path: str = LIB_PATH) -> C.CDLL:
    """Load the HIP library (once).  Raises RuntimeError when it is not built."""
    global _lib_handle
    if _lib_handle is not None:
        return _lib_handle
    if not os.path.exists(path):
        raise RuntimeError(
            f"forgedb HIP library not found at {path}; build it with "
            "`python -c 'import __graft_entry__ as g; g.build()'` (make -C forge-db_amd)")
    lib = C.CDLL(path)
    lib.fdb_last_error.restype = C.c_char_p
    lib.fdb_version.restype = C.c_char_p
    st = C.c_int32
    sig = {
        "fdb_ivfpq_create": [_P, C.c_uint32, C.c_uint32, _P, C.c_uint32, _P, _P, _P, C.c_uint32, _P],
        "fdb_ivfpq_build": [_P, _P, C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
                            C.c_uint64, _P],
        "fdb_ivfpq_load": [C.c_char_p, _P],
        "fdb_ivfpq_save": [_P, C.c_char_p],
        "fdb_ivfpq_describe": [_P, _P],
        "fdb_ivfpq_export": [_P, _P, _P, _P, _P, _P],
        "fdb_ivfpq_enable_reranking": [_P, _P, C.c_uint64],
        "fdb_ivfpq_search": [_P, _P, C.c_uint32, C.c_uint32, _P, _P, _P],
        "fdb_ivfpq_batch_search": [_P, _P, C.c_uint64, C.c_uint32, C.c_uint32, _P, _P, _P],
        "fdb_ivfpq_batch_search_device": [_P, _P, C.c_uint64, C.c_uint32, _P, _P, _P, _P],
        "fdb_ivfpq_batch_search_device_noalloc": [_P, _P, C.c_uint64, C.c_uint32, _P, _P, _P, _P],
        "fdb_ivfpq_batch_search_device_timed": [_P, _P, C.c_uint64, C.c_uint32, _P, _P, _P, _P,
                                                _P, _P],
        "fdb_ivfpq_sync": [_P, _P],
        "fdb_ivfpq_probe": [_P, _P, C.c_uint64, C.c_uint32, C.c_uint32, _P, _P],
        "fdb_ivfpq_encode": [_P, _P, C.c_uint64, C.c_uint32, _P],
        "fdb_ivfpq_set_lut_mode": [_P, C.c_uint32],
        "fdb_ivfpq_search_filtered": [_P, _P, C.c_uint64, C.c_uint32, C.c_uint32, _P, C.c_uint64, _P,
                                      _P, _P],
        "fdb_ivfpq_delete": [_P, C.c_uint64, _P],
        "fdb_ivfpq_insert": [_P, _P, _P, C.c_uint64, C.c_uint32],
        "fdb_ivfpq_compact": [_P],
        "fdb_ivfpq_set_coarse_mode": [_P, C.c_uint32],
        "fdb_ivfpq_set_search_mode": [_P, C.c_uint32],
        "fdb_ivfpq_last_screen_stats": [_P, _P, _P, _P],
        "fdb_ivfpq_last_search_path": [_P, _P],
        "fdb_ivfpq_last_screen_kernel_ms": [_P, _P],
        "fdb_ivf_set_coarse_mode": [_P, C.c_uint32],
        "fdb_ivf_set_search_mode": [_P, C.c_uint32],
        "fdb_ivf_last_fallbacks": [_P, _P, _P],
        "fdb_ivf_last_search_path": [_P, _P],
        "fdb_ivf_last_screen_kernel_ms": [_P, _P],
        "fdb_bf_create": [C.c_uint32, _P],
        "fdb_bf_add": [_P, _P, _P, C.c_uint64, C.c_uint32],
        "fdb_bf_remove": [_P, C.c_uint64, _P],
        "fdb_bf_load": [C.c_char_p, _P],
        "fdb_bf_save": [_P, C.c_char_p],
        "fdb_bf_export": [_P, _P, _P],
        "fdb_bf_search": [_P, _P, C.c_uint32, C.c_uint32, _P, _P, _P],
        "fdb_bf_batch_search": [_P, _P, C.c_uint64, C.c_uint32, C.c_uint32, _P, _P, _P],
        "fdb_bf_batch_search_device": [_P, _P, C.c_uint64, C.c_uint32, _P, _P, _P, _P, _P],
        "fdb_bf_set_search_mode": [_P, C.c_uint32],
        "fdb_bf_last_fallbacks": [_P, _P, _P],
        "fdb_bf_last_search_path": [_P, _P],
        "fdb_ivf_create": [_P, C.c_uint32, C.c_uint32, _P, _P, _P, C.c_uint32, _P],
        "fdb_ivf_build": [_P, _P, C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint64, _P],
        "fdb_ivf_export": [_P, _P, _P, _P, _P],
        "fdb_ivf_search": [_P, _P, C.c_uint32, C.c_uint32, _P, _P, _P],
        "fdb_ivf_batch_search": [_P, _P, C.c_uint64, C.c_uint32, C.c_uint32, _P, _P, _P],
        "fdb_ivf_batch_search_device": [_P, _P, C.c_uint64, C.c_uint32, _P, _P, _P, _P, _P, _P],
        "fdb_ivf_sync": [_P, _P],
        "fdb_ivf_probe": [_P, _P, C.c_uint64, C.c_uint32, C.c_uint32, _P],
    }
    for name, args in sig.items():
        f = getattr(lib, name)
        f.argtypes = args
        f.restype = st
    lib.fdb_ivfpq_destroy.argtypes = [_P]
    lib.fdb_ivfpq_destroy.restype = None
    lib.fdb_ivfpq_set_nprobe.argtypes = [_P, C.c_uint64]
    lib.fdb_ivfpq_set_nprobe.restype = None
    lib.fdb_ivfpq_nprobe.argtypes = [_P]
    lib.fdb_ivfpq_nprobe.restype = C.c_uint64
    lib.fdb_ivfpq_lut_mode.argtypes = [_P]
    lib.fdb_ivfpq_lut_mode.restype = C.c_uint32
    for name, res in (("fdb_ivfpq_len", C.c_uint64), ("fdb_ivfpq_num_tombstones", C.c_uint64),
                      ("fdb_bf_destroy", None), ("fdb_bf_len", C.c_uint64),
                      ("fdb_bf_dimension", C.c_uint32), ("fdb_bf_metric", C.c_uint32),
                      ("fdb_ivf_destroy", None), ("fdb_ivf_nprobe", C.c_uint64),
                      ("fdb_ivf_len", C.c_uint64), ("fdb_ivf_num_partitions", C.c_uint32),
                      ("fdb_ivf_dimension", C.c_uint32)):
        f = getattr(lib, name)
        f.argtypes = [_P]
        f.restype = res
    lib.fdb_ivf_set_nprobe.argtypes = [_P, C.c_uint64]
    lib.fdb_ivf_set_nprobe.restype = None
    _lib_handle = lib
    return lib


def _check(lib, status: int) -> None:
    if status != 0:
        raise ForgeDbError(status, lib.fdb_last_error().decode(errors="replace"))


def _ptr(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _rows(results_ids: np.ndarray, results_d: np.ndarray, counts: np.ndarray):
    return [[(int(results_ids[q, j]), float(results_d[q, j])) for j in range(int(counts[q]))]
            for q in range(results_ids.shape[0])]


class IVFPQIndex:
    """IVF-PQ index resident in HBM — src/index/ivf_pq.rs:343-359.

    Lists are stored in list order as CSR: ``list_offsets[nlist+1]`` into
    ``ids[N]`` (u64) and ``codes[N, M]`` (u8); ``centroids[nlist, dim]`` and
    ``codebooks[M, 256, dim // M]`` are f32.
    """

    def __init__(self, handle: int):
        self._lib = load_library()
        self._h = C.c_void_p(handle)
        d = _Desc()
        _check(self._lib, self._lib.fdb_ivfpq_describe(self._h, C.byref(d)))
        self.nlist, self._dim = int(d.nlist), int(d.dim)
        self.n_subvectors, self.subvector_dim = int(d.n_subvectors), int(d.subvector_dim)
        self.metric = DistanceMetric(int(d.metric))

    # -- construction -------------------------------------------------------
    @classmethod
    def from_artifacts(cls, centroids, codebooks, list_offsets, ids, codes,
                       metric: DistanceMetric = DistanceMetric.Euclidean) -> "IVFPQIndex":
        lib = load_library()
        cen = _f32(centroids)
        cb = _f32(codebooks)
        off = np.ascontiguousarray(list_offsets, dtype=np.uint64)
        idv = np.ascontiguousarray(ids, dtype=np.uint64)
        cod = np.ascontiguousarray(codes, dtype=np.uint8)
        nlist, dim = cen.shape
        M = cb.shape[0]
        out = C.c_void_p()
        _check(lib, lib.fdb_ivfpq_create(_ptr(cen), nlist, dim, _ptr(cb), M, _ptr(off),
                                         _ptr(idv), _ptr(cod), int(metric), C.byref(out)))
        return cls(out.value)

    @classmethod
    def build(cls, vectors, n_clusters: int, n_subvectors: int,
              metric: DistanceMetric = DistanceMetric.Euclidean, seed: int = 0,
              ids=None) -> "IVFPQIndex":
        """IVFPQIndex::build (ivf_pq.rs:374-506), on the GPU, seeded."""
        lib = load_library()
        v = _f32(vectors)
        idv = None if ids is None else np.ascontiguousarray(ids, dtype=np.uint64)
        out = C.c_void_p()
        _check(lib, lib.fdb_ivfpq_build(_ptr(v), _ptr(idv), v.shape[0], v.shape[1], n_clusters,
                                        n_subvectors, int(metric), seed, C.byref(out)))
        return cls(out.value)

    @classmethod
    def load(cls, path: str) -> "IVFPQIndex":
        """Persistable::load (ivf_pq.rs:1977-1982)."""
        lib = load_library()
        out = C.c_void_p()
        _check(lib, lib.fdb_ivfpq_load(os.fsencode(path), C.byref(out)))
        return cls(out.value)

    load_mmap = load  # ivf_pq.rs:1984-1993 deserialises into owned memory too

    def save(self, path: str) -> None:
        _check(self._lib, self._lib.fdb_ivfpq_save(self._h, os.fsencode(path)))

    def close(self) -> None:
        if self._h is not None and self._h.value:
            self._lib.fdb_ivfpq_destroy(self._h)
        self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- configuration --------------------------------------------------------
    def set_nprobe(self, nprobe: int) -> None:
        self._lib.fdb_ivfpq_set_nprobe(self._h, int(nprobe))

    def nprobe(self) -> int:
        return int(self._lib.fdb_ivfpq_nprobe(self._h))

    def set_lut_mode(self, mode: int) -> None:
        """LUT_EXACT (default, bit-identical distances) or LUT_FAST."""
        _check(self._lib, self._lib.fdb_ivfpq_set_lut_mode(self._h, int(mode)))

    def lut_mode(self) -> int:
        return int(self._lib.fdb_ivfpq_lut_mode(self._h))

    def set_coarse_mode(self, mode: int) -> None:
        """COARSE_AUTO, COARSE_EXACT or COARSE_SCREEN; same probes in every mode."""
        _check(self._lib, self._lib.fdb_ivfpq_set_coarse_mode(self._h, int(mode)))

    def set_search_mode(self, mode: int) -> None:
        """IVFPQ_AUTO (default: half-precision screening with exact rescoring
        for large plain batches), IVFPQ_EXACT (table scan only) or
        IVFPQ_SCREEN (screening wherever it applies) or IVFPQ_SCREEN_SORTED
        (screening with the size-sorted tile schedule of large indexes,
        whatever the size); same results."""
        _check(self._lib, self._lib.fdb_ivfpq_set_search_mode(self._h, int(mode)))

    def last_screen_stats(self, stream: int = 0):
        """(queries rescanned exactly, candidates rescored) of the last batch."""
        fb, cand = C.c_uint64(), C.c_uint64()
        _check(self._lib, self._lib.fdb_ivfpq_last_screen_stats(self._h, C.c_void_p(stream), C.byref(fb),
                                                                C.byref(cand)))
        return int(fb.value), int(cand.value)

    def last_search_path(self) -> int:
        """How the last batch ran: 0 table scan, 2 fp16 screening."""
        out = C.c_uint32()
        _check(self._lib, self._lib.fdb_ivfpq_last_search_path(self._h, C.byref(out)))
        return int(out.value)

    def last_screen_kernel_ms(self) -> float:
        """The threshold screening kernel's duration in the last timed batch
        (HIP events on its stream; 0 after a table scan)."""
        out = C.c_float()
        _check(self._lib, self._lib.fdb_ivfpq_last_screen_kernel_ms(self._h, C.byref(out)))
        return float(out.value)

    def dim(self) -> int:
        return self._dim

    def n_partitions(self) -> int:
        return self.nlist

    def describe(self) -> dict:
        d = _Desc()
        _check(self._lib, self._lib.fdb_ivfpq_describe(self._h, C.byref(d)))
        return {f: getattr(d, f) for f, _ in _Desc._fields_}

    def __len__(self) -> int:
        """len (ivf_pq.rs:1088-1094): entries minus tombstones."""
        return int(self._lib.fdb_ivfpq_len(self._h))

    def len_with_tombstones(self) -> int:
        return int(self.describe()["n_vectors"])

    def num_tombstones(self) -> int:
        return int(self._lib.fdb_ivfpq_num_tombstones(self._h))

    def delete(self, vector_id: int) -> bool:
        """delete (ivf_pq.rs:1786-1804)."""
        out = C.c_int()
        _check(self._lib, self._lib.fdb_ivfpq_delete(self._h, int(vector_id), C.byref(out)))
        return bool(out.value)

    def insert_batch(self, vectors, ids=None) -> None:
        """insert_batch (ivf_pq.rs:1731-1776)."""
        v = _f32(vectors)
        idv = None if ids is None else np.ascontiguousarray(ids, np.uint64)
        _check(self._lib, self._lib.fdb_ivfpq_insert(self._h, _ptr(v), _ptr(idv), v.shape[0],
                                                     v.shape[1]))

    def compact(self) -> None:
        """compact (ivf_pq.rs:1828-1851)."""
        _check(self._lib, self._lib.fdb_ivfpq_compact(self._h))

    def search_filtered_arrays(self, queries, k: int, allowed_ids):
        """search_filtered per query; the filter given as the admitted ids."""
        q = _f32(queries)
        if q.ndim == 1:
            q = q.reshape(1, -1)
        allow = np.ascontiguousarray(allowed_ids, np.uint64)
        nq = q.shape[0]
        ids = np.empty((nq, max(k, 1)), np.uint64)
        d = np.empty((nq, max(k, 1)), np.float32)
        counts = np.empty(nq, np.uint32)
        _check(self._lib, self._lib.fdb_ivfpq_search_filtered(
            self._h, _ptr(q), nq, q.shape[1], k, _ptr(allow), allow.shape[0], _ptr(ids), _ptr(d),
            _ptr(counts)))
        return ids[:, :k], d[:, :k], counts

    def search_filtered(self, query, k: int, allowed_ids) -> List[Tuple[int, float]]:
        """search_filtered (ivf_pq.rs:692-831) -> [(id, dist)] ascending."""
        ids, d, c = self.search_filtered_arrays(query, k, allowed_ids)
        return [(int(ids[0, j]), float(d[0, j])) for j in range(int(c[0]))]

    def enable_reranking(self, vectors_list_order, rerank_factor: int) -> None:
        """enable_reranking (ivf_pq.rs:513-517); vectors given in list order."""
        v = _f32(vectors_list_order)
        _check(self._lib, self._lib.fdb_ivfpq_enable_reranking(self._h, _ptr(v), rerank_factor))

    def export(self) -> dict:
        d = self.describe()
        n, M, dim = d["n_vectors"], d["n_subvectors"], d["dim"]
        out = dict(centroids=np.empty((self.nlist, dim), np.float32),
                   codebooks=np.empty((M, 256, d["subvector_dim"]), np.float32),
                   list_offsets=np.empty(self.nlist + 1, np.uint64),
                   ids=np.empty(n, np.uint64), codes=np.empty((n, M), np.uint8))
        _check(self._lib, self._lib.fdb_ivfpq_export(
            self._h, _ptr(out["centroids"]), _ptr(out["codebooks"]), _ptr(out["list_offsets"]),
            _ptr(out["ids"]), _ptr(out["codes"])))
        return out

    def list_offsets(self) -> np.ndarray:
        off = np.empty(self.nlist + 1, np.uint64)
        _check(self._lib, self._lib.fdb_ivfpq_export(self._h, None, None, _ptr(off), None, None))
        return off

    # -- search -------------------------------------------------------------
    def search(self, query, k: int) -> List[Tuple[int, float]]:
        """search (ivf_pq.rs:590-677) -> [(id, squared ADC distance)] ascending."""
        q = _f32(query).reshape(-1)
        ids = np.empty(max(k, 1), np.uint64)
        d = np.empty(max(k, 1), np.float32)
        cnt = C.c_uint32()
        _check(self._lib, self._lib.fdb_ivfpq_search(self._h, _ptr(q), q.shape[0], k, _ptr(ids),
                                                     _ptr(d), C.byref(cnt)))
        return [(int(ids[j]), float(d[j])) for j in range(cnt.value)]

    def batch_search_arrays(self, queries, k: int):
        """batch_search as arrays: (ids [nq,k] u64, dists [nq,k] f32, counts [nq])."""
        q = _f32(queries)
        if q.ndim != 2:
            raise ForgeDbError(-1, "queries must be [nq, dim]")
        nq = q.shape[0]
        ids = np.empty((nq, max(k, 1)), np.uint64)
        d = np.empty((nq, max(k, 1)), np.float32)
        counts = np.empty(nq, np.uint32)
        _check(self._lib, self._lib.fdb_ivfpq_batch_search(self._h, _ptr(q), nq, q.shape[1], k,
                                                           _ptr(ids), _ptr(d), _ptr(counts)))
        return ids[:, :k], d[:, :k], counts

    def batch_search(self, queries: Sequence, k: int) -> List[List[Tuple[int, float]]]:
        """batch_search (ivf_pq.rs:850-1047) -> per query [(id, dist)] ascending."""
        if len(queries) == 0:
            return []
        ids, d, counts = self.batch_search_arrays(np.asarray(queries, np.float32), k)
        return _rows(ids, d, counts)

    # on the GPU the chunked Rayon variant (ivf_pq.rs:1060-1084) is the same launch
    batch_search_parallel = batch_search

    def batch_search_device(self, d_queries: int, nq: int, k: int, d_ids: int, d_dists: int,
                            d_counts: int, stream: int = 0, timed: bool = False):
        """Device pointers in and out; enqueues on `stream`.  With timed=True
        waits and returns (coarse_ms, scan_ms) from HIP events on that stream."""
        if timed:
            cm, sm = C.c_float(), C.c_float()
            _check(self._lib, self._lib.fdb_ivfpq_batch_search_device_timed(
                self._h, C.c_void_p(d_queries), nq, k, C.c_void_p(d_ids), C.c_void_p(d_dists),
                C.c_void_p(d_counts), C.c_void_p(stream), C.byref(cm), C.byref(sm)))
            return cm.value, sm.value
        _check(self._lib, self._lib.fdb_ivfpq_batch_search_device(
            self._h, C.c_void_p(d_queries), nq, k, C.c_void_p(d_ids), C.c_void_p(d_dists),
            C.c_void_p(d_counts), C.c_void_p(stream)))
        return None

    def batch_search_device_noalloc(self, d_queries: int, nq: int, k: int, d_ids: int, d_dists: int,
                                    d_counts: int, stream: int = 0) -> None:
        """batch_search_device without device allocation (its probe lists in
        a static device array; plain indexes, nq * nprobe <= 2^21)."""
        _check(self._lib, self._lib.fdb_ivfpq_batch_search_device_noalloc(
            self._h, C.c_void_p(d_queries), nq, k, C.c_void_p(d_ids), C.c_void_p(d_dists),
            C.c_void_p(d_counts), C.c_void_p(stream)))

    def sync(self, stream: int = 0) -> None:
        _check(self._lib, self._lib.fdb_ivfpq_sync(self._h, C.c_void_p(stream)))

    def probe(self, queries, nprobe: int):
        """Coarse quantizer: (lists [nq,nprobe] i32, dists [nq,nprobe] f32)."""
        q = _f32(queries)
        nq = q.shape[0]
        lists = np.empty((nq, nprobe), np.int32)
        d = np.empty((nq, nprobe), np.float32)
        _check(self._lib, self._lib.fdb_ivfpq_probe(self._h, _ptr(q), nq, q.shape[1], nprobe,
                                                    _ptr(lists), _ptr(d)))
        return lists, d

    def encode(self, residuals) -> np.ndarray:
        """ProductQuantizer::encode (pq.rs:114-139) of residual rows."""
        r = _f32(residuals)
        nq = r.shape[0]
        codes = np.empty((nq, self.n_subvectors), np.uint8)
        _check(self._lib, self._lib.fdb_ivfpq_encode(self._h, _ptr(r), nq, r.shape[1], _ptr(codes)))
        return codes


def _search_one(fn, h, query, k: int):
    q = _f32(query).reshape(-1)
    ids = np.empty(max(k, 1), np.uint64)
    d = np.empty(max(k, 1), np.float32)
    cnt = C.c_uint32()
    _check(load_library(), fn(h, _ptr(q), q.shape[0], k, _ptr(ids), _ptr(d), C.byref(cnt)))
    return [(int(ids[j]), float(d[j])) for j in range(cnt.value)]


def _search_batch(fn, h, queries, k: int):
    q = _f32(queries)
    if q.ndim != 2:
        raise ForgeDbError(-1, "queries must be [nq, dim]")
    nq = q.shape[0]
    ids = np.empty((nq, max(k, 1)), np.uint64)
    d = np.empty((nq, max(k, 1)), np.float32)
    counts = np.empty(nq, np.uint32)
    _check(load_library(), fn(h, _ptr(q), nq, q.shape[1], k, _ptr(ids), _ptr(d), _ptr(counts)))
    return ids[:, :k], d[:, :k], counts


def _query_rows(queries) -> np.ndarray:
    """Accepts [nq, dim] arrays or a sequence of vectors (or objects with .data)."""
    if isinstance(queries, np.ndarray):
        return queries
    return np.asarray([getattr(q, "data", q) for q in queries], np.float32)


class BruteForceIndex:
    """Exact search over all rows in HBM — src/index/brute_force.rs:60-225.

    Distances are bit-identical to DistanceMetric::compute; equal distances
    keep the earlier row first.
    """

    def __init__(self, metric: DistanceMetric = DistanceMetric.Euclidean, _handle: int = 0):
        self._lib = load_library()
        if _handle:
            self._h = C.c_void_p(_handle)
        else:
            out = C.c_void_p()
            _check(self._lib, self._lib.fdb_bf_create(int(metric), C.byref(out)))
            self._h = out
        self.metric = DistanceMetric(int(self._lib.fdb_bf_metric(self._h)))

    new = classmethod(lambda cls, metric: cls(metric))  # BruteForceIndex::new (:67)

    @classmethod
    def from_arrays(cls, rows, ids=None, metric: DistanceMetric = DistanceMetric.Euclidean):
        ix = cls(metric)
        ix.add_batch(rows, ids)
        return ix

    def add(self, vector_id: int, data) -> None:
        """add (:75) / MutableVectorIndex::add (:254-265)."""
        self.add_batch(_f32(data).reshape(1, -1), np.array([vector_id], np.uint64))

    def add_batch(self, rows, ids=None) -> None:
        r = _f32(rows)
        idv = None if ids is None else np.ascontiguousarray(ids, np.uint64)
        _check(self._lib, self._lib.fdb_bf_add(self._h, _ptr(r), _ptr(idv), r.shape[0], r.shape[1]))

    def set_search_mode(self, mode: int) -> None:
        """BF_AUTO (default), BF_EXACT (exact-order scan only), BF_SCREEN
        (matrix-core screening + exact rescoring where it applies; fp16
        products when the rows fit) or BF_SCREEN_F32 (screening with fp32
        products); same results."""
        _check(self._lib, self._lib.fdb_bf_set_search_mode(self._h, int(mode)))

    def last_search_path(self) -> int:
        """How the last search ran: 0 exact scan, 1 fp32 screening, 2 fp16
        screening."""
        out = C.c_uint32()
        _check(self._lib, self._lib.fdb_bf_last_search_path(self._h, C.byref(out)))
        return int(out.value)

    def last_fallbacks(self, stream: int = 0) -> int:
        """Queries of the last search that were rescanned exactly."""
        out = C.c_uint64()
        _check(self._lib, self._lib.fdb_bf_last_fallbacks(self._h, C.c_void_p(stream), C.byref(out)))
        return int(out.value)

    def remove(self, vector_id: int) -> bool:
        """MutableVectorIndex::remove (:267-274)."""
        out = C.c_int()
        _check(self._lib, self._lib.fdb_bf_remove(self._h, int(vector_id), C.byref(out)))
        return bool(out.value)

    def __len__(self) -> int:
        return int(self._lib.fdb_bf_len(self._h))

    def is_empty(self) -> bool:
        return len(self) == 0

    def dimension(self) -> int:
        return int(self._lib.fdb_bf_dimension(self._h))

    def export(self):
        n, dim = len(self), self.dimension()
        rows = np.empty((n, dim), np.float32)
        ids = np.empty(n, np.uint64)
        _check(self._lib, self._lib.fdb_bf_export(self._h, _ptr(rows), _ptr(ids)))
        return rows, ids

    @classmethod
    def load(cls, path: str) -> "BruteForceIndex":
        """Persistable::load (:322-385)."""
        lib = load_library()
        out = C.c_void_p()
        _check(lib, lib.fdb_bf_load(os.fsencode(path), C.byref(out)))
        return cls(_handle=out.value)

    def save(self, path: str) -> None:
        """Persistable::save (:278-320)."""
        _check(self._lib, self._lib.fdb_bf_save(self._h, os.fsencode(path)))

    def close(self) -> None:
        if self._h is not None and self._h.value:
            self._lib.fdb_bf_destroy(self._h)
        self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def search(self, query, k: int) -> List[Tuple[int, float]]:
        """search (:162-166) -> [(id, distance)] ascending."""
        return _search_one(self._lib.fdb_bf_search, self._h, query, k)

    search_prefetch = search    # :172-174
    search_parallel = search    # :180-214: one launch covers every chunk

    def batch_search_arrays(self, queries, k: int):
        return _search_batch(self._lib.fdb_bf_batch_search, self._h, queries, k)

    def batch_search(self, queries, k: int) -> List[List[Tuple[int, float]]]:
        """batch_search (:220-225)."""
        if len(queries) == 0:
            return []
        return _rows(*self.batch_search_arrays(_query_rows(queries), k))

    def batch_search_device(self, d_queries: int, nq: int, k: int, d_ids: int, d_dists: int,
                            d_counts: int, stream: int = 0, timed: bool = False):
        ms = C.c_float()
        _check(self._lib, self._lib.fdb_bf_batch_search_device(
            self._h, C.c_void_p(d_queries), nq, k, C.c_void_p(d_ids), C.c_void_p(d_dists),
            C.c_void_p(d_counts), C.c_void_p(stream), C.byref(ms) if timed else None))
        return ms.value if timed else None


class IVFIndex:
    """IVF over full vectors in HBM — src/index/ivf.rs:70-405.

    Lists are CSR in list order: ``list_offsets[nlist+1]`` into ``ids[N]`` and
    ``rows[N, dim]``.
    """

    def __init__(self, handle: int):
        self._lib = load_library()
        self._h = C.c_void_p(handle)
        self.nlist = int(self._lib.fdb_ivf_num_partitions(self._h))
        self._dim = int(self._lib.fdb_ivf_dimension(self._h))

    @classmethod
    def from_artifacts(cls, centroids, list_offsets, ids, rows,
                       metric: DistanceMetric = DistanceMetric.Euclidean) -> "IVFIndex":
        lib = load_library()
        cen = _f32(centroids)
        off = np.ascontiguousarray(list_offsets, np.uint64)
        idv = np.ascontiguousarray(ids, np.uint64)
        r = _f32(rows)
        out = C.c_void_p()
        _check(lib, lib.fdb_ivf_create(_ptr(cen), cen.shape[0], cen.shape[1], _ptr(off), _ptr(idv),
                                       _ptr(r), int(metric), C.byref(out)))
        ix = cls(out.value)
        ix.metric = DistanceMetric(int(metric))
        return ix

    @classmethod
    def build(cls, vectors, n_clusters: int, metric: DistanceMetric = DistanceMetric.Euclidean,
              seed: int = 0, ids=None) -> "IVFIndex":
        """IVFIndex::build (ivf.rs:91-119), on the GPU, seeded."""
        lib = load_library()
        v = _f32(vectors)
        idv = None if ids is None else np.ascontiguousarray(ids, np.uint64)
        out = C.c_void_p()
        _check(lib, lib.fdb_ivf_build(_ptr(v), _ptr(idv), v.shape[0], v.shape[1], n_clusters,
                                      int(metric), seed, C.byref(out)))
        ix = cls(out.value)
        ix.metric = DistanceMetric(int(metric))
        return ix

    def close(self) -> None:
        if self._h is not None and self._h.value:
            self._lib.fdb_ivf_destroy(self._h)
        self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_nprobe(self, nprobe: int) -> None:
        """set_nprobe (ivf.rs:125-127): min(nprobe, nlist)."""
        self._lib.fdb_ivf_set_nprobe(self._h, int(nprobe))

    def nprobe(self) -> int:
        return int(self._lib.fdb_ivf_nprobe(self._h))

    def set_coarse_mode(self, mode: int) -> None:
        """COARSE_AUTO, COARSE_EXACT or COARSE_SCREEN; same probes in every mode."""
        _check(self._lib, self._lib.fdb_ivf_set_coarse_mode(self._h, int(mode)))

    def set_search_mode(self, mode: int) -> None:
        """IVF_AUTO (default: half-precision screening + exact rescoring for
        Euclidean, squared Euclidean and Manhattan; large Euclidean batches
        screen list by list on the matrix cores), IVF_EXACT (exact-order scan
        only) or IVF_SCREEN_LISTS (list screening wherever it applies); same
        results."""
        _check(self._lib, self._lib.fdb_ivf_set_search_mode(self._h, int(mode)))

    def last_fallbacks(self, stream: int = 0) -> int:
        """Queries of the last search that were rescanned exactly."""
        out = C.c_uint64()
        _check(self._lib, self._lib.fdb_ivf_last_fallbacks(self._h, C.c_void_p(stream), C.byref(out)))
        return int(out.value)

    def last_search_path(self) -> int:
        """How the last search ran: 0 exact scan, 2 fp16 screening per query,
        3 list screening on the matrix cores."""
        out = C.c_uint32()
        _check(self._lib, self._lib.fdb_ivf_last_search_path(self._h, C.byref(out)))
        return int(out.value)

    def last_screen_kernel_ms(self) -> float:
        """The list screening's threshold kernel duration in the last timed
        batch (HIP events on its stream; 0 when it took another path)."""
        out = C.c_float()
        _check(self._lib, self._lib.fdb_ivf_last_screen_kernel_ms(self._h, C.byref(out)))
        return float(out.value)

    def __len__(self) -> int:
        return int(self._lib.fdb_ivf_len(self._h))

    def is_empty(self) -> bool:
        return len(self) == 0

    def num_partitions(self) -> int:
        return self.nlist

    def dimension(self) -> int:
        return self._dim

    def export(self) -> dict:
        n = len(self)
        out = dict(centroids=np.empty((self.nlist, self._dim), np.float32),
                   list_offsets=np.empty(self.nlist + 1, np.uint64),
                   ids=np.empty(n, np.uint64), rows=np.empty((n, self._dim), np.float32))
        _check(self._lib, self._lib.fdb_ivf_export(self._h, _ptr(out["centroids"]),
                                                   _ptr(out["list_offsets"]), _ptr(out["ids"]),
                                                   _ptr(out["rows"])))
        return out

    def search(self, query, k: int) -> List[Tuple[int, float]]:
        """search (ivf.rs:162-216)."""
        return _search_one(self._lib.fdb_ivf_search, self._h, query, k)

    search_parallel = search  # ivf.rs:245-290

    def batch_search_arrays(self, queries, k: int):
        return _search_batch(self._lib.fdb_ivf_batch_search, self._h, queries, k)

    def batch_search(self, queries, k: int) -> List[List[Tuple[int, float]]]:
        """batch_search (ivf.rs:292-297)."""
        if len(queries) == 0:
            return []
        return _rows(*self.batch_search_arrays(_query_rows(queries), k))

    batch_search_optimized = batch_search  # ivf.rs:313-405

    def batch_search_device(self, d_queries: int, nq: int, k: int, d_ids: int, d_dists: int,
                            d_counts: int, stream: int = 0, timed: bool = False):
        cm, sm = C.c_float(), C.c_float()
        _check(self._lib, self._lib.fdb_ivf_batch_search_device(
            self._h, C.c_void_p(d_queries), nq, k, C.c_void_p(d_ids), C.c_void_p(d_dists),
            C.c_void_p(d_counts), C.c_void_p(stream), C.byref(cm) if timed else None,
            C.byref(sm) if timed else None))
        return (cm.value, sm.value) if timed else None

    def sync(self, stream: int = 0) -> None:
        _check(self._lib, self._lib.fdb_ivf_sync(self._h, C.c_void_p(stream)))

    def probe(self, queries, nprobe: int) -> np.ndarray:
        """Coarse step: lists [nq, nprobe] i32, nearest first."""
        q = _f32(queries)
        lists = np.empty((q.shape[0], nprobe), np.int32)
        _check(self._lib, self._lib.fdb_ivf_probe(self._h, _ptr(q), q.shape[0], q.shape[1], nprobe,
                                                  _ptr(lists)))
        return lists
