"""Reranking against original_vectors as the reference keeps them: a map
id -> vector (ivf_pq.rs:356).  delete removes the id's vector (:1793-1797),
insert_batch replaces it (:1769-1773), a loaded file holds whatever records
were saved (from_serializable, :1918-1925; tombstones are not saved, so a
deleted entry comes back without a vector), and rerank_results drops a
candidate without one (filter_map, :562-571).  The HIP path against the
oracle's literal map, bit for bit."""
import os
import tempfile

import numpy as np
import pytest

import refcpu
from forgedb import IVFPQIndex, datagen
from test_ivfpq_gpu import _bincode_ivfpq, _bincode_vector, _fdb_file, check_batch, gpu_index

pytestmark = pytest.mark.gpu


def _check_single(gx, ox, queries, k, label):
    for t, q in enumerate(queries):
        res = gx.search(q, k)
        gi = np.array([i for i, _ in res], np.uint64)
        gd = np.array([d for _, d in res], np.float32)
        oi, od = ox.search(q, k)
        assert np.array_equal(gd, od), f"{label} q{t}"
        assert np.array_equal(gi, oi), f"{label} q{t}"


@pytest.fixture(scope="module")
def dup_index():
    base, queries = datagen.workload("ivfpq_int", n=6000, nq=32)
    base[4000:4200] = base[0:200]
    ox = refcpu.IvfPq.build(base, nlist=16, M=16, seed=8)
    art = ox.export()
    ids = art["ids"].copy()
    ids[ids < 150] += 700  # ids 700..849 held by two list entries each
    art = dict(art, ids=ids)
    qs = np.concatenate([queries, base[700:708], base[0:8] + 1.0]).astype(np.float32)
    return base, qs, art


def test_rerank_by_id_through_delete_and_insert(dup_index):
    print("rerank by id: enable, delete, insert", flush=True)
    base, qs, art = dup_index
    orig = base[np.arange(len(art["ids"]))]  # any list-order vectors
    gx = gpu_index(art)
    ox = refcpu.IvfPq.create(art["centroids"], art["codebooks"], art["list_offsets"], art["ids"], art["codes"])
    gx.enable_reranking(orig, 4)
    ox.enable_reranking(orig, 4)
    for nprobe in (3, 16):
        gx.set_nprobe(nprobe)
        ox.set_nprobe(nprobe)
        check_batch(gx, ox, qs, 10, f"enable np{nprobe}")
        _check_single(gx, ox, qs[:12], 10, f"enable single np{nprobe}")
    # deleting a duplicated id: one entry tombstoned, the other loses its vector
    for vid in (705, 711, 3000):
        assert gx.delete(vid) and ox.delete(vid)
    check_batch(gx, ox, qs, 10, "delete")
    _check_single(gx, ox, qs[:12], 10, "delete single")
    # inserting an existing id: every entry of it reranks with the new vector
    newv = (base[[720, 705, 9]] + 2.0).astype(np.float32)
    nid = np.array([720, 705, 9], np.uint64)
    gx.insert_batch(newv, nid)
    ox.insert(newv, nid)
    check_batch(gx, ox, qs, 10, "insert")
    _check_single(gx, ox, qs[:12], 10, "insert single")
    gx.compact()
    ox.compact()
    check_batch(gx, ox, qs, 10, "compact")


def test_delete_save_reload_drops_the_deleted_entry_at_rerank(dup_index):
    print("delete, save, reload, reranked search", flush=True)
    base, qs, art = dup_index
    orig = base[np.arange(len(art["ids"]))]
    gx = gpu_index(art)
    gx.enable_reranking(orig, 3)
    gx.set_nprobe(16)
    deleted = (int(art["ids"][5]), 712)
    for vid in deleted:
        assert gx.delete(vid)
    with tempfile.TemporaryDirectory() as d:
        p = os.path.join(d, "ix.fdb")
        gx.save(p)
        lx = IVFPQIndex.load(p)
    ex = lx.export()
    # tombstones are not saved: every entry is back
    for key in ("list_offsets", "ids", "codes"):
        assert np.array_equal(ex[key], art[key]), key
    assert lx.describe()["reranking"] == 1
    # the oracle as the reference's load leaves it: the records saved are
    # one per id with a vector, the deleted ids without one
    ox = refcpu.IvfPq.create(ex["centroids"], ex["codebooks"], ex["list_offsets"], ex["ids"], ex["codes"])
    seen, rid, rvec = set(), [], []
    for pos, vid in enumerate(art["ids"].tolist()):
        if vid in deleted or vid in seen:
            continue
        seen.add(vid)
        rid.append(vid)
        last = max(i for i, v in enumerate(art["ids"].tolist()) if v == vid) if vid >= 700 else pos
        rvec.append(orig[last])
    ox.set_originals(np.array(rid, np.uint64), np.stack(rvec), 3)
    ox.set_nprobe(16)
    check_batch(lx, ox, qs, 10, "reloaded")
    _check_single(lx, ox, qs[:12], 10, "reloaded single")


def test_load_partial_originals_and_stored_fields():
    """An independently written file whose original_vectors lacks some
    indexed ids, a stored nprobe above nlist and a rerank factor of 0."""
    print("partial originals file", flush=True)
    base, qs = datagen.workload("ivfpq_int", n=3000, nq=16)
    ox0 = refcpu.IvfPq.build(base, nlist=8, M=16, seed=3)
    art = ox0.export()
    keep = [int(i) for i in art["ids"] if int(i) % 5]
    recs = [(i, base[i]) for i in keep]
    with tempfile.TemporaryDirectory() as d:
        p = os.path.join(d, "ix.fdb")
        open(p, "wb").write(_fdb_file(1, _bincode_ivfpq(art, 99, 0, 2, originals=recs)))
        lx = IVFPQIndex.load(p)
        # from_serializable keeps the stored nprobe (ivf_pq.rs:1937); searches clamp it
        assert lx.nprobe() == 99
        ox = refcpu.IvfPq.create(art["centroids"], art["codebooks"], art["list_offsets"], art["ids"],
                                 art["codes"])
        ox.set_originals(np.array(keep, np.uint64), np.stack([v for _, v in recs]), 2)
        ox.set_nprobe(8)
        check_batch(lx, ox, qs, 10, "partial")
        _check_single(lx, ox, qs[:8], 10, "partial single")
        # saving writes back exactly the records it holds (as a set)
        p2 = os.path.join(d, "ix2.fdb")
        lx.save(p2)
        raw = open(p2, "rb").read()[24:]
        head = _bincode_ivfpq(art, 99, 0, 2)[:-9]
        assert raw[:len(head)] == head
        rec = 16 + 4 * art["centroids"].shape[1]
        n = int(np.frombuffer(raw[len(head) + 1:len(head) + 9], "<u8")[0])
        assert n == len(keep)
        body = raw[len(head) + 9:len(head) + 9 + n * rec]
        assert {body[r * rec:(r + 1) * rec] for r in range(n)} == {_bincode_vector(i, v) for i, v in recs}
        # a stored rerank factor of 0 keeps no candidate: empty results
        open(p, "wb").write(_fdb_file(1, _bincode_ivfpq(art, 4, 0, 0, originals=recs)))
        zx = IVFPQIndex.load(p)
        ids, d0, cnt = zx.batch_search_arrays(qs, 10)
        assert np.all(cnt == 0)
        oz = refcpu.IvfPq.create(art["centroids"], art["codebooks"], art["list_offsets"], art["ids"],
                                 art["codes"])
        oz.set_originals(np.array(keep, np.uint64), np.stack([v for _, v in recs]), 0)
        oz.set_nprobe(4)
        assert np.all(oz.batch_search(qs, 10)[2] == 0)
        assert zx.search(qs[0], 10) == [] and len(oz.search(qs[0], 10)[0]) == 0
