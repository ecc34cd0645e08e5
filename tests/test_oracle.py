"""Pins the oracle (oracle/refcpu.*) before anything is checked against it.

Each check is one of: a known answer from the reference's own tests (cited),
a closed form, an identity the summation orders must satisfy, or brute force
on tiny inputs with float64 arithmetic.  CPU only.
"""
import math

import numpy as np
import pytest

import refcpu
from conftest import tie_aware_match

EUC, EUC2, COS, DOT, L1 = 0, 1, 2, 3, 4


# ---- known answers from the reference's tests ------------------------------
def test_metric_kats():
    # distance/mod.rs:55-105
    assert refcpu.metric(EUC, [0, 0], [3, 4]) == pytest.approx(5.0, abs=1e-5)
    assert refcpu.metric(DOT, [1, 0], [1, 0]) == pytest.approx(-1.0, abs=1e-5)
    assert refcpu.metric(COS, [1, 0], [0, 1]) == pytest.approx(1.0, abs=1e-5)
    assert abs(refcpu.metric(COS, [1, 0], [1, 0])) < 1e-5
    assert refcpu.metric(L1, [0, 0], [3, 4]) == pytest.approx(7.0, abs=1e-5)
    # tests/correctness.rs:132-178
    a = [0.0] * 8
    b = [3.0, 4.0] + [0.0] * 6
    assert refcpu.dist("l2", a, b) == pytest.approx(5.0, abs=1e-5)
    assert refcpu.dist("l2sq", a, b) == pytest.approx(25.0, abs=1e-5)
    e1 = [1.0] + [0.0] * 7
    e2 = [0.0, 1.0] + [0.0] * 6
    assert abs(refcpu.dist("dot", e1, e2)) < 1e-6
    assert refcpu.dist("l2", e1, e2) == pytest.approx(math.sqrt(2), abs=1e-5)
    # distance/scalar.rs:105-157 and simd.rs:926-1233 closed forms
    assert refcpu.dist("dot", [1, 2, 3], [4, 5, 6]) == 32.0
    assert refcpu.dist("dot", list(range(1, 9)), [1.0] * 8) == 36.0
    assert refcpu.dist("l1", [1, -2, 3], [-1, 2, -3]) == 12.0
    assert refcpu.dist("l2sq", [0.0] * 16, list(range(16))) == 1240.0


def test_cosine_zero_vector_rule():
    # simd.rs:510-516: a zero denominator gives 0 on the AVX2 path
    assert refcpu.dist("cosine", [0.0] * 8, [1.0] * 8) == 0.0
    assert refcpu.dist("cosine", [0.0] * 3, [1.0] * 3) == 0.0
    # scalar.rs:86-88 gives 1 - 0 = 1 for the same input (documented quirk)
    assert refcpu.dist("scalar_cosine", [0.0] * 8, [1.0] * 8) == 1.0


@pytest.mark.parametrize("n", [1, 3, 7, 8, 9, 15, 16, 17, 31, 64, 96, 100, 128, 1024, 4096])
def test_simd_matches_scalar_within_reference_tolerance(n):
    # tests/property.rs:51-90: SIMD == scalar within 1e-5*|s| + 1e-5;
    # deterministic ramps as in simd.rs:964-1133
    a = (np.arange(n, dtype=np.float32) * 0.01 + 0.1).astype(np.float32)
    b = (np.arange(n, dtype=np.float32) * 0.02 - 0.5).astype(np.float32)
    for simd, scal in (("l2sq", "scalar_l2sq"), ("dot", "scalar_dot"), ("l1", "scalar_l1"),
                       ("cosine", "scalar_cosine")):
        s, c = refcpu.dist(simd, a, b), refcpu.dist(scal, a, b)
        assert abs(s - c) <= 1e-5 * abs(c) + 1e-5 * max(1.0, n / 64), (simd, n, s, c)


# ---- identities that fix the summation order --------------------------------
def _seq_sum_f32(terms):
    s = np.float32(0.0)
    for t in terms:
        s = np.float32(s + np.float32(t))
    return s


@pytest.mark.parametrize("n", [1, 2, 3, 5, 8])
def test_l2sq_short_vectors_are_sequential_sums(n):
    # For n <= 8 the AVX2 routine is 8 lanes holding one rounded square each
    # (or none, below 8, all in the scalar tail), summed left to right: a
    # plain sequential f32 sum of rounded squares.
    rng = np.random.default_rng(n)
    for _ in range(200):
        a = rng.standard_normal(n).astype(np.float32) * 100
        b = rng.standard_normal(n).astype(np.float32) * 100
        d = (a - b).astype(np.float32)
        want = _seq_sum_f32(np.float32(x) * np.float32(x) for x in d)
        assert np.float32(refcpu.dist("l2sq", a, b)) == want


def test_l2sq_lane_order_differs_from_sequential_and_matches_lane_model():
    # 16 elements: lane l = fma(d[l+8], d[l+8], d[l]^2); total = lanes left to
    # right.  A sequential sum is a different rounding on this input.
    rng = np.random.default_rng(3)
    hits = 0
    for _ in range(300):
        a = (rng.standard_normal(16) * 1000).astype(np.float32)
        b = np.zeros(16, np.float32)
        d = a.astype(np.float64)
        lanes = []
        for l in range(8):
            first = np.float32(d[l] * d[l])  # exact square rounded once
            lanes.append(np.float32(np.float64(first) + d[l + 8] * d[l + 8]))  # fma: one rounding
        model = _seq_sum_f32(lanes)
        got = np.float32(refcpu.dist("l2sq", a, b))
        assert got == model
        hits += got != _seq_sum_f32(np.float32(x * x) for x in a)
    assert hits > 0  # the order matters on these inputs


def test_adc_orders():
    rng = np.random.default_rng(11)
    for M in (1, 2, 3, 4, 7, 8, 9, 12, 16, 24, 32, 33):
        lut = (rng.random((M, 256)) * 1e4).astype(np.float32)
        code = rng.integers(0, 256, M).astype(np.uint8)
        terms = [lut[m, code[m]] for m in range(M)]
        seq = _seq_sum_f32(terms)
        assert np.float32(refcpu.adc("seq", lut, code)) == seq
        # lanes8 == sequential when M <= 8 (one term per lane, lanes in order)
        if M <= 8:
            assert np.float32(refcpu.adc("lanes8", lut, code)) == seq
        # groups4 == sequential when M < 4 (all terms in the tail)
        if M < 4:
            assert np.float32(refcpu.adc("groups4", lut, code)) == seq
        # every order equals the exact sum within a few ulps
        exact = float(np.sum(np.asarray(terms, np.float64)))
        for o in ("lanes8", "groups4", "seq"):
            assert abs(refcpu.adc(o, lut, code) - exact) <= 4e-7 * M * exact


def test_adc_batch4_equals_lanes8():
    # batch_asymmetric_distance_avx2 (pq.rs:318-402) and
    # asymmetric_distance_simd_avx2 (pq.rs:435-485) share the lane order
    rng = np.random.default_rng(5)
    for M in (8, 16, 32, 12):
        luts = [(rng.random((M, 256)) * 100).astype(np.float32) for _ in range(4)]
        code = rng.integers(0, 256, M).astype(np.uint8)
        got = refcpu.adc_batch4(luts, code)
        for t in range(4):
            assert got[t] == np.float32(refcpu.adc("lanes8", luts[t], code))


def test_lut_closed_form():
    # table[m][j] = l2sq(r_m, cb[m][j]) (pq.rs:175-189); size M x 256 (pq.rs:1128-1144)
    rng = np.random.default_rng(2)
    M, dsub = 4, 3
    cb = rng.standard_normal((M, 256, dsub)).astype(np.float32)
    r = rng.standard_normal(M * dsub).astype(np.float32)
    lut = refcpu.pq_lut(cb, r)
    assert lut.shape == (M, 256)
    for m in range(M):
        for j in range(0, 256, 17):
            assert lut[m, j] == np.float32(refcpu.dist("l2sq", r[m * dsub:(m + 1) * dsub], cb[m, j]))
            exact = float(np.sum((r[m * dsub:(m + 1) * dsub].astype(np.float64) - cb[m, j]) ** 2))
            assert lut[m, j] == pytest.approx(exact, rel=1e-5, abs=1e-6)


def test_encode_is_first_argmin():
    # pq.rs:114-139: argmin with min_by keeping the first of equal minima
    rng = np.random.default_rng(9)
    M, dsub = 4, 2
    cb = rng.integers(-3, 4, (M, 256, dsub)).astype(np.float32)  # many exact ties
    for _ in range(50):
        x = rng.integers(-3, 4, M * dsub).astype(np.float32)
        code = refcpu.pq_encode(cb, x)
        for m in range(M):
            d = ((cb[m] - x[m * dsub:(m + 1) * dsub]) ** 2).sum(axis=1)
            assert code[m] == int(np.argmin(d))  # numpy argmin returns the first minimum


# ---- index-level checks --------------------------------------------------------
def _tiny_index(seed=0, n=3000, dim=16, nlist=8, M=4):
    from forgedb import datagen
    x = datagen.gaussian_mixture(seed + 100, seed + 200, n, dim, ncomp=16, centre_std=3.0)
    return x, refcpu.IvfPq.build(x, nlist=nlist, M=M, seed=seed)


def test_kmeans_find_nearest_centroids_kat():
    # kmeans.rs:381-395: centroids (0,0),(10,0),(5,10); query (0.1,0.1) -> 0 first
    cents = np.array([[0, 0], [10, 0], [5, 10]], np.float32)
    assert list(refcpu.ivf_probes(cents, [0.1, 0.1], 2))[0] == 0
    cb = np.zeros((1, 256, 2), np.float32)
    ix = refcpu.IvfPq.create(cents, cb, [0, 0, 0, 0], np.zeros(0, np.uint64), np.zeros((0, 1), np.uint8))
    lists, d = ix.probes([0.1, 0.1], 2)
    assert list(lists) == [0, 1]
    assert d[0] == np.float32(np.float32(0.1) ** 2 * 2)


def test_probe_selection_brute_force():
    x, ix = _tiny_index()
    art = ix.export()
    rng = np.random.default_rng(1)
    for _ in range(50):
        q = x[rng.integers(len(x))] + rng.standard_normal(x.shape[1]).astype(np.float32)
        for nprobe in (1, 3, 8):
            lists, d = ix.probes(q, nprobe)
            exact = ((art["centroids"].astype(np.float64) - q) ** 2).sum(axis=1)
            order = np.lexsort((np.arange(len(exact)), exact))
            assert set(lists) == set(order[:nprobe]) or np.isclose(
                exact[order[nprobe - 1]], exact[order[nprobe]], rtol=1e-6)
            assert np.all(np.diff(d) >= 0)


def test_nprobe_clamp():
    # ivf_pq.rs:2029-2042: set_nprobe(100) on 10 lists -> 10
    _, ix = _tiny_index(nlist=10)
    assert ix.nprobe() == 1  # ivf_pq.rs:501
    ix.set_nprobe(100)
    assert ix.nprobe() == 10


def test_search_returns_k_smallest_adc():
    # brute force over every code of the probed lists with the oracle's LUT
    x, ix = _tiny_index(seed=3)
    art = ix.export()
    ix.set_nprobe(3)
    off = art["list_offsets"].astype(np.int64)
    rng = np.random.default_rng(4)
    for _ in range(20):
        q = x[rng.integers(len(x))]
        ids, d = ix.search(q, 10)
        assert len(ids) == 10 and np.all(np.diff(d) >= 0)  # ivf_pq.rs:2023-2026
        lists, _ = ix.probes(q, 3)
        cand = []
        for p in lists:
            r = (q - art["centroids"][p]).astype(np.float32)
            lut = refcpu.pq_lut(art["codebooks"], r)
            for j in range(off[p], off[p + 1]):
                cand.append((refcpu.adc("groups4", lut, art["codes"][j]), int(art["ids"][j])))
        cand.sort()
        ok, msg = tie_aware_match(ids, d, [c[1] for c in cand[:10]], [c[0] for c in cand[:10]], rel=0)
        assert ok, msg


def test_batch_equals_single_at_full_nprobe():
    # ivf_pq.rs:2090-2121: at nprobe = nlist batch and single give the same ids
    x, ix = _tiny_index(seed=5)
    ix.set_nprobe(8)
    q = x[:40] + 0.5
    bi, bd, bc = ix.batch_search(q, 10)
    pi, pd, pc = ix.batch_search(q, 10, parallel=True, nthreads=4)
    assert np.array_equal(bi, pi) and np.array_equal(bd, pd) and np.array_equal(bc, pc)
    for t in range(len(q)):
        si, sd = ix.search(q[t], 10)
        ok, msg = tie_aware_match(si, sd, bi[t][:bc[t]], bd[t][:bc[t]])
        assert ok, msg


def test_batch_nprobe_zero_probes_one_list():
    # ivf_pq.rs:877-881 ([..=nth]) vs :546-552 (search probes none)
    x, ix = _tiny_index(seed=6)
    ix.set_nprobe(0)
    ids, d = ix.search(x[0], 5)
    assert len(ids) == 0
    bi, bd, bc = ix.batch_search(x[:3], 5)
    assert np.all(bc == 5)


def test_bf_remove_kat_equivalent():
    # brute_force.rs:434-455: rows [i;4] for i in 0..10 without id 5; query [5;4]
    data = np.array([[i] * 4 for i in range(10) if i != 5], np.float32)
    ids = np.array([i for i in range(10) if i != 5], np.uint64)
    oid, od = refcpu.bf_search(data, ids, EUC, [5.0] * 4, 10)
    assert 5 not in set(oid.tolist()) and len(oid) == 9
    assert od[0] == pytest.approx(2.0)


def test_bf_top1_is_argmin_and_parallel_matches():
    # tests/property.rs:176-201 and brute_force.rs:411-432
    rng = np.random.default_rng(8)
    data = rng.random((2500, 24)).astype(np.float32)
    ids = np.arange(2500, dtype=np.uint64)
    for m in (EUC, EUC2, COS, DOT, L1):
        q = rng.random(24).astype(np.float32)
        a_ids, a_d = refcpu.bf_search(data, ids, m, q, 7)
        p_ids, p_d = refcpu.bf_search(data, ids, m, q, 7, parallel=True)
        assert np.array_equal(a_d, p_d)
        every = np.array([refcpu.metric(m, q, r) for r in data], np.float32)
        assert a_d[0] == every.min() and int(a_ids[0]) == int(np.argmin(every))


def test_kmeans_converges_and_is_seeded():
    from forgedb import datagen
    x = datagen.gaussian_mixture(1, 2, 2000, 8, ncomp=5, centre_std=5.0)
    c1 = refcpu.kmeans_fit(x, 5, 25, seed=42)
    c2 = refcpu.kmeans_fit(x, 5, 25, seed=42)
    assert np.array_equal(c1, c2)
    # Stopped by the convergence rule (mean squared shift < 0.001,
    # kmeans.rs:74): one more Lloyd step moves every centroid only a little
    a = np.argmin(((x[:, None, :] - c1[None]) ** 2).sum(-1), axis=1)
    for k in range(5):
        if np.any(a == k):
            assert np.allclose(c1[k], x[a == k].mean(axis=0), atol=0.1)


def test_splitmix64_known_values():
    # SplitMix64 reference outputs for seed 0 (the first three of the
    # published sequence 0xe220a8397b1dcdaf, 0x6e789e6aa1b965f4, 0x06c45d188009454f)
    assert refcpu.lib().fdbo_splitmix64_at(0, 0) == 0xE220A8397B1DCDAF
    assert refcpu.lib().fdbo_splitmix64_at(0, 1) == 0x6E789E6AA1B965F4
    assert refcpu.lib().fdbo_splitmix64_at(0, 2) == 0x06C45D188009454F
    from forgedb import datagen
    assert [int(v) for v in datagen.splitmix64(0, 0, 3)] == [
        0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
    s = int(datagen.seeds(3)[0])
    assert int(datagen.splitmix64(s, 12345, 1)[0]) == refcpu.lib().fdbo_splitmix64_at(s, 12345)


# ---- IVF (full vectors) ------------------------------------------------------
def _small_ivf(seed=3, n=1500, dim=20, nlist=12):
    rng = np.random.default_rng(seed)
    x = (rng.random((n, dim)) * 4).astype(np.float32)
    cen, off, order = refcpu.ivf_build(x, nlist, seed=11)
    return x, cen, off, order


def test_ivf_build_is_kmeans_then_first_minimum_assignment():
    # ivf.rs:91-119: centroids = KMeans(n_clusters, 100).fit(all vectors);
    # each vector in the list of its first-minimum centroid, input order kept
    x, cen, off, order = _small_ivf()
    assert np.array_equal(cen, refcpu.kmeans_fit(x, 12, 100, refcpu.splitmix64_at(11, 1)))
    assert sorted(order.tolist()) == list(range(len(x)))
    for l in range(12):
        members = order[int(off[l]):int(off[l + 1])]
        assert np.all(np.diff(members.astype(np.int64)) > 0)
        for i in members[:40]:
            d = [refcpu.dist("l2sq", x[i], c) for c in cen]
            assert int(np.argmin(d)) == l  # np.argmin returns the first minimum


def test_ivf_search_is_brute_force_over_probed_lists():
    x, cen, off, order = _small_ivf()
    rows, ids = x[order], order.astype(np.uint64)
    rng = np.random.default_rng(5)
    for m in (EUC, EUC2, COS, DOT, L1):
        q = (rng.random(20) * 4).astype(np.float32)
        for nprobe in (0, 1, 3, 12):
            oi, od, oc = refcpu.ivf_batch_search(cen, off, ids, rows, m, nprobe, q[None], 9)
            probes = refcpu.ivf_probes(cen, q, nprobe)
            # stable sort of centroid distances (ivf.rs:164-177)
            cd = np.array([refcpu.dist("l2sq", q, c) for c in cen], np.float32)
            assert probes.tolist() == np.argsort(cd, kind="stable")[:nprobe].tolist()
            pos = [p for l in probes for p in range(int(off[l]), int(off[l + 1]))]
            d = np.array([refcpu.metric(m, q, rows[p]) for p in pos], np.float32)
            srt = sorted(range(len(pos)), key=lambda j: (d[j], pos[j]))[:9]
            assert int(oc[0]) == len(srt)
            assert np.array_equal(od[0, :len(srt)], d[srt])
            assert np.array_equal(oi[0, :len(srt)], ids[[pos[j] for j in srt]])


# ---- tombstones, insert, compact, filtered search (ivf_pq.rs:692-831, 1731-1851)
def _small_pq(seed=4):
    from forgedb import datagen
    base, queries = datagen.workload("ivfpq_int", n=3000, nq=12)
    ix = refcpu.IvfPq.build(base, nlist=16, M=16, seed=seed)
    return base, queries, ix


def _brute_adc(ix, q, allowed_pos, k):
    """k smallest groups-of-4 ADC over the given list positions, in
    (distance, position) order, as search() ranks them at nprobe = nlist."""
    art = ix.export()
    off = art["list_offsets"].astype(np.int64)
    lst = np.searchsorted(off, np.arange(len(art["ids"])), side="right") - 1
    luts = {}
    out = []
    for p in allowed_pos:
        l = int(lst[p])
        if l not in luts:
            luts[l] = refcpu.pq_lut(art["codebooks"], np.asarray(q, np.float32) - art["centroids"][l])
        out.append((refcpu.adc("groups4", luts[l], art["codes"][p]), p))
    out.sort()
    return [(int(art["ids"][p]), d) for d, p in out[:k]]


def test_search_skips_tombstones_and_matches_compaction():
    base, queries, ix = _small_pq()
    ix.set_nprobe(16)
    assert ix.delete(7) and not ix.delete(7) and ix.delete(100)
    assert ix.num_tombstones() == 2
    art = ix.export()
    live = [p for p in range(len(art["ids"])) if int(art["ids"][p]) not in (7, 100)]
    for q in queries[:4]:
        ids, d = ix.search(q, 10)
        want = _brute_adc(ix, q, live, 10)
        assert [int(i) for i in ids] == [i for i, _ in want]
        assert np.array_equal(d, np.array([x for _, x in want], np.float32))
    bi, bd, bc = ix.batch_search(queries, 10)
    ix.compact()
    assert ix.num_tombstones() == 0 and len(ix.export()["ids"]) == 2998
    ci, cd, cc = ix.batch_search(queries, 10)
    assert np.array_equal(bd, cd) and np.array_equal(bc, cc)
    assert 7 not in set(ci.ravel().tolist()) and 100 not in set(ci.ravel().tolist())


def test_insert_goes_to_nearest_list_with_residual_code():
    base, queries, ix = _small_pq()
    art0 = ix.export()
    new = (queries[:5] + 1.0).astype(np.float32)
    ix.insert(new, np.arange(90000, 90005, dtype=np.uint64))
    art = ix.export()
    for i in range(5):
        d = [refcpu.dist("l2sq", new[i], c) for c in art["centroids"]]
        l = int(np.argmin(d))  # first minimum
        s, e = int(art["list_offsets"][l]), int(art["list_offsets"][l + 1])
        pos = s + list(art["ids"][s:e]).index(90000 + i)
        assert np.array_equal(art["codes"][pos],
                              refcpu.pq_encode(art["codebooks"], new[i] - art["centroids"][l]))
    assert len(art["ids"]) == len(art0["ids"]) + 5


def test_search_filtered_is_brute_force_over_admitted_live_entries():
    base, queries, ix = _small_pq()
    ix.set_nprobe(16)
    art = ix.export()
    rng = np.random.default_rng(3)
    allowed = rng.choice(3000, 400, replace=False).astype(np.uint64)
    ix.delete(int(allowed[0]))
    aset = set(int(a) for a in allowed[1:])
    pos = [p for p in range(len(art["ids"])) if int(art["ids"][p]) in aset]
    for q in queries[:4]:
        ids, d = ix.search_filtered(q, 10, allowed)
        want = _brute_adc(ix, q, pos, 10)
        assert [int(i) for i in ids] == [i for i, _ in want]
        assert np.array_equal(d, np.array([x for _, x in want], np.float32))
    assert len(ix.search_filtered(queries[0], 10, np.array([], np.uint64))[0]) == 0
