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


# ---- independent models of the ADC sums, written from pq.rs ----------------------
def _lanes8_model(lut, code):
    """asymmetric_distance_simd_avx2 (pq.rs:435-485): lane l of an 8-wide f32
    accumulator adds table[m][code[m]] for m = l (mod 8) below 8*floor(M/8);
    the lanes are added left to right, then the tail m >= 8*floor(M/8) one
    by one.  Every add is one f32 rounding."""
    M = len(code)
    lanes = [np.float32(0.0)] * 8
    full = M // 8 * 8
    for i in range(0, full, 8):
        for l in range(8):
            lanes[l] = np.float32(lanes[l] + lut[i + l, code[i + l]])
    total = lanes[0]
    for l in range(1, 8):
        total = np.float32(total + lanes[l])
    for m in range(full, M):
        total = np.float32(total + lut[m, code[m]])
    return total


def _groups4_model(lut, code):
    """asymmetric_distance_fast (pq.rs:218-245): per group of 4 the value
    ((t0 + t1) + t2) + t3 is added to the running sum; the tail one by one."""
    M = len(code)
    s = np.float32(0.0)
    i = 0
    while i + 4 <= M:
        g = np.float32(lut[i, code[i]] + lut[i + 1, code[i + 1]])
        g = np.float32(g + lut[i + 2, code[i + 2]])
        g = np.float32(g + lut[i + 3, code[i + 3]])
        s = np.float32(s + g)
        i += 4
    while i < M:
        s = np.float32(s + lut[i, code[i]])
        i += 1
    return s


@pytest.mark.parametrize("M", [4, 8, 12, 16, 20, 24, 32, 40])
def test_adc_orders_match_independent_lane_models(M):
    # 8,000 random codes per M; tables with a wide dynamic range so that the
    # orders round differently.  A sequential sum in place of either order
    # (or a different grouping) fails: the test also requires that the
    # models differ from the sequential sum on a good share of the inputs.
    rng = np.random.default_rng(100 + M)
    lut = (rng.random((M, 256)) * 10.0 ** rng.integers(0, 5, (M, 256))).astype(np.float32)
    differ8 = differ4 = 0
    for _ in range(8000):
        code = rng.integers(0, 256, M).astype(np.uint8)
        seq = _seq_sum_f32(lut[m, code[m]] for m in range(M))
        m8, m4 = _lanes8_model(lut, code), _groups4_model(lut, code)
        assert np.float32(refcpu.adc("lanes8", lut, code)) == m8
        assert np.float32(refcpu.adc("groups4", lut, code)) == m4
        differ8 += m8 != seq
        differ4 += m4 != seq
    # below 16 terms each lane holds at most one term and the 8-lane order is
    # the sequential sum; below 8 terms so is the groups-of-4 order
    if M >= 16:
        assert differ8 > 800, differ8
    if M >= 8:
        assert differ4 > 400, differ4


@pytest.mark.parametrize("M", [8, 16, 32, 20])
def test_adc_batch4_matches_lane_model(M):
    # batch_asymmetric_distance_avx2 (pq.rs:318-402): per query the same
    # 8-lane accumulation; the lane array is folded with iter().sum() (from
    # zero, left to right), then the tail; queries beyond a multiple of 4 go
    # through asymmetric_distance_simd_avx2.  Both equal the lane model.
    rng = np.random.default_rng(7 + M)
    for _ in range(500):
        luts = [(rng.random((M, 256)) * 10.0 ** rng.integers(0, 4, (M, 256))).astype(np.float32)
                for _ in range(4)]
        code = rng.integers(0, 256, M).astype(np.uint8)
        got = refcpu.adc_batch4(luts, code)
        for t in range(4):
            assert got[t] == _lanes8_model(luts[t], code)


# ---- splitmix64 streams and the build's shuffles ---------------------------------
def _splitmix64(seed, i):
    m = (1 << 64) - 1
    z = (seed + (i + 1) * 0x9E3779B97F4A7C15) & m
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & m
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m
    return z ^ (z >> 31)


def test_shuffle_is_fisher_yates_from_the_back():
    # rand 0.8 SliceRandom::shuffle: for i = n..2, swap v[i-1] with v[j],
    # j uniform in [0, i); here j = (draw * i) >> 64 with the stream's next
    # 64-bit draw (splitmix64 output number 0, 1, 2, ...)
    for seed, n in ((5, 1), (5, 2), (123, 17), (0xF0DB0031, 1000)):
        v = list(range(n))
        draw = 0
        for i in range(n, 1, -1):
            j = (_splitmix64(seed, draw) * i) >> 64
            draw += 1
            v[i - 1], v[j] = v[j], v[i - 1]
        assert refcpu.shuffle_indices(seed, n).tolist() == v


# ---- IVFPQIndex::build composition (ivf_pq.rs:374-506) ---------------------------
def test_ivfpq_build_composition():
    """The build is: a 30k training sample (the first 30k of a shuffle) ->
    k-means with nlist clusters and 25 iterations (:383-400); every vector in
    the list of its first-minimum centroid, lists in input order (:403-414);
    a 100k residual sample (the first of another shuffle) -> per subspace
    k-means with 256 clusters (:422-446, pq.rs:60-105); every code the
    first-argmin encode of its vector's residual (:450-478).  Each step is
    recomputed here from the pinned primitives (shuffle, l2sq, encode) and
    the oracle's k-means."""
    from forgedb import datagen
    n, dim, nlist, M, seed = 31_000, 8, 6, 4, 9
    x = datagen.gaussian_mixture(seed + 1, seed + 2, n, dim, ncomp=12, centre_std=4.0)
    ix = refcpu.IvfPq.build(x, nlist=nlist, M=M, seed=seed)
    art = ix.export()
    cen = art["centroids"]
    # 1. coarse centroids from the first 30,000 of a shuffle
    sample = x[refcpu.shuffle_indices(refcpu.splitmix64_at(seed, 0), n)[:30_000].astype(np.int64)]
    assert np.array_equal(cen, refcpu.kmeans_fit(sample, nlist, 25, refcpu.splitmix64_at(seed, 1)))
    # 2. first-minimum assignment (l2sq in the reference order; numpy's
    # argmin returns the first minimum), lists in input order
    d = np.array([[refcpu.dist("l2sq", v, c) for c in cen] for v in x[:4000]], np.float32)
    want_list = np.argmin(d, axis=1)
    off = art["list_offsets"].astype(np.int64)
    pos_of = np.empty(n, np.int64)
    pos_of[art["ids"].astype(np.int64)] = np.arange(n)
    list_of = np.searchsorted(off, pos_of, side="right") - 1
    assert np.array_equal(list_of[:4000], want_list)
    for l in range(nlist):
        assert np.all(np.diff(art["ids"][off[l]:off[l + 1]].astype(np.int64)) > 0)
    # 3. codebooks from the residuals of the first 100,000 (here all n) of
    # a second shuffle, each subspace with its own seed
    idx = refcpu.shuffle_indices(refcpu.splitmix64_at(seed, 2), n).astype(np.int64)
    resid = (x[idx] - cen[list_of[idx]]).astype(np.float32)
    dsub = dim // M
    for m in range(M):
        sub = np.ascontiguousarray(resid[:, m * dsub:(m + 1) * dsub])
        want = refcpu.kmeans_fit(sub, 256, 25, refcpu.splitmix64_at(seed, 16 + m))
        assert np.array_equal(art["codebooks"][m], want), m
    # 4. codes = first-argmin encode of each residual
    for i in range(0, n, 97):
        r = (x[i] - cen[list_of[i]]).astype(np.float32)
        assert np.array_equal(art["codes"][pos_of[i]], refcpu.pq_encode(art["codebooks"], r))


# ---- rerank_results (ivf_pq.rs:555-582, 1022-1040) -------------------------------
def _rerank_model(q, pool_ids, originals_by_id, k):
    """filter_map over the ADC candidates in their ascending order: sqrt of the
    reference-order l2sq to the candidate's original vector (dropped when it
    has none), a stable ascending sort by that distance, truncated to k."""
    rr = []
    for i in pool_ids:
        v = originals_by_id.get(int(i))
        if v is None:
            continue
        rr.append((int(i), np.float32(np.sqrt(np.float32(refcpu.dist("l2sq", q, v))))))
    rr.sort(key=lambda t: t[1])  # Python's sort is stable
    return rr[:k]


def test_rerank_is_exact_sqrt_l2_over_the_adc_pool():
    from forgedb import datagen
    base, queries = datagen.workload("ivfpq_int", n=4000, nq=24)
    # duplicated rows: equal ADC distances and equal exact distances, so the
    # stable sort's order (the ADC order) is exercised
    base[3000:3200] = base[100:300]
    ix = refcpu.IvfPq.build(base, nlist=16, M=16, seed=2)
    art = ix.export()
    plain = refcpu.IvfPq.create(art["centroids"], art["codebooks"], art["list_offsets"],
                                art["ids"], art["codes"])
    rf, k = 4, 10
    ix.enable_reranking(base[art["ids"].astype(np.int64)], rf)
    orig = {int(i): base[int(i)] for i in art["ids"]}
    for nprobe in (1, 3, 16):
        ix.set_nprobe(nprobe)
        plain.set_nprobe(nprobe)
        qs = np.concatenate([queries, base[100:104] + 0.0])
        # search (:590-677): the pool is search()'s k*rf ADC best
        for q in qs:
            pool, _ = plain.search(q, k * rf)
            want = _rerank_model(q, pool, orig, k)
            gi, gd = ix.search(q, k)
            assert [int(i) for i in gi] == [i for i, _ in want]
            assert np.array_equal(gd, np.array([d for _, d in want], np.float32))
        # batch_search (:1022-1040): the pool is batch_search's k*rf best
        pi, _, pc = plain.batch_search(qs, k * rf)
        bi, bd, bc = ix.batch_search(qs, k)
        for t, q in enumerate(qs):
            want = _rerank_model(q, pi[t][:pc[t]], orig, k)
            assert int(bc[t]) == len(want)
            assert [int(i) for i in bi[t][:bc[t]]] == [i for i, _ in want]
            assert np.array_equal(bd[t][:bc[t]], np.array([d for _, d in want], np.float32))


# ---- brute-force top-k (brute_force.rs:105-157) -----------------------------------
@pytest.mark.parametrize("metric", [EUC, EUC2, COS, DOT, L1])
def test_bf_topk_is_full_sort_by_distance_then_row(metric):
    # scan_range keeps a row only when strictly closer than the heap's worst,
    # so among equal distances the earlier row wins; the result is the k
    # smallest (distance, row) pairs in ascending order.  Duplicated rows
    # make exact ties.
    rng = np.random.default_rng(40 + metric)
    data = rng.integers(0, 4, (1500, 12)).astype(np.float32)
    data[700:900] = data[0:200]
    ids = (np.arange(1500, dtype=np.uint64) * 7 + 3)
    for _ in range(6):
        q = rng.integers(0, 4, 12).astype(np.float32)
        every = [refcpu.metric(metric, q, r) for r in data]
        order = sorted(range(len(data)), key=lambda i: (every[i], i))
        for k in (1, 10, 57, 1500, 2000):
            oi, od = refcpu.bf_search(data, ids, metric, q, k)
            want = order[:k]
            assert oi.tolist() == [int(ids[i]) for i in want]
            assert np.array_equal(od, np.array([every[i] for i in want], np.float32))


def test_assignment_takes_the_first_of_twin_centroids():
    # ivf_pq.rs:403-414 and :1740-1747 (min_by keeps the first minimum):
    # with two identical centroids every vector nearest to them goes to the
    # lower list.  Random data almost never ties exactly, so twins are
    # planted; the same assignment routine serves build and insert.
    rng = np.random.default_rng(12)
    dim, M = 8, 4
    cen = rng.standard_normal((5, dim)).astype(np.float32) * 10
    cen[3] = cen[1]
    cb = rng.standard_normal((M, 256, dim // M)).astype(np.float32)
    ix = refcpu.IvfPq.create(cen, cb, np.zeros(6, np.uint64), np.zeros(0, np.uint64),
                             np.zeros((0, M), np.uint8))
    v = (cen[1] + rng.standard_normal((40, dim)) * 0.1).astype(np.float32)
    ix.insert(v, np.arange(40, dtype=np.uint64))
    off = ix.export()["list_offsets"].astype(np.int64)
    assert off[2] - off[1] == 40 and off[4] - off[3] == 0


def test_rerank_follows_original_vectors_by_id():
    """original_vectors is a map id -> vector (ivf_pq.rs:356): delete removes
    the id's vector (:1793-1797), insert_batch replaces it (:1769-1773), a
    loaded file holds whatever records were saved (:1918-1925); rerank_results
    drops candidates without one (filter_map, :562-571).  Duplicate ids make
    one map entry serve several list entries."""
    from forgedb import datagen
    base, queries = datagen.workload("ivfpq_int", n=3000, nq=8)
    base[2000:2100] = base[0:100]  # ids 2000..2099 duplicate the rows of 0..99
    ix = refcpu.IvfPq.build(base, nlist=8, M=16, seed=5)
    art = ix.export()
    # duplicate ids: list entries 0..99 of id 500..599 too
    ids = art["ids"].copy()
    ids[ids < 100] += 500
    plain = refcpu.IvfPq.create(art["centroids"], art["codebooks"], art["list_offsets"], ids, art["codes"])
    rr = refcpu.IvfPq.create(art["centroids"], art["codebooks"], art["list_offsets"], ids, art["codes"])
    rr.enable_reranking(base[art["ids"].astype(np.int64)], 3)
    for h in (plain, rr):
        h.set_nprobe(8)
    # the map after enable_reranking: the last vector of each id in list order
    orig = {}
    for p, i in enumerate(ids):
        orig[int(i)] = base[int(art["ids"][p])]
    k = 10

    def check(tag):
        for q in np.concatenate([queries, base[500:503], base[50:53]]):
            pool, _ = plain.search(q, k * 3)
            want = _rerank_model(q, pool, orig, k)
            gi, gd = rr.search(q, k)
            assert [int(i) for i in gi] == [i for i, _ in want], tag
            assert np.array_equal(gd, np.array([d for _, d in want], np.float32)), tag

    check("enable")
    # delete: one list entry tombstoned, the id's vector gone for all entries
    victim = int(ids[np.where(ids == 510)[0][0]])
    assert rr.delete(victim) and plain.delete(victim)
    del orig[victim]
    check("delete")
    # insert of an existing id: every entry of it reranks with the new vector
    newv = (base[520] + 3.0).astype(np.float32)
    rr.insert(newv[None], np.array([520], np.uint64))
    plain.insert(newv[None], np.array([520], np.uint64))
    orig[520] = newv
    check("insert")
    # a loaded file's records: only some ids have vectors
    keep = [i for i in sorted(orig) if i % 3]
    rr.set_originals(np.array(keep, np.uint64), np.stack([orig[i] for i in keep]), 3)
    orig = {i: orig[i] for i in keep}
    check("records")
