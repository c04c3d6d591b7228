"""The oracle (oracle/vdb_oracle.c) pinned before it is trusted as the GPU path's reference.

Three kinds of evidence per function:
  * golden vectors written by the reference's own code (tests/golden/make_golden.py);
  * the compiled reference itself on fresh random inputs (skipped where oracle/_ref is
    not built, e.g. on a box without the reference sources);
  * closed forms and invariants the mathematics fixes (sorting, brute force, half-step
    reconstruction, ADC == distance to the decoded vector, exhaustive IVF == flat).
"""
import os

import numpy as np
import pytest

from ivf_file import parse_ivfpq
from oracle_lib import KSET, METRIC

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def gold(name):
    return np.load(os.path.join(GOLD, name + ".npz"), allow_pickle=False)


def bits(x):
    return np.asarray(x, np.float32).view(np.uint32)


# ------------------------------------------------------------------ distances

def test_distance_kernels_match_golden_bit_patterns(oracle):
    g = gold("distances")
    L = oracle.lib
    for i, d in enumerate(g["dims"]):
        a, b = g["a"][i, :d].copy(), g["b"][i, :d].copy()
        c, vm, sc = g["codes"][i, :d].copy(), g["vmin"][i, :d].copy(), g["scale"][i, :d].copy()
        for ks in ["scalar", "avx2", "avx512"]:
            assert bits(L.or_l2(KSET[ks], a, b, d)) == bits(g[f"l2_{ks}"][i]), (ks, i, d)
            assert bits(L.or_dot(KSET[ks], a, b, d)) == bits(g[f"dot_{ks}"][i]), (ks, i, d)
            assert bits(L.or_sq8_l2(KSET[ks], a, c, vm, sc, d)) == bits(g[f"sq8l2_{ks}"][i])
            assert bits(L.or_sq8_ip(KSET[ks], a, c, vm, sc, d)) == bits(g[f"sq8ip_{ks}"][i])
        assert bits(L.or_l2sq_any(a, b, d - 3)) == bits(g["l2any"][i])
        assert bits(L.or_dot_any(a, b, d - 3)) == bits(g["dotany"][i])


def test_golden_distances_distinguish_summation_orders():
    # The fixtures are sensitive to the accumulation order: a restatement that used the
    # wrong order (scalar instead of AVX-512 tree, say) would fail the test above.
    g = gold("distances")
    assert (bits(g["l2_scalar"]) != bits(g["l2_avx512"])).sum() > 20
    assert (bits(g["l2_avx2"]) != bits(g["l2_avx512"])).sum() > 20
    assert (bits(g["sq8l2_scalar"]) != bits(g["sq8l2_avx512"])).sum() > 20


def test_distance_closed_forms(oracle):
    L = oracle.lib
    # metric convention (tests/distance_test.cc:86-91)
    a = np.zeros(16, np.float32)
    b = np.zeros(16, np.float32)
    a[0] = 1
    b[:2] = 0.5
    for ks in range(3):
        assert L.or_metric_dist(ks, 0, a, b, 16) == np.float32(0.5)
        assert L.or_metric_dist(ks, 1, a, b, 16) == np.float32(-0.5)
        assert L.or_metric_dist(ks, 2, a, b, 16) == np.float32(-0.5)
    # integer data: every order is exact, all kernel sets agree with numpy
    rng = np.random.default_rng(1)
    for d in [16, 48, 128]:
        x = rng.integers(0, 256, d).astype(np.float32)
        y = rng.integers(0, 256, d).astype(np.float32)
        want = np.float32(((x.astype(np.int64) - y.astype(np.int64)) ** 2).sum())
        for ks in range(3):
            assert L.or_l2(ks, x, y, d) == want
            assert L.or_dot(ks, x, y, d) == np.float32((x.astype(np.int64) * y).sum())


def test_distance_kernels_match_reference_random(oracle, reference):
    L, R = oracle.lib, reference.lib
    rng = np.random.default_rng(7)
    for d in [16, 32, 64, 96, 128, 384, 960]:
        for _ in range(30):
            a = rng.standard_normal(d).astype(np.float32)
            b = rng.standard_normal(d).astype(np.float32)
            c = rng.integers(0, 256, d).astype(np.uint8)
            vm = rng.standard_normal(d).astype(np.float32)
            sc = (np.abs(rng.standard_normal(d)) / 255).astype(np.float32)
            for ks in ["scalar", "avx2", "avx512"]:
                e = ks.encode()
                assert bits(L.or_l2(KSET[ks], a, b, d)) == bits(R.ref_l2(e, a, b, d))
                assert bits(L.or_dot(KSET[ks], a, b, d)) == bits(R.ref_dot(e, a, b, d))
                assert bits(L.or_sq8_l2(KSET[ks], a, c, vm, sc, d)) == bits(
                    R.ref_sq8_l2(e, a, c, vm, sc, d))
                assert bits(L.or_sq8_ip(KSET[ks], a, c, vm, sc, d)) == bits(
                    R.ref_sq8_ip(e, a, c, vm, sc, d))


# ------------------------------------------------------------------ top-k

def test_topk_matches_golden_and_sort(oracle):
    g = gold("topk")
    t = 0
    while f"d{t}" in g:
        d, i, k = g[f"d{t}"], g[f"i{t}"], int(g[f"k{t}"][0])
        od = np.empty(k, np.float32)
        oi = np.empty(k, np.uint32)
        m = oracle.lib.or_topk(d, i, len(d), k, od, oi)
        assert np.array_equal(od[:m], g[f"od{t}"]) and np.array_equal(oi[:m], g[f"oi{t}"])
        # closed form: lexicographic sort by (dist, id), first k
        order = np.lexsort((i, d))[:k]
        assert np.array_equal(oi[:m], i[order]) and np.array_equal(od[:m], d[order])
        t += 1
    assert t == 40


def test_topk_k_zero(oracle):
    d = np.ones(5, np.float32)
    i = np.arange(5, dtype=np.uint32)
    od = np.empty(1, np.float32)
    oi = np.empty(1, np.uint32)
    assert oracle.lib.or_topk(d, i, 5, 0, od, oi) == 0


# ------------------------------------------------------------------ flat

def test_flat_matches_golden(oracle):
    g = gold("flat")
    base, qs, allow = g["base"], g["queries"], g["allow"]
    for met in ["l2", "ip"]:
        for ks in ["scalar", "avx2", "avx512"]:
            od, oi = oracle.flat_search(base, qs, 10, metric=met, kset=ks)
            assert np.array_equal(oi, g[f"{met}_{ks}_i"]), (met, ks)
            assert np.array_equal(bits(od), bits(g[f"{met}_{ks}_d"])), (met, ks)
        od, oi = oracle.flat_search(base, qs, 10, metric=met, allow=allow)
        assert np.array_equal(oi, g[f"{met}_allow_i"])
        assert (oi % 3 == 0).all()
    od, oi = oracle.flat_search(base[:5], qs[:3], 8)
    assert np.array_equal(oi, g["small_i"]) and (oi[:, 5:] == 0xFFFFFFFF).all()


def test_flat_closed_form_integer_data(oracle):
    # integer data: the distance is exact in any order, so brute force with int64 fixes it
    rng = np.random.default_rng(5)
    base = rng.integers(0, 16, (4000, 32)).astype(np.float32)
    qs = rng.integers(0, 16, (20, 32)).astype(np.float32)
    od, oi = oracle.flat_search(base, qs, 25)
    d = ((qs[:, None, :].astype(np.int64) - base[None].astype(np.int64)) ** 2).sum(-1)
    for q in range(20):
        order = np.lexsort((np.arange(4000), d[q]))[:25]
        assert np.array_equal(oi[q], order)
        assert np.array_equal(od[q], d[q][order].astype(np.float32))


def test_flat_matches_reference_random(oracle, reference):
    rng = np.random.default_rng(9)
    base = rng.random((5000, 128), dtype=np.float32)
    qs = rng.random((30, 128), dtype=np.float32)
    for met in ["l2", "ip"]:
        od, oi = oracle.flat_search(base, qs, 20, metric=met)
        rd, ri = reference.flat_search(base, 128, qs, 20, metric=met)
        assert np.array_equal(oi, ri) and np.array_equal(bits(od), bits(rd))


# ------------------------------------------------------------------ SQ8

def test_sq8_matches_golden(oracle):
    g = gold("sq8")
    base, dim = g["base"], 100
    vmin, scale = oracle.sq8_train(base, dim)
    assert np.array_equal(bits(vmin), bits(g["vmin"])) and np.array_equal(bits(scale),
                                                                             bits(g["scale"]))
    codes = oracle.sq8_encode(base, dim, vmin, scale)
    assert np.array_equal(codes, g["codes"])
    assert (codes[:, 5] == 0).all() and (codes[:, dim:] == 0).all()
    for met in ["l2", "ip"]:
        od, oi = oracle.sq8_search(base, codes, vmin, scale, g["queries"], 10, 50, metric=met)
        assert np.array_equal(oi, g[f"{met}_i"]) and np.array_equal(bits(od), bits(g[f"{met}_d"]))


def test_sq8_reconstruction_within_half_step(oracle):
    # tests/distance_test.cc:106-126
    rng = np.random.default_rng(5)
    n, dim, pd = 2000, 100, 112
    base = np.zeros((n, pd), np.float32)
    base[:, :dim] = rng.normal(0, 3, (n, dim))
    vmin, scale = oracle.sq8_train(base, dim)
    assert np.array_equal(vmin[:dim], base[:, :dim].min(0))
    assert np.array_equal(scale[:dim], ((base[:, :dim].max(0) - vmin[:dim]) / np.float32(255)))
    codes = oracle.sq8_encode(base, dim, vmin, scale)
    back = vmin[None] + codes.astype(np.float32) * scale[None]
    err = np.abs(back[:, :dim] - base[:, :dim])
    assert (err <= scale[None, :dim] * 0.5 * 1.0001 + 1e-6).all()
    assert (back[:, dim:] == 0).all()
    # closed form of the encoder: IEEE divide, round half to even, clamp
    c = np.clip(np.rint((base[:, :dim] - vmin[None, :dim]) / scale[None, :dim]), 0, 255)
    assert np.array_equal(codes[:, :dim], c.astype(np.uint8))


def test_sq8_matches_reference_random(oracle, reference):
    rng = np.random.default_rng(11)
    base = rng.random((3000, 64), dtype=np.float32) * 10
    vmin = np.empty(64, np.float32)
    scale = np.empty(64, np.float32)
    codes = np.empty((3000, 64), np.uint8)
    reference.lib.ref_sq8_train_encode(base, 3000, 64, 64, vmin, scale, codes)
    v2, s2 = oracle.sq8_train(base, 64)
    assert np.array_equal(bits(v2), bits(vmin)) and np.array_equal(bits(s2), bits(scale))
    assert np.array_equal(oracle.sq8_encode(base, 64, v2, s2), codes)


# ------------------------------------------------------------------ PQ

def test_pq_matches_golden_and_adc_equals_decoded_distance(oracle):
    g = gold("pq")
    L = oracle.lib
    data, cen, m = g["data"], g["centroids"], 8
    dim = data.shape[1]
    dsub = dim // m
    codes = np.empty((len(data), m), np.uint8)
    for i in range(len(data)):
        L.or_pq_encode(cen, m, dsub, data[i], codes[i])
    assert np.array_equal(codes, g["codes"])
    cen3 = cen.reshape(m, 256, dsub)
    for met in ["l2", "ip"]:
        for qi in range(4):
            t = np.empty(m * 256, np.float32)
            L.or_pq_compute_table(cen, m, dsub, g["queries"][qi], METRIC[met], t)
            assert np.array_equal(bits(t), bits(g[f"table_{met}"][qi]))
            for j in range(50):
                a = L.or_pq_adc(t, m, codes[j])
                assert bits(a) == bits(g[f"adc_{met}"][qi][j])
                dec = np.concatenate([cen3[s, codes[j, s]] for s in range(m)]).astype(np.float32)
                q = g["queries"][qi]
                exact = (L.or_l2sq_any(q, dec, dim) if met == "l2"
                         else -L.or_dot_any(q, dec, dim))
                assert abs(a - exact) <= 1e-3 * max(1.0, abs(exact))  # pq_test.cc:64-83


def test_pq_encode_is_first_argmin(oracle):
    # closed form: strict < keeps the lowest centroid index among equal distances
    m, dsub = 2, 4
    cen = np.zeros((m, 256, dsub), np.float32)
    cen[:, :, 0] = np.arange(256) % 7  # many centroids at equal distance
    x = np.full(m * dsub, 3.0, np.float32)
    x[1::dsub] = 0
    code = np.empty(m, np.uint8)
    oracle.lib.or_pq_encode(np.ascontiguousarray(cen.ravel()), m, dsub, x, code)
    assert list(code) == [3, 3]


# ------------------------------------------------------------------ assignment

def test_assign_nearest_matches_golden(oracle):
    g = gold("kmeans")
    data, cen = g["data"], g["centroids_pp"]
    asg = np.empty(len(data), np.uint32)
    dist = np.empty(len(data), np.float32)
    oracle.lib.or_assign_nearest(2, data, len(data), 16, 16, cen, 40, asg, dist, 4)
    assert np.array_equal(asg, g["assign"]) and np.array_equal(bits(dist), bits(g["dist"]))
    # brute force: argmin with ties to the lowest index
    d = ((data[:, None, :] - cen.reshape(40, 16)[None]) ** 2).sum(-1)
    close = np.abs(d.min(1) - d[np.arange(len(data)), asg]) <= 1e-4 * d.min(1) + 1e-6
    assert close.all()


# ------------------------------------------------------------------ IVF-PQ

def _ivf_search(oracle, ix, base, qs, k, nprobe, rerank, kset="avx512", metric="l2"):
    nq = len(qs)
    od = np.empty((nq, k), np.float32)
    oi = np.empty((nq, k), np.uint32)
    dc = np.empty(nq, np.uint64)
    term2 = None
    if metric == "l2":  # precompute_tables keeps term2 for L2 only (ivf_pq.cc:152-167)
        term2 = np.empty(ix["nlist"] * ix["m"] * 256, np.float32)
        dsub = ix["dim"] // ix["m"]
        oracle.lib.or_ivfpq_term2(ix["coarse"], ix["nlist"], ix["pd"], ix["pq_centroids"],
                                  ix["m"], dsub, term2)
    oracle.lib.or_ivfpq_search_batch(KSET[kset], METRIC[metric], base, ix["dim"], ix["pd"], ix["coarse"],
                                     ix["nlist"], ix["pq_centroids"], ix["m"], ix["list_off"],
                                     ix["list_ids"], ix["list_codes"], term2, qs, nq, k,
                                     nprobe, rerank, None, od, oi, dc, 4)
    return od, oi, dc


def test_ivfpq_matches_golden(oracle):
    g = gold("ivfpq")
    ix = parse_ivfpq(g["index_file"])
    assert oracle.lib.or_crc32c(0, ix["crc_covered"], len(ix["crc_covered"])) == ix["crc"]
    assert int(ix["list_off"][-1]) == len(g["base"])
    for nprobe, rr in [(1, 0), (4, 0), (4, -1), (24, 0), (24, 5000)]:
        tag = f"np{nprobe}_r{rr if rr >= 0 else 'auto'}"
        od, oi, dc = _ivf_search(oracle, ix, g["base"], g["queries"], 10, nprobe, rr)
        assert np.array_equal(oi, g[f"{tag}_i"]), tag
        assert np.array_equal(bits(od), bits(g[f"{tag}_d"])), tag
        assert np.array_equal(dc, g[f"{tag}_dc"]), tag


def test_ivfpq_exhaustive_rerank_equals_flat(oracle):
    # nprobe = nlist and rerank >= n: every row is re-ranked exactly, so IVF-PQ == flat
    g = gold("ivfpq")
    ix = parse_ivfpq(g["index_file"])
    od, oi, _ = _ivf_search(oracle, ix, g["base"], g["queries"], 10, ix["nlist"], 5000)
    fd, fi = oracle.flat_search(g["base"], g["queries"], 10)
    assert np.array_equal(oi, fi) and np.array_equal(bits(od), bits(fd))


def test_ivfpq_matches_reference_random(oracle, reference):
    rng = np.random.default_rng(13)
    base = (rng.random((6000, 32), dtype=np.float32) * 4).astype(np.float32)
    qs = rng.random((20, 32), dtype=np.float32) * 4
    blob = reference.ivfpq_build(base, 32, nlist=32, m=8, seed=3, max_points=64)
    ix = parse_ivfpq(blob)
    for nprobe, rr in [(3, 0), (8, -1)]:
        od, oi, dc = _ivf_search(oracle, ix, base, qs, 10, nprobe, rr)
        rd = np.empty((20, 10), np.float32)
        ri = np.empty((20, 10), np.uint32)
        rdc = np.empty(20, np.uint64)
        assert reference.lib.ref_ivfpq_search_batch(0, blob, len(blob), base, 6000, 32, 32, qs,
                                                    20, 10, nprobe, rr, None, rd, ri, rdc,
                                                    1) == 0
        assert np.array_equal(oi, ri) and np.array_equal(bits(od), bits(rd))
        assert np.array_equal(dc, rdc)


# ------------------------------------------------------------------ misc

def test_normalize_matches_golden(oracle):
    g = gold("misc")
    for i in range(len(g["norm_in"])):
        v = g["norm_in"][i].copy()
        ok = oracle.lib.or_normalize(v, len(v))
        assert ok == g["norm_ok"][i]
        if ok:
            assert np.array_equal(bits(v), bits(g["norm_out"][i]))
            assert abs(np.linalg.norm(v.astype(np.float64)) - 1) < 1e-6


def test_crc32c_known_answers(oracle):
    g = gold("misc")
    L = oracle.lib
    assert L.or_crc32c(0, b"123456789", 9) == 0xE3069283  # tests/distance_test.cc:94
    assert L.or_crc32c(0, b"", 0) == 0
    blob = g["crc_blob"].tobytes()
    assert L.or_crc32c(0, blob, len(blob)) == g["crc"][2]
    # Extend(Value(a), b) == Value(a + b)
    assert L.or_crc32c(L.or_crc32c(0, blob[:123], 123), blob[123:], len(blob) - 123) == g["crc"][2]


def test_merge_parts_closed_form(oracle):
    # collection_impl.cc:1076-1112: sort by (dist, part, row), first occurrence of each
    # external id, stop at k
    k = 4
    part_d = np.array([[1, 2, 5, np.inf], [1, 2, 3, 4], [0.5, 2, 2, 9]], np.float32)
    part_r = np.array([[0, 1, 2, 0xFFFFFFFF], [0, 1, 2, 3], [0, 1, 2, 3]], np.uint32)
    ext = np.array([10, 11, 12, 20, 21, 22, 23, 11, 30, 31, 32], np.uint64)
    off = np.array([0, 3, 7], np.uint64)
    od = np.empty(k, np.float32)
    oe = np.empty(k, np.uint64)
    n = oracle.lib.or_merge_parts(3, k, part_d.ravel().copy(), part_r.ravel().copy(), ext, off,
                                  od, oe)
    # candidates: (0.5,p2,r0)=11 (1,p0,r0)=10 (1,p1,r0)=20 (2,p0,r1)=11 dup (2,p1,r1)=21 ...
    assert n == 4
    assert list(oe) == [11, 10, 20, 21]
    assert list(od) == [0.5, 1, 1, 2]


def test_filtered_collection_search_matches_reference(oracle, reference):
    # the oracle's pieces (pad + NormalizeVector, per-segment filtered exact scan, merge)
    # composed as CollectionImpl::Search composes them, against the reference's kernels,
    # TopK and NormalizeVector driven by the planner's loop
    from vdbg import datagen

    dim, k = 40, 10
    pd = 48
    rng = np.random.default_rng(5)
    sizes = [700, 1500, 64, 900]
    segs, allows, exts = [], [], []
    for i, n in enumerate(sizes):
        segs.append(datagen.pad(datagen.clustered_unit(n, dim, 10 + i, 9, 20, 0.4), pd))
        a = rng.random(n) < [0.05, 0.5, 1.0, 0.0][i]
        w = np.zeros((n + 63) // 64, np.uint64)
        rows = np.nonzero(a)[0]
        np.bitwise_or.at(w, rows // 64, np.uint64(1) << (rows % 64).astype(np.uint64))
        allows.append(w)
        exts.append(rng.permutation(10 ** 6)[:n].astype(np.uint64))
    exts[1][:30] = exts[0][:30]  # the same external id in two segments
    ext = np.concatenate(exts)
    raw = datagen.clustered_unit(50, dim, 99, 9, 20, 0.4) * 2.5
    re, rd = reference.filtered_collection_search(segs, dim, allows, ext, raw, k)
    # oracle composition
    q = np.zeros((50, pd), np.float32)
    q[:, :dim] = raw
    for i in range(50):
        assert oracle.lib.or_normalize(q[i], dim) == 1
    nseg = len(segs)
    pdist = np.empty((nseg, 50, k), np.float32)
    prow = np.empty((nseg, 50, k), np.uint32)
    for p in range(nseg):
        pdist[p], prow[p] = oracle.flat_search(segs[p], q, k, metric="cosine", allow=allows[p])
    off = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.uint64)
    for i in range(50):
        od = np.empty(k, np.float32)
        oe = np.empty(k, np.uint64)
        n = oracle.lib.or_merge_parts(nseg, k, np.ascontiguousarray(pdist[:, i]),
                                      np.ascontiguousarray(prow[:, i]), ext, off, od, oe)
        assert list(re[i, :n]) == list(oe[:n])
        assert np.array_equal(rd[i, :n].view(np.uint32), od[:n].view(np.uint32))
        assert (re[i, n:] == np.iinfo(np.uint64).max).all()


def test_plan_segment_known_answers(oracle):
    # SearchDiskSegment's choice (src/engine/planner.cc:53-108) at the edges of its cost
    # model, worked by hand from the formulas: selectivity s = matches / live rows; exact when
    # matches <= prefilter_threshold, or matches <= 10 * max(ef, k) / s, or the index is flat;
    # an Auto filtered index search probes max(nprobe, ceil(nprobe / s)) lists.
    import ctypes as C
    L = oracle.lib
    npb = C.c_size_t()

    def plan(has_filter, rows, deleted, matches, flat=0, strategy=0, ef=64, k=10, nprobe=16,
             threshold=10000):
        p = L.or_plan_segment(has_filter, rows, deleted, matches, flat, strategy, ef, k, nprobe,
                              threshold, C.byref(npb))
        return p, npb.value

    assert plan(0, 100000, 500, 0) == (0, 16)            # no filter: the index
    assert plan(1, 100000, 0, 0) == (1, 16)              # nothing matches: empty
    assert plan(1, 100000, 0, 10000) == (2, 16)          # at the threshold: exact
    assert plan(1, 100000, 0, 10001) == (3, 160)         # s = .10001: cost 6399 < 10001
    assert plan(1, 100000, 0, 50000) == (3, 32)          # s = .5: 16 / .5 probes
    assert plan(1, 100000, 0, 50000, flat=1) == (2, 16)  # a flat index always scans exactly
    assert plan(1, 100000, 50000, 50000) == (3, 16)      # deletes raise s to 1: no boost
    # cost model: 2000 matches of 10,000 live (s = .2) cost 10 * 64 / .2 = 3200 > 2000
    assert plan(1, 10000, 0, 2000, threshold=100) == (2, 16)
    assert plan(1, 10000, 0, 2000, threshold=100, ef=10) == (3, 80)  # 10 * 10 / .2 = 500
    assert plan(1, 100000, 0, 50000, strategy=1) == (2, 16)   # PreFilter
    assert plan(1, 100000, 0, 50000, strategy=2) == (3, 16)   # Graph: no boost when explicit
    assert plan(1, 100000, 0, 50000, strategy=3) == (5, 16)   # PostFilter
    assert plan(1, 100000, 0, 0, strategy=3) == (1, 16)       # empty wins over the strategy


# ------------------------------------------------------------------ HNSW-SQ8 search

METRICS = ["l2", "ip", "cosine"]


def hnsw_case(g, tag):
    rows = np.ascontiguousarray(g[f"{tag}_rows"], np.float32)
    return (rows, g[f"{tag}_q"], METRICS[int(g[f"{tag}_metric"])], int(g[f"{tag}_dim"]),
            g[f"{tag}_file"].tobytes())


def test_hnsw_sq8_matches_golden(oracle):
    """HnswSq8Index::search results recorded from the reference (graph beam on SQ8 codes,
    then Rerank): ids, distances and distance computations, every setting and filter."""
    g = gold("hnsw")
    ks = str(g["kernels"])
    for tag in ("c", "d", "e"):
        rows, q, metric, dim, f = hnsw_case(g, tag)
        for fi in range(4):
            allow = g[f"{tag}_allow{fi}"] if fi else None
            for si, (k, ef, rr) in enumerate(g["settings"]):
                od, oi, dc = oracle.hnsw_sq8_search(f, rows, q, int(k), int(ef), int(rr),
                                                    metric=metric, allow=allow, kset=ks)
                key = f"{tag}_f{fi}_s{si}"
                assert np.array_equal(oi, g[key + "_i"]), key
                assert np.array_equal(bits(od), bits(g[key + "_d"])), key
                assert np.array_equal(dc, g[key + "_dc"]), key


def test_hnsw_sq8_golden_exercises_every_branch():
    """The recorded cases reach the parts of the walk a slip would change: the upper-layer
    descent (several layers), short results under a sparse filter, depth 0 (no rerank) and
    rerank depths below, at and above k."""
    g = gold("hnsw")
    for tag in ("c", "d", "e"):
        f = g[f"{tag}_file"].tobytes()
        n = int.from_bytes(f[8:16], "little")
        pd = int.from_bytes(f[20:24], "little")
        off = 8 + 8 + 8 + 8 * pd + n * pd + 16 + 8 + 8
        assert int.from_bytes(f[off:off + 4], "little") >= 2, tag  # max level
        short = g[f"{tag}_f3_s5_i"]  # about 2 % of the rows allowed, k = 60
        assert (short == 0xFFFFFFFF).any(), tag
    assert {int(s[2]) for s in g["settings"]} >= {-1, 0, 3, 100}


def test_hnsw_sq8_beam_over_every_node_equals_flat(oracle):
    """Closed form: with ef at least the row count the beam never fills, so it visits every
    node reachable from the entry point (all of them: vdb repairs connectivity after the
    build), and rerank depth max(ef, k) re-scores them all: exact flat search."""
    g = gold("segment")
    for tag in ("a", "b"):
        rows = g[f"{tag}_rows"]
        n, pd = rows.shape
        metric = ["l2", "ip", "cosine"][int(g[f"{tag}_metric"])]
        rng = np.random.default_rng(3)
        q = np.zeros((20, pd), np.float32)
        q[:, :int(g[f"{tag}_dim"])] = rng.uniform(-3, 5, (20, int(g[f"{tag}_dim"])))
        f = g[f"{tag}_file"].tobytes()
        for k in (1, 10, 33):
            od, oi, dc = oracle.hnsw_sq8_search(f, rows, q, k, n, -1, metric=metric)
            fd, fi = oracle.flat_search(rows, q, k, metric=metric)
            assert np.array_equal(oi, fi) and np.array_equal(bits(od), bits(fd)), (tag, k)
            assert (dc >= n + n).all()  # every node scored by the walk, then reranked


def test_hnsw_sq8_matches_reference_random(oracle, reference):
    g = gold("segment")
    rng = np.random.default_rng(11)
    for tag in ("a", "b"):
        rows = g[f"{tag}_rows"]
        n, pd = rows.shape
        dim = int(g[f"{tag}_dim"])
        metric = ["l2", "ip", "cosine"][int(g[f"{tag}_metric"])]
        f = g[f"{tag}_file"].tobytes()
        q = np.zeros((30, pd), np.float32)
        q[:, :dim] = rng.uniform(-3, 5, (30, dim))
        for k, ef, rr in ((10, 64, -1), (7, 12, 0), (15, 20, 50), (3, 5, 2)):
            for frac in (None, 0.4):
                allow = None
                if frac is not None:
                    a = rng.random(n) < frac
                    w = np.zeros(((n + 63) // 64) * 8, np.uint8)
                    b = np.packbits(a, bitorder="little")
                    w[:b.size] = b
                    allow = w.view(np.uint64)
                rd, ri, rdc = reference.hnsw_sq8_search(f, rows, dim, q, k, ef, rr, metric, allow)
                od, oi, dc = oracle.hnsw_sq8_search(f, rows, q, k, ef, rr, metric=metric,
                                                    allow=allow,
                                                    kset=reference.lib.ref_best_kernels().decode())
                assert np.array_equal(oi, ri) and np.array_equal(bits(od), bits(rd))
                assert np.array_equal(dc, rdc)


# ------------------------------------------------------------------ PQ-flat search

def test_pqflat_matches_golden(oracle):
    from ivf_file import parse_pqflat
    g = gold("pqflat")
    ks = str(g["kernels"])
    for tag in ("a", "b", "c"):
        ix = parse_pqflat(g[f"{tag}_file"].tobytes())
        rows, q, metric = g[f"{tag}_rows"], g[f"{tag}_q"], str(g[f"{tag}_metric"])
        for fi, allow in enumerate((None, g[f"{tag}_allow"])):
            for si, (k, rr) in enumerate(g["settings"]):
                od, oi, dc = oracle.pqflat_search(ix, rows, q, int(k), int(rr), metric, allow,
                                                  kset=ks)
                key = f"{tag}_f{fi}_s{si}"
                assert np.array_equal(oi, g[key + "_i"]), key
                assert np.array_equal(bits(od), bits(g[key + "_d"])), key
                assert np.array_equal(dc, g[key + "_dc"]), key


def test_pqflat_full_rerank_equals_flat(oracle):
    """Closed form: a rerank depth of at least the row count re-scores every row exactly."""
    from ivf_file import parse_pqflat
    g = gold("pqflat")
    for tag in ("a", "b", "c"):
        ix = parse_pqflat(g[f"{tag}_file"].tobytes())
        rows, q, metric = g[f"{tag}_rows"], g[f"{tag}_q"], str(g[f"{tag}_metric"])
        n = rows.shape[0]
        od, oi, dc = oracle.pqflat_search(ix, rows, q, 10, n, metric)
        fd, fi = oracle.flat_search(rows, q, 10, metric=metric)
        assert np.array_equal(oi, fi) and np.array_equal(bits(od), bits(fd)), tag
        assert (dc == 2 * n).all()


def test_pqflat_matches_reference_random(oracle, reference):
    from ivf_file import parse_pqflat
    rng = np.random.default_rng(21)
    for n, dim, m, metric in ((900, 32, 8, "l2"), (700, 20, 5, "ip")):
        pd = (dim + 15) // 16 * 16
        base = np.zeros((n, pd), np.float32)
        base[:, :dim] = rng.uniform(-2, 3, (n, dim))
        f = reference.pqflat_file(base, dim, m, metric, seed=7)
        ix = parse_pqflat(f)
        q = np.zeros((20, pd), np.float32)
        q[:, :dim] = rng.uniform(-2, 3, (20, dim))
        for k, rr in ((10, -1), (4, 0), (12, 30)):
            rd, ri, rdc = reference.pqflat_search(f, base, dim, q, k, rr, metric)
            od, oi, dc = oracle.pqflat_search(ix, base, q, k, rr, metric,
                                              kset=reference.lib.ref_best_kernels().decode())
            assert np.array_equal(oi, ri) and np.array_equal(bits(od), bits(rd))
            assert np.array_equal(dc, rdc)


# ------------------------------------------------------------------ IVF-PQ shapes

def ivf_shape_case(g, tag):
    import sys
    sys.path.insert(0, GOLD)
    from make_golden import ivf_shape_rows
    n, dim, m, nlist, seed = (int(v) for v in g[f"{tag}_shape"])
    return ivf_shape_rows(n, dim, seed), ivf_shape_rows(20, dim, seed + 100), dim, m, nlist


def test_ivfpq_shapes_match_golden(oracle):
    """m = 64 and 48 (one- and two-dim sub-vectors) and m = 2 over 136 dims (68-dim
    sub-vectors): the oracle's IVF-PQ search equals the reference's on indexes it built."""
    g = gold("ivf_shapes")
    for tag in ("w", "x", "y"):
        base, q, dim, m, nlist = ivf_shape_case(g, tag)
        metric = str(g[f"{tag}_metric"])
        ix = parse_ivfpq(g[f"{tag}_file"].tobytes())
        assert ix["m"] == m and ix["dim"] == dim and ix["nlist"] == nlist
        for si, (nprobe, rr) in enumerate(g["settings"]):
            od, oi, dc = _ivf_search(oracle, ix, base, q, 10, int(nprobe), int(rr), metric=metric)
            key = f"{tag}_s{si}"
            assert np.array_equal(oi, g[key + "_i"]), key
            assert np.array_equal(bits(od), bits(g[key + "_d"])), key
            assert np.array_equal(dc, g[key + "_dc"]), key
