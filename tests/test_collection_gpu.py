"""The collection read path in one batch (vdbg_collection_search_host) against the oracle's
composition of the same steps: CollectionImpl::SearchBatch / Search
(src/engine/collection_impl.cc:1023-1135), SearchDiskSegment's plan per segment
(src/engine/planner.cc:42-129) over flat, SQ8 and IVF-PQ segments with deletes and filters,
and the merge by (dist, part, row) with one hit per external id.  External ids, distances,
distance computations and the plan chosen for every segment must all agree."""
import numpy as np
import pytest

import vdbg
from ivf_file import parse_ivfpq, synth_ivfpq
from vdbg import datagen

pytestmark = pytest.mark.gpu

DIM = 64
FAR = 6000  # rows of the IVF-PQ segment in the far cluster


def _mask(n, frac, seed):
    bits = np.random.default_rng(seed).random(n) < frac
    w = np.zeros((n + 63) // 64, np.uint64)
    r = np.nonzero(bits)[0]
    np.bitwise_or.at(w, r // 64, np.uint64(1) << (r % 64).astype(np.uint64))
    return w


def _words(rows, n):
    w = np.zeros((n + 63) // 64, np.uint64)
    r = np.asarray(rows, np.int64)
    np.bitwise_or.at(w, r // 64, np.uint64(1) << (r % 64).astype(np.uint64))
    return w


@pytest.fixture(scope="module")
def coll(ctx, oracle):
    """Four segments: flat (deletes), SQ8 codes made on the GPU (this library's SQ8 scan index,
    no graph), IVF-PQ (deletes), a small flat one that re-inserts external ids of the first (an
    upsert visible in both)."""
    pd = vdbg.padded_dim(DIM)
    sizes = [6000, 8000, 20000, 500]
    kinds = ["flat", "sq8", "ivf", "flat"]
    segs, handles = [], []
    next_id = 1000
    for i, (n, kind) in enumerate(zip(sizes, kinds)):
        x = datagen.uniform_rows(n, DIM, 700 + i) * 10
        if kind == "ivf":
            x[:FAR] += 50.0  # a far cluster of 30 % of the rows, spread over ~10 lists
        base = datagen.pad(x, pd)
        ext = (np.arange(next_id, next_id + n, dtype=np.uint64) * 3)
        next_id += n
        if i == 3:
            ext[:100] = segs[0]["ext"][:100]
        ds = vdbg.Dataset(ctx, base, DIM)
        ds.set_external_ids(ext)
        sg = {"base": base, "ext": ext, "kind": kind}
        ix = None
        if kind == "sq8":
            ix = vdbg.Sq8Index(ds)
            sg.update(codes=ix.codes(), vmin=ix.vmin, scale=ix.scale)
        elif kind == "ivf":
            blob = synth_ivfpq(base, DIM, 32, 8, seed=3)
            ix = vdbg.IvfPqIndex.load(ds, blob)
            p = parse_ivfpq(blob)
            t2 = np.empty(p["nlist"] * p["m"] * 256, np.float32)
            oracle.lib.or_ivfpq_term2(p["coarse"], p["nlist"], p["pd"], p["pq_centroids"],
                                      p["m"], p["dim"] // p["m"], t2)
            sg.update(ix=p, term2=t2)
        deleted = _mask(n, 0.03, 800 + i) if i in (0, 2) else None
        sg["deleted"] = deleted
        segs.append(sg)
        handles.append((ds, ix))
    yield segs, handles
    for ds, ix in handles:
        if ix is not None:
            ix.close()
        ds.close()


def _run(ctx, oracle, coll, filters, raw, k, metric="l2", **kw):
    segs, handles = coll
    for sg, f in zip(segs, filters):
        sg["filter"] = f
    params = vdbg.SearchParams(**kw)
    gi, gd, gdc, gplans = vdbg.collection_search(
        ctx, [(ds, ix, sg["deleted"], sg["filter"]) for (ds, ix), sg in zip(handles, segs)],
        DIM, metric, raw, k, params)
    okw = dict(kw)
    okw["strategy"] = vdbg.STRATEGIES[okw.get("strategy", "auto")]
    oi, od, odc, oplans = oracle.collection_search(segs, DIM, metric, raw, k, **okw)
    assert gplans == oplans
    bad = np.nonzero((gi != oi).any(axis=1) | (gd.view(np.uint32) != od.view(np.uint32)).any(axis=1))[0]
    assert bad.size == 0, (bad[:5], gi[bad[0]], oi[bad[0]], gd[bad[0]], od[bad[0]])
    assert np.array_equal(gdc, odc)
    return gplans


def _queries(n, seed):
    return (datagen.uniform_rows(n, DIM, seed) * 10).astype(np.float32)


@pytest.mark.parametrize("k", [1, 10, 100])
def test_no_filter_every_index_type(ctx, oracle, coll, k):
    print(f"collection no filter k={k}", flush=True)
    plans = _run(ctx, oracle, coll, [None] * 4, _queries(40, 901), k, nprobe=8)
    assert plans == ["index"] * 4


def test_filter_planned_per_segment(ctx, oracle, coll):
    # 50 % of every segment: flat segments scan exactly, the SQ8 and IVF-PQ segments search
    # their index under the filter (nprobe raised to 16 / 0.5 = 32)
    print("collection filter 50%", flush=True)
    n = [sg["base"].shape[0] for sg in coll[0]]
    filt = [_mask(m, 0.5, 810 + i) for i, m in enumerate(n)]
    plans = _run(ctx, oracle, coll, filt, _queries(32, 902), 10, prefilter_threshold=1000)
    assert plans == ["prefilter_exact", "filtered_index", "filtered_index", "prefilter_exact"]
    # the default threshold (10,000 matches) keeps everything exact
    plans = _run(ctx, oracle, coll, filt, _queries(32, 903), 10)
    assert plans == ["prefilter_exact"] * 4


def test_filtered_ivf_falls_back_to_exact(ctx, oracle, coll):
    # only the far cluster (30 % of the IVF-PQ segment) is allowed: nprobe 2 / 0.3 = 7 probes
    # of the lists nearest each query find none of it, so every query takes the exact scan
    # of the allowed rows (planner.cc:103-108)
    print("collection ivf exact fallback", flush=True)
    segs = coll[0]
    filt = [None, None, _words(np.arange(FAR), segs[2]["base"].shape[0]), None]
    plans = _run(ctx, oracle, coll, filt, _queries(24, 904), 10, ef=1, nprobe=2,
                 prefilter_threshold=100)
    assert plans == ["index", "index", "filtered_index+exact_fallback", "index"]


@pytest.mark.parametrize("strategy", ["prefilter", "graph", "post_filter"])
def test_explicit_strategies(ctx, oracle, coll, strategy):
    print(f"collection strategy={strategy}", flush=True)
    n = [sg["base"].shape[0] for sg in coll[0]]
    filt = [_mask(m, 0.3, 820 + i) for i, m in enumerate(n)]
    plans = _run(ctx, oracle, coll, filt, _queries(20, 905), 10, strategy=strategy,
                 post_filter_alpha=3, nprobe=4)
    want = {"prefilter": "prefilter_exact", "graph": "filtered_index",
            "post_filter": "post_filter"}[strategy]
    assert plans == [want] * 4


def test_empty_segment_filter(ctx, oracle, coll):
    n = [sg["base"].shape[0] for sg in coll[0]]
    filt = [np.zeros((m + 63) // 64, np.uint64) for m in n]
    filt[1] = _mask(n[1], 0.01, 830)
    plans = _run(ctx, oracle, coll, filt, _queries(10, 906), 10)
    assert plans == ["empty", "prefilter_exact", "empty", "empty"]


def test_cosine_collection(ctx, oracle):
    # cosine: queries normalised once (PrepareQuery), unit rows, flat and SQ8 segments
    pd = vdbg.padded_dim(96)
    segs, handles = [], []
    for i, (n, kind) in enumerate([(5000, "flat"), (7000, "sq8")]):
        base = datagen.pad(datagen.clustered_unit(n, 96, 840 + i, 79, 40, 0.5), pd)
        ext = np.arange(n, dtype=np.uint64) + 100000 * (i + 1)
        ds = vdbg.Dataset(ctx, base, 96, metric="cosine")
        ds.set_external_ids(ext)
        sg = {"base": base, "ext": ext, "kind": kind, "deleted": _mask(n, 0.02, 850 + i),
              "filter": None}
        ix = None
        if kind == "sq8":
            ix = vdbg.Sq8Index(ds)
            sg.update(codes=ix.codes(), vmin=ix.vmin, scale=ix.scale)
        segs.append(sg)
        handles.append((ds, ix))
    raw = datagen.clustered_unit(30, 96, 860, 79, 40, 0.5) * 2.5
    gi, gd, gdc, gp = vdbg.collection_search(
        ctx, [(ds, ix, sg["deleted"], None) for (ds, ix), sg in zip(handles, segs)], 96, "cosine",
        raw, 10)
    oi, od, odc, op = oracle.collection_search(segs, 96, "cosine", raw, 10)
    assert gp == op == ["index", "index"]
    assert np.array_equal(gi, oi) and np.array_equal(gd.view(np.uint32), od.view(np.uint32))
    assert np.array_equal(gdc, odc)
    for ds, ix in handles:
        if ix is not None:
            ix.close()
        ds.close()


def test_collection_errors(ctx, coll):
    segs, handles = coll
    args = [(ds, ix, sg["deleted"], None) for (ds, ix), sg in zip(handles, segs)]
    q = _queries(4, 907)
    for k in (0, 10001):
        with pytest.raises(vdbg.VdbgError) as e:
            vdbg.collection_search(ctx, args, DIM, "l2", q, k)
        assert e.value.code == 1 and "k must be in 1..10000" in str(e.value)
    bad = q.copy()
    bad[2, 5] = np.nan
    with pytest.raises(vdbg.VdbgError) as e:
        vdbg.collection_search(ctx, args, DIM, "l2", bad, 10)
    assert e.value.code == 1 and "NaN or infinite" in str(e.value)
    ds = vdbg.Dataset(ctx, segs[0]["base"][:100], DIM)  # no external ids
    with pytest.raises(vdbg.VdbgError) as e:
        vdbg.collection_search(ctx, [(ds, None, None, None)], DIM, "l2", q, 10)
    assert e.value.code == 6
    with pytest.raises(vdbg.VdbgError) as e:
        vdbg.collection_search(ctx, args, DIM, "ip", q, 10)
    assert e.value.code == 1
    ds.close()
    # no segments: every query gets padding
    gi, gd, gdc, gp = vdbg.collection_search(ctx, [], DIM, "l2", q, 5)
    assert (gi == np.iinfo(np.uint64).max).all() and np.isinf(gd).all() and gp == []


def test_hnsw_sq8_segment_is_the_references(ctx, oracle):
    """An HnswSq8Index segment (a VDBHSQ81 file the reference built and saved) inside the
    one-batch collection search: its graph is walked and its beam reranked, so the answer is
    HnswSq8Index::search's.  Alone in a collection it must return exactly what the reference's
    own search returned on that file (tests/golden/hnsw.npz), with no filter and under a
    DeleteFilter; mixed with flat segments, filters and every strategy, the oracle's
    composition (whose HNSW search the same fixtures pin)."""
    import os
    g = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "hnsw.npz"))
    ctx.set_kernels(str(g["kernels"]))
    rows = np.ascontiguousarray(g["c_rows"], np.float32)
    q, f, dim = g["c_q"], g["c_file"].tobytes(), int(g["c_dim"])
    n, pd = rows.shape
    assert list(g["settings"][0]) == [10, 64, -1]  # SearchParams' defaults, k = 10
    ds = vdbg.Dataset(ctx, rows, dim)
    ext = np.arange(n, dtype=np.uint64) * 7 + 5
    ds.set_external_ids(ext)
    sq = vdbg.Sq8Index.load(ds, f)
    print(f"collection hnsw-sq8 segment n={n} dim={dim}", flush=True)
    # alone, no filter: the "index" plan, HnswSq8Index::search with the default params
    gi, gd, gdc, gp = vdbg.collection_search(ctx, [(ds, sq, None, None)], dim, "l2", q, 10)
    want = g["c_f0_s0_i"]
    assert gp == ["index"]
    assert np.array_equal(gi, np.where(want == 0xFFFFFFFF, np.iinfo(np.uint64).max,
                                       ext[np.minimum(want, n - 1)]))
    assert np.array_equal(gd.view(np.uint32), g["c_f0_s0_d"].view(np.uint32))
    assert np.array_equal(gdc, g["c_f0_s0_dc"])
    # alone, the rows outside the ~98 % filter deleted: the DeleteFilter of planner.cc:56-61
    deleted = ~np.asarray(g["c_allow1"], np.uint64)
    gi, gd, gdc, gp = vdbg.collection_search(ctx, [(ds, sq, deleted, None)], dim, "l2", q, 10)
    want = g["c_f1_s0_i"]
    assert gp == ["index"]
    assert np.array_equal(gi, np.where(want == 0xFFFFFFFF, np.iinfo(np.uint64).max,
                                       ext[np.minimum(want, n - 1)]))
    assert np.array_equal(gd.view(np.uint32), g["c_f1_s0_d"].view(np.uint32))
    assert np.array_equal(gdc, g["c_f1_s0_dc"])
    # with two flat segments, deletes and filters, against the oracle's composition
    segs = [{"base": rows, "ext": ext, "kind": "hnsw_sq8", "file": f,
             "deleted": _mask(n, 0.05, 870), "filter": None}]
    handles = [(ds, sq)]
    for i, m in enumerate((3000, 800)):
        b = np.clip(np.rint(rows[np.random.default_rng(880 + i).integers(0, n, m)] +
                            np.random.default_rng(890 + i).normal(0, 3, (m, pd))), 0, 255)
        b = np.ascontiguousarray(b * (np.arange(pd) < dim), np.float32)
        e = np.arange(m, dtype=np.uint64) + 10 ** 6 * (i + 1)
        if i == 1:
            e[:50] = ext[:50]  # an upsert seen in both segments
        d2 = vdbg.Dataset(ctx, b, dim)
        d2.set_external_ids(e)
        segs.append({"base": b, "ext": e, "kind": "flat", "deleted": None, "filter": None})
        handles.append((d2, None))
    qq = q[:24]
    try:
        for filt, kw in ((None, {}), ("f", {"prefilter_threshold": 100}),
                         ("f", {"strategy": "graph"}), ("f", {"strategy": "post_filter",
                                                              "post_filter_alpha": 4}),
                         (None, {"ef": 16, "rerank": 0}), (None, {"ef": 8, "rerank": 30})):
            for i, sg in enumerate(segs):
                sg["filter"] = None if filt is None else _mask(sg["base"].shape[0], 0.4, 900 + i)
            k = 10
            gi, gd, gdc, gplans = vdbg.collection_search(
                ctx, [(d_, ix, sg["deleted"], sg["filter"]) for (d_, ix), sg in zip(handles, segs)],
                dim, "l2", qq, k, vdbg.SearchParams(**kw))
            okw = dict(kw)
            okw["strategy"] = vdbg.STRATEGIES[okw.get("strategy", "auto")]
            oi, od, odc, oplans = oracle.collection_search(segs, dim, "l2", qq, k,
                                                           kset=str(g["kernels"]), **okw)
            assert gplans == oplans, (filt, kw)
            assert np.array_equal(gi, oi) and np.array_equal(gd.view(np.uint32), od.view(np.uint32)), (filt, kw)
            assert np.array_equal(gdc, odc), (filt, kw)
    finally:
        sq.close()
        for d_, _ in handles:
            d_.close()


def test_pqflat_segment(ctx, oracle):
    """A PQ-flat segment (VDBPQFL1, built on the GPU) next to a flat one, with deletes,
    filters and the planner's strategies, against the oracle's composition."""
    from ivf_file import parse_pqflat
    dim = 32
    pd = vdbg.padded_dim(dim)
    segs, handles = [], []
    for i, (n, kind) in enumerate([(6000, "pqflat"), (2500, "flat")]):
        base = datagen.pad(datagen.uniform_rows(n, dim, 930 + i) * 10, pd)
        ext = np.arange(n, dtype=np.uint64) * 11 + 100000 * (i + 1)
        ds = vdbg.Dataset(ctx, base, dim)
        ds.set_external_ids(ext)
        sg = {"base": base, "ext": ext, "kind": kind, "deleted": _mask(n, 0.03, 940 + i),
              "filter": None}
        ix = None
        if kind == "pqflat":
            ix = vdbg.PqFlatIndex.build(ds, 8, seed=5)
            sg["pq"] = parse_pqflat(ix.save())
        segs.append(sg)
        handles.append((ds, ix))
    print("collection pq-flat segment", flush=True)
    raw = _queries(20, 950)[:, :dim].copy()
    try:
        for filt, kw in ((None, {}), (None, {"rerank": 0}), ("f", {"prefilter_threshold": 500}),
                         ("f", {"strategy": "post_filter", "post_filter_alpha": 3}),
                         (None, {"rerank": 40})):
            for i, sg in enumerate(segs):
                sg["filter"] = None if filt is None else _mask(sg["base"].shape[0], 0.5, 960 + i)
            gi, gd, gdc, gp = vdbg.collection_search(
                ctx, [(d_, ix, sg["deleted"], sg["filter"]) for (d_, ix), sg in zip(handles, segs)],
                dim, "l2", raw, 10, vdbg.SearchParams(**kw))
            okw = dict(kw)
            okw["strategy"] = vdbg.STRATEGIES[okw.get("strategy", "auto")]
            oi, od, odc, op = oracle.collection_search(segs, dim, "l2", raw, 10, **okw)
            assert gp == op, (filt, kw)
            assert np.array_equal(gi, oi) and np.array_equal(gd.view(np.uint32), od.view(np.uint32)), (filt, kw)
            assert np.array_equal(gdc, odc), (filt, kw)
    finally:
        for d_, ix in handles:
            if ix is not None:
                ix.close()
            d_.close()


# ---------------------------------------------------------------- a segment searched on the host

def _hnswf():
    """vdb's default index type: a float-row HNSW segment (VDBHNSW1) the reference built, and
    its own HnswIndex::search results recorded on it (tests/golden/hnswf.npz), keyed as the
    oracle's segment_hits looks them up: (k, ef, allowed words)."""
    import os
    import sys
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
    from make_golden import HNSWF_EF, hnswf_allows, hnswf_inputs
    z = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "hnswf.npz"))
    rows, raw, deleted, filters = hnswf_inputs()
    assert np.array_equal(deleted, z["deleted"])
    for name, w in filters.items():
        assert np.array_equal(w, z[name])
    allows = hnswf_allows(deleted, filters)
    recorded = {}
    for i, (k, name) in enumerate(zip(z["keys_k"], z["keys_allow"])):
        k = int(k)
        recorded[(k, max(HNSWF_EF, k), allows[str(name)].tobytes())] = (
            z[f"r{i}_d"], z[f"r{i}_i"], z[f"r{i}_dc"])
    return rows, raw, deleted, filters, recorded, HNSWF_EF


def test_host_searched_hnsw_segment(ctx, oracle):
    """vdb's default index type (IndexType::Hnsw, options.h:22) keeps its graph search on the
    CPU: its segment has no GPU copy, and vdb's own SearchDiskSegment result for it (here the
    reference's recorded HnswIndex::search calls, composed by the planner's rules) joins the
    device batch as a host part, in its snapshot position between device-searched flat and
    IVF-PQ segments with deletes and filters.  External ids (one hit per id, an id shared
    with the HNSW segment included), distances, distance computations and plans must equal the
    oracle's composition of the whole collection."""
    rows_h, raw, del_h, filt_h, recorded, ef = _hnswf()
    dim = rows_h.shape[1]
    nh = rows_h.shape[0]
    ext_h = np.arange(nh, dtype=np.uint64) * 7 + 5
    segs, handles = [], []
    for i, (n, kind) in enumerate([(5000, "flat"), (None, "hnsw"), (9000, "ivf"), (800, "flat")]):
        if kind == "hnsw":
            segs.append({"base": rows_h, "ext": ext_h, "kind": "hnsw", "recorded": recorded,
                         "deleted": del_h})
            handles.append(None)
            continue
        base = datagen.pad(datagen.uniform_rows(n, dim, 1720 + i) * 10, dim)
        ext = np.arange(n, dtype=np.uint64) * 7 + 6 + 100000 * i
        if i == 3:
            ext[:50] = ext_h[:50]  # upserted rows of the HNSW segment
        ds = vdbg.Dataset(ctx, base, dim)
        ds.set_external_ids(ext)
        sg = {"base": base, "ext": ext, "kind": kind, "deleted": _mask(n, 0.03, 1730 + i)}
        ix = None
        if kind == "ivf":
            blob = synth_ivfpq(base, dim, 24, 8, seed=5)
            ix = vdbg.IvfPqIndex.load(ds, blob)
            p = parse_ivfpq(blob)
            t2 = np.empty(p["nlist"] * p["m"] * 256, np.float32)
            oracle.lib.or_ivfpq_term2(p["coarse"], p["nlist"], p["pd"], p["pq_centroids"],
                                      p["m"], p["dim"] // p["m"], t2)
            sg.update(ix=p, term2=t2)
        segs.append(sg)
        handles.append((ds, ix))
    q = np.zeros((raw.shape[0], dim), np.float32)
    q[:, :raw.shape[1]] = raw  # L2: the prepared query is the raw one (64 dims)
    cases = [(None, {}), ("f50", {"prefilter_threshold": 100}),
             ("f01", {"strategy": "graph"}), ("f10", {"strategy": "graph"}),
             ("f50", {"strategy": "graph"}), ("f10", {"strategy": "post_filter"}),
             ("f10", {})]
    try:
        for fname, kw in cases:
            for i, sg in enumerate(segs):
                if sg["kind"] == "hnsw":
                    sg["filter"] = None if fname is None else filt_h[fname]
                else:
                    n = sg["base"].shape[0]
                    sg["filter"] = None if fname is None else _mask(n, {"f01": .01, "f10": .1, "f50": .5}[fname], 1740 + i)
            for k in (1, 10, 40):
                print(f"host-searched HNSW segment: filter {fname} {kw} k={k}", flush=True)
                okw = dict(kw, ef=ef)
                okw["strategy"] = vdbg.STRATEGIES[okw.get("strategy", "auto")]
                # the host part: vdb's SearchDiskSegment on the HNSW segment
                hd, hr, hdc, hplan = oracle.segment_hits(segs[1], "l2", q, k, **okw)
                hext = np.where(hr == 0xFFFFFFFF, np.uint64(0), ext_h[np.minimum(hr, nh - 1)])
                host = vdbg.HostHits(hd, hr, hext, hdc)
                parts = []
                for sg, h in zip(segs, handles):
                    if h is None:
                        parts.append(host)
                    else:
                        parts.append((h[0], h[1], sg["deleted"], sg["filter"]))
                gi, gd, gdc, gp = vdbg.collection_search(
                    ctx, parts, dim, "l2", raw, k, vdbg.SearchParams(ef=ef, **kw))
                oi, od, odc, op = oracle.collection_search(segs, dim, "l2", raw, k, **okw)
                assert gp[1] == "host" and gp[0] == op[0] and gp[2:] == op[2:], (gp, op)
                assert np.array_equal(gi, oi), (fname, kw, k)
                assert np.array_equal(gd.view(np.uint32), od.view(np.uint32)), (fname, kw, k)
                assert np.array_equal(gdc, odc), (fname, kw, k)
                if fname == "f50" and kw.get("prefilter_threshold") == 100:
                    assert hplan == "filtered_index", hplan  # the HNSW walk under the filter
    finally:
        for h in handles:
            if h is not None:
                if h[1] is not None:
                    h[1].close()
                h[0].close()


def test_host_part_rejects_unsorted_hits(ctx):
    """A host part's lists must be in ascending (dist, row) order, as Index::search returns
    them: the device merge keeps that order as the (dist, part, row) tie rule."""
    d = np.array([[1.0, 0.5, np.inf]], np.float32)
    r = np.array([[3, 4, 0xFFFFFFFF]], np.uint32)
    e = np.array([[30, 40, 0]], np.uint64)
    raw = np.zeros((1, 16), np.float32)
    with pytest.raises(vdbg.VdbgError) as ex:
        vdbg.collection_search(ctx, [vdbg.HostHits(d, r, e)], 16, "l2", raw, 3)
    assert ex.value.code == 1
    d2 = np.array([[0.5, 1.0, np.inf]], np.float32)
    gi, gd, gdc, gp = vdbg.collection_search(ctx, [vdbg.HostHits(d2, r, e, [9])], 16, "l2", raw, 3)
    assert gp == ["host"] and list(gi[0]) == [30, 40, 2**64 - 1] and gdc[0] == 9


def test_device_entry_equals_host_entry(ctx, oracle, coll):
    """vdbg_collection_search_device (raw queries and results in device memory, the segments'
    flat scans on the call's lanes) returns what vdbg_collection_search_host returns: ids,
    distances, distance computations and plans, with and without filters."""
    import torch

    segs, handles = coll
    dev = torch.device("cuda:0")
    for fkind in (None, 0.5, 0.02):
        n = [sg["base"].shape[0] for sg in segs]
        filt = [None if fkind is None else _mask(m, fkind, 1800 + i) for i, m in enumerate(n)]
        parts = [(ds, ix, sg["deleted"], f) for (ds, ix), sg, f in zip(handles, segs, filt)]
        raw = _queries(37, 1810)
        for k in (1, 10, 100):
            print(f"collection device entry filter={fkind} k={k}", flush=True)
            hi, hd, hdc, hp = vdbg.collection_search(ctx, parts, DIM, "l2", raw, k,
                                                     vdbg.SearchParams(nprobe=8))
            q = torch.from_numpy(raw).to(dev)
            oi = torch.empty((37, k), dtype=torch.int64, device=dev)
            od = torch.empty((37, k), dtype=torch.float32, device=dev)
            ddc, dp = vdbg.collection_search_device(
                ctx, parts, DIM, "l2", q.data_ptr(), 37, k, oi.data_ptr(), od.data_ptr(),
                vdbg.SearchParams(nprobe=8), stream=torch.cuda.current_stream().cuda_stream)
            torch.cuda.synchronize()
            assert dp == hp
            assert np.array_equal(oi.cpu().numpy().view(np.uint64), hi)
            assert np.array_equal(od.cpu().numpy().view(np.uint32), hd.view(np.uint32))
            assert np.array_equal(ddc, hdc)


@pytest.mark.parametrize("metric,memory", [("l2", False), ("cosine", False), ("l2", True)])
def test_collection_schedules_agree(ctx, oracle, metric, memory):
    """Flat segments (deletes, filters from 0.5 % to 60 %, an external id held by two segments,
    optionally an in-memory part first) searched under every schedule of the collection
    search: one combined scan of all allowed rows (taken when no part is an in-memory one,
    whose appended ids are not checked for uniqueness), segments side by side on threaded
    lanes, on unthreaded lanes, and in turn.  Every schedule returns the oracle's composition
    of vdb's per-segment searches and merge."""
    dim = 48
    pd = vdbg.padded_dim(dim)
    sizes = [(1200, memory), (9000, False), (7000, False), (20000, False), (3000, False)]
    segs, handles = [], []
    for i, (n, in_memory) in enumerate(sizes):
        x = datagen.uniform_rows(n, dim, 1900 + i) * (3 if metric == "l2" else 1)
        if metric == "cosine":
            x = x - np.float32(0.5)
        base = datagen.pad(x, pd)
        if metric == "cosine":
            base = base / np.linalg.norm(base, axis=1, keepdims=True).astype(np.float32)
        ext = np.arange(n, dtype=np.uint64) * 5 + 100000 * i
        if i == 4:
            ext[:40] = segs[1]["ext"][:40]  # upserted rows of segment 1
        if in_memory:
            ds = vdbg.Dataset.appendable(ctx, dim, metric, capacity=512)
            ds.append(base, ext)
        else:
            ds = vdbg.Dataset(ctx, base, dim, metric=metric)
            ds.set_external_ids(ext)
        segs.append({"base": base, "ext": ext, "kind": "memory" if in_memory else "flat",
                     "deleted": _mask(n, 0.02, 1910 + i)})
        handles.append(ds)
    raw = (datagen.uniform_rows(33, dim, 1920) * 3).astype(np.float32)
    if metric == "cosine":
        raw = raw - np.float32(0.5)
    schedules = [(True, 4, True), (False, 4, True), (False, 3, False), (False, 0, False)]
    try:
        for frac in (None, 0.005, 0.05, 0.6):
            for i, sg in enumerate(segs):
                sg["filter"] = None if frac is None else _mask(sg["base"].shape[0], frac, 1930 + i)
            for k in (1, 10, 25):
                oi, od, odc, op = oracle.collection_search(segs, dim, metric, raw, k)
                for combine, lanes, threaded in schedules:
                    print(f"schedules {metric} filter={frac} k={k} combine={combine} "
                          f"lanes={lanes} threaded={threaded}", flush=True)
                    ctx.set_collection_schedule(combine, lanes, threaded)
                    ctx.profile(True)
                    ctx.profile_reset()
                    gi, gd, gdc, gp = vdbg.collection_search(
                        ctx, [(ds, None, sg["deleted"], sg["filter"], sg["kind"] == "memory")
                              for ds, sg in zip(handles, segs)], dim, metric, raw, k)
                    if combine and not memory:  # one gather of every segment's rows
                        assert ctx.profile_get("compact")[1] == 1
                    ctx.profile(False)
                    assert gp == op, (frac, k, combine, lanes)
                    assert np.array_equal(gi, oi), (frac, k, combine, lanes)
                    assert np.array_equal(gd.view(np.uint32), od.view(np.uint32)), (frac, k, combine, lanes)
                    assert np.array_equal(gdc, odc), (frac, k, combine, lanes)
    finally:
        ctx.set_collection_schedule(True, 2, True)
        for ds in handles:
            ds.close()


def test_combined_scan_over_many_segments(ctx, oracle):
    """Twenty flat segments (more than one launch's sixteen: the masks compact and the rows
    gather in two rounds of launches), filters of 1 % and 20 % on some segments and none on
    others, deletes on all: the one combined scan (k x segments <= 240) returns the oracle's
    composition of vdb's per-segment searches and merge, and so do the lanes past it."""
    dim = 32
    pd = vdbg.padded_dim(dim)
    nseg = 20
    segs, handles = [], []
    for i in range(nseg):
        n = 1500 + 97 * i
        base = datagen.pad(datagen.uniform_rows(n, dim, 2100 + i) * 4, pd)
        ext = np.arange(n, dtype=np.uint64) * 3 + 50000 * i
        ds = vdbg.Dataset(ctx, base, dim)
        ds.set_external_ids(ext)
        frac = None if i % 5 == 3 else (0.01 if i % 2 == 0 else 0.2)
        segs.append({"base": base, "ext": ext, "kind": "flat",
                     "deleted": _mask(n, 0.03, 2140 + i),
                     "filter": None if frac is None else _mask(n, frac, 2160 + i)})
        handles.append(ds)
    raw = (datagen.uniform_rows(40, dim, 2190) * 4).astype(np.float32)
    try:
        ctx.set_collection_schedule(True, 2, True)
        for k in (1, 10, 30):
            print(f"many segments k={k}", flush=True)
            oi, od, odc, op = oracle.collection_search(segs, dim, "l2", raw, k)
            ctx.profile(True)
            ctx.profile_reset()
            gi, gd, gdc, gp = vdbg.collection_search(
                ctx, [(ds, None, sg["deleted"], sg["filter"], False)
                      for ds, sg in zip(handles, segs)], dim, "l2", raw, k)
            if k * nseg <= 240:
                assert ctx.profile_get("compact")[1] == 1  # the combined scan's one gather
            else:
                assert ctx.profile_get("compact")[1] > 1  # the segments' own compactions
            ctx.profile(False)
            assert gp == op, k
            assert np.array_equal(gi, oi), k
            assert np.array_equal(gd.view(np.uint32), od.view(np.uint32)), k
            assert np.array_equal(gdc, odc), k
    finally:
        ctx.profile(False)
        for ds in handles:
            ds.close()
