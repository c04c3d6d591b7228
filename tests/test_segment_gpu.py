"""The collection-level read path on the GPU: filtered scans over one segment (delete and
filter masks, src/engine/planner.cc:31-38 and :64-65), PrepareQuery / NormalizeVector
(src/engine/collection_impl.cc:1023-1034, src/util/dataset.cc:33-41) and the cross-segment
merge of CollectionImpl::Search (collection_impl.cc:1076-1112), each against the oracle:
ids, external ids and distances bit-exact."""
import numpy as np
import pytest

import vdbg
from vdbg import datagen

pytestmark = pytest.mark.gpu


def _mask(n, frac, seed):
    rng = np.random.default_rng(seed)
    rows = np.nonzero(rng.random(n) < frac)[0]
    allow = np.zeros((n + 63) // 64, np.uint64)
    np.bitwise_or.at(allow, rows // 64, np.uint64(1) << (rows % 64).astype(np.uint64))
    return allow, rows


def _same(gi, gd, oi, od):
    assert gi.shape == oi.shape
    bad = np.nonzero((gi != oi).any(axis=1) |
                     (gd.view(np.uint32) != od.view(np.uint32)).any(axis=1))[0]
    assert bad.size == 0, (f"{bad.size} queries differ; q={bad[0]} gpu={gi[bad[0]].tolist()} "
                           f"oracle={oi[bad[0]].tolist()}")


@pytest.mark.parametrize("frac", [0.001, 0.01, 0.1, 0.45, 0.6, 0.98])
def test_flat_filter_selectivity(ctx, oracle, frac):
    # at most half allowed -> compacted rows; above -> per-row mask in the scan
    n, nq, k = 40000, 96, 10
    print(f"flat filter frac={frac}", flush=True)
    base = datagen.uniform_rows(n, 128, 31)
    qs = datagen.uniform_rows(nq, 128, 32)
    allow, rows = _mask(n, frac, 33)
    ds = vdbg.Dataset(ctx, base, 128)
    gi, gd = ds.flat_search(qs, k, allow=allow)
    od, oi = oracle.flat_search(base, qs, k, allow=allow)
    _same(gi, gd, oi, od)
    real = gi[gi != vdbg.NO_ID]
    assert np.isin(real, rows).all()


def test_flat_filter_cosine_384(ctx, oracle):
    # unit rows of 384 dims under cosine with 2% deleted and 10% passing a filter
    n, nq, k = 30000, 64, 10
    base = datagen.clustered_unit(n, 384, 41, 40, 100, 0.5)
    qs = datagen.clustered_unit(nq, 384, 42, 40, 100, 0.5)
    allow, _ = _mask(n, 0.1, 43)
    deleted, _ = _mask(n, 0.02, 44)
    allow &= ~deleted
    ds = vdbg.Dataset(ctx, base, 384, metric="cosine")
    gi, gd = ds.flat_search(qs, k, allow=allow)
    od, oi = oracle.flat_search(base, qs, k, metric="cosine", allow=allow)
    _same(gi, gd, oi, od)


def test_flat_filter_fewer_than_k(ctx, oracle):
    n = 20000
    base = datagen.uniform_rows(n, 64, 51)
    qs = datagen.uniform_rows(40, 64, 52)
    allow = np.zeros((n + 63) // 64, np.uint64)
    for r in (5, 700, 19999):
        allow[r // 64] |= np.uint64(1) << np.uint64(r % 64)
    ds = vdbg.Dataset(ctx, base, 64)
    gi, gd = ds.flat_search(qs, 10, allow=allow)
    od, oi = oracle.flat_search(base, qs, 10, allow=allow)
    _same(gi, gd, oi, od)
    assert (gi[:, 3:] == vdbg.NO_ID).all() and np.isinf(gd[:, 3:]).all()


def test_flat_filter_none_allowed(ctx):
    n = 5000
    base = datagen.uniform_rows(n, 32, 61)
    ds = vdbg.Dataset(ctx, base, 32)
    gi, gd = ds.flat_search(base[:50], 7, allow=np.zeros((n + 63) // 64, np.uint64))
    assert (gi == vdbg.NO_ID).all() and np.isinf(gd).all()


@pytest.mark.parametrize("frac,depth", [(0.02, 40), (0.3, 0)])
def test_sq8_filter_selectivity(ctx, oracle, frac, depth):
    n, nq, k = 30000, 64, 10
    base = datagen.sift_like(n, 128, 71)
    qs = datagen.sift_like(nq, 128, 72)
    allow, _ = _mask(n, frac, 73)
    ds = vdbg.Dataset(ctx, base, 128)
    sq = vdbg.Sq8Index(ds)
    gi, gd = sq.search(qs, k, depth, allow=allow)
    od, oi = oracle.sq8_search(base, sq.codes(), sq.vmin, sq.scale, qs, k, depth, allow=allow)
    _same(gi, gd, oi, od)


# ---------------------------------------------------------------- query preparation

@pytest.mark.parametrize("metric,dim", [("l2", 128), ("cosine", 384), ("cosine", 100),
                                        ("ip", 7)])
def test_prepare_queries(ctx, oracle, metric, dim):
    rng = np.random.default_rng(dim)
    raw = (rng.standard_normal((300, dim)) * rng.uniform(1e-3, 1e3, (300, 1))).astype(np.float32)
    pd = vdbg.padded_dim(dim)
    got = vdbg.prepare_queries(ctx, raw, pd, metric)
    want = np.zeros((300, pd), np.float32)
    want[:, :dim] = raw
    if metric == "cosine":
        for i in range(300):
            assert oracle.lib.or_normalize(want[i], dim) == 1
    assert (got.view(np.uint32) == want.view(np.uint32)).all()


@pytest.mark.parametrize("bad", [np.nan, np.inf, -np.inf])
def test_prepare_rejects_non_finite(ctx, bad):
    raw = np.ones((4, 20), np.float32)
    raw[2, 13] = bad
    with pytest.raises(vdbg.VdbgError) as e:
        vdbg.prepare_queries(ctx, raw, 32, "l2")
    assert e.value.code == 1 and "NaN or infinite" in str(e.value)


def test_prepare_rejects_zero_cosine(ctx):
    raw = np.ones((3, 20), np.float32)
    raw[1] = 0
    vdbg.prepare_queries(ctx, raw, 32, "l2")  # fine without normalisation
    with pytest.raises(vdbg.VdbgError) as e:
        vdbg.prepare_queries(ctx, raw, 32, "cosine")
    assert e.value.code == 1 and "zero query" in str(e.value)


# ---------------------------------------------------------------- cross-segment merge

def _oracle_merge(oracle, pdist, prow, ext, off, k):
    nparts, nq, _ = pdist.shape
    oe = np.full((nq, k), np.iinfo(np.uint64).max, np.uint64)
    od = np.full((nq, k), np.inf, np.float32)
    for q in range(nq):
        d = np.ascontiguousarray(pdist[:, q, :])
        r = np.ascontiguousarray(prow[:, q, :])
        e = np.empty(k, np.uint64)
        dd = np.empty(k, np.float32)
        cnt = oracle.lib.or_merge_parts(nparts, k, d, r, ext, off, dd, e)
        oe[q, :cnt] = e[:cnt]
        od[q, :cnt] = dd[:cnt]
    return oe, od


@pytest.mark.parametrize("nparts,k", [(9, 10), (3, 100), (16, 64), (1, 7), (20, 100), (12, 500)])
def test_merge_parts(ctx, oracle, nparts, k):
    rng = np.random.default_rng(nparts * 1000 + k)
    nq = 200
    sizes = rng.integers(k // 2, 4 * k + 2, nparts)
    off = np.concatenate([[0], np.cumsum(sizes)]).astype(np.uint64)
    # a few external ids appear in two parts (an upsert visible in old and new segment)
    ext = rng.permutation(int(off[-1]) * 3)[: int(off[-1])].astype(np.uint64)
    dup = rng.choice(int(off[-1]), int(off[-1]) // 5, replace=False)
    ext[dup] = ext[rng.choice(int(off[-1]), dup.size)]
    pdist = np.full((nparts, nq, k), np.inf, np.float32)
    prow = np.full((nparts, nq, k), vdbg.NO_ID, np.uint32)
    for p in range(nparts):
        for q in range(nq):
            cnt = min(k, int(sizes[p]))
            if q % 11 == 0:
                cnt = cnt // 3  # short lists
            rows = rng.choice(int(sizes[p]), cnt, replace=False).astype(np.uint32)
            d = np.round(rng.random(cnt) * 20).astype(np.float32)  # many ties
            order = np.lexsort((rows, d))
            pdist[p, q, :cnt] = d[order]
            prow[p, q, :cnt] = rows[order]
    ge, gd = vdbg.merge_parts(ctx, pdist, prow, ext, off[:-1])
    oe, od = _oracle_merge(oracle, pdist, prow, ext, off[:-1].copy(), k)
    assert (ge == oe).all()
    assert (gd.view(np.uint32) == od.view(np.uint32)).all()


def test_collection_search_end_to_end(ctx, oracle):
    # four segments of unit rows under cosine, each with deletes; per-segment exact
    # search on the GPU, then the GPU merge, against the oracle's same pipeline
    dim, k, nq = 96, 10, 64
    sizes = [6000, 4500, 8000, 1200]
    segs, exts, allows = [], [], []
    next_id = 0
    for i, n in enumerate(sizes):
        segs.append(datagen.clustered_unit(n, dim, 80 + i, 79, 60, 0.5))
        exts.append(np.arange(next_id, next_id + n, dtype=np.uint64) * 7 + 3)
        next_id += n
        deleted, _ = _mask(n, 0.05, 90 + i)
        allows.append(~deleted)
    # the last segment re-inserts 200 ids of the first (upsert): same external id twice
    exts[3][:200] = exts[0][:200]
    raw = datagen.clustered_unit(nq, dim, 99, 79, 60, 0.5) * 3.0
    pd = vdbg.padded_dim(dim)
    q = vdbg.prepare_queries(ctx, raw, pd, "cosine")
    qo = np.zeros((nq, pd), np.float32)
    qo[:, :dim] = raw
    for i in range(nq):
        assert oracle.lib.or_normalize(qo[i], dim) == 1
    assert (q.view(np.uint32) == qo.view(np.uint32)).all()
    pdist = np.empty((len(sizes), nq, k), np.float32)
    prow = np.empty((len(sizes), nq, k), np.uint32)
    odist = np.empty_like(pdist)
    orow = np.empty_like(prow)
    for p, (base, allow) in enumerate(zip(segs, allows)):
        ds = vdbg.Dataset(ctx, base, dim, metric="cosine")
        prow[p], pdist[p] = ds.flat_search(q, k, allow=allow)
        odist[p], orow[p] = oracle.flat_search(vdbg.pad_rows(base, pd), qo, k, metric="cosine",
                                               allow=allow)
    assert (prow == orow).all() and (pdist.view(np.uint32) == odist.view(np.uint32)).all()
    ext = np.concatenate(exts)
    off = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.uint64)
    ge, gd = vdbg.merge_parts(ctx, pdist, prow, ext, off)
    oe, od = _oracle_merge(oracle, odist, orow, ext, off, k)
    assert (ge == oe).all() and (gd.view(np.uint32) == od.view(np.uint32)).all()


@pytest.mark.parametrize("k,fallbacks", [(10, 0), (10, 1), (10, 2), (300, 0)])
def test_flat_filter_float_rows_remapped(ctx, oracle, k, fallbacks):
    # float rows held as high fp16 halves, at most half allowed: the compacted source keeps
    # no fp32 rows and re-scores through the id map, on the first pass, the second chance
    # (fallbacks 1), the exact re-scan (fallbacks 2) and the k > 240 exact path
    n, nq = 30000, 48
    print(f"remapped compaction k={k} fallbacks={fallbacks}", flush=True)
    base = datagen.clustered_unit(n, 384, 61, 40, 100, 0.5)
    qs = datagen.clustered_unit(nq, 384, 62, 40, 100, 0.5)
    allow, rows = _mask(n, 0.2, 63)
    ds = vdbg.Dataset(ctx, base, 384, metric="cosine")
    ctx.set_test_fallbacks(fallbacks)
    try:
        gi, gd = ds.flat_search(qs, k, allow=allow)
        if fallbacks == 2:
            assert ctx.last_fallbacks() == nq
    finally:
        ctx.set_test_fallbacks(0)
    od, oi = oracle.flat_search(base, qs, k, metric="cosine", allow=allow)
    _same(gi, gd, oi, od)
    real = gi[gi != vdbg.NO_ID]
    assert np.isin(real, rows).all()
