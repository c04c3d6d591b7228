"""vdb's MutableSegment on the GPU: an appendable dataset (vdbg_dataset_create_appendable /
vdbg_dataset_append, src/engine/mutable_segment.cc:10-44) searched exactly over the rows not
deleted and matching the filter (MutableSegment::Search, :46-64), alone and as the in-memory
parts of a collection search, which vdb lists before its disk segments
(collection_impl.cc:1050-1060).  Expected results: the oracle's flat search over the allowed
rows (MutableSegment::Search's loop is an exact TopK over them; its source file needs
nlohmann_json and CRoaring, absent here, so it is restated, not compiled) and the oracle's
collection composition."""
import numpy as np
import pytest

import vdbg
from vdbg import datagen

pytestmark = pytest.mark.gpu


def _mask(n, frac, seed):
    bits = np.random.default_rng(seed).random(n) < frac
    w = np.zeros((n + 63) // 64, np.uint64)
    r = np.nonzero(bits)[0]
    np.bitwise_or.at(w, r // 64, np.uint64(1) << (r % 64).astype(np.uint64))
    return w


@pytest.mark.parametrize("kind", ["int", "float", "cosine"])
def test_append_then_search(ctx, oracle, kind):
    dim = 48
    pd = vdbg.padded_dim(dim)
    metric = "cosine" if kind == "cosine" else "l2"
    total = 5000
    if kind == "int":
        rows = datagen.sift_like(total, dim, 970)
        rows = datagen.pad(rows, pd)
    elif kind == "float":
        rows = datagen.pad(datagen.uniform_rows(total, dim, 971) * 3, pd)
    else:
        rows = datagen.pad(datagen.clustered_unit(total, dim, 972, 79, 30, 0.4), pd)
    q = rows[np.random.default_rng(973).integers(0, total, 30)] + np.float32(0.5) * (np.arange(pd) < dim)
    if kind == "cosine":
        q /= np.linalg.norm(q, axis=1, keepdims=True)
    ds = vdbg.Dataset.appendable(ctx, dim, metric, capacity=1000)
    ext = np.arange(total, dtype=np.uint64) * 3 + 7
    at = 0
    # grows past the capacity three times; the threshold sample is gathered at 2,202 rows and
    # again at 5,000 (the rows doubled), so the search at 3,202 rows reads a sample that
    # trails the rows
    for step, chunk in enumerate((1, 700, 1, 1500, 1000, 1798)):
        first = ds.append(rows[at:at + chunk], ext[at:at + chunk])
        assert first == at
        at += chunk
        assert ds.n == at
        print(f"mutable {kind}: {at} rows", flush=True)
        cur = rows[:at]
        for k in (1, 10, 100):
            for frac in (None, 0.3):
                allow = None if frac is None else _mask(at, frac, 980 + step)
                ids, d = ds.flat_search(q, k, allow=allow)
                od, oi = oracle.flat_search(cur, q, k, metric=metric, allow=allow)
                assert np.array_equal(ids, oi), (kind, at, k, frac)
                assert np.array_equal(d.view(np.uint32), od.view(np.uint32)), (kind, at, k, frac)
    ds.close()


def test_memory_parts_in_a_collection(ctx, oracle):
    """The active and a frozen mutable segment ahead of two disk segments: memory parts are
    scanned exactly (plan "scan" / "scan_filter"), win ties on distance, and an external id
    they hold hides its older disk copy."""
    dim = 32
    pd = vdbg.padded_dim(dim)
    sizes = [(700, "memory"), (1800, "memory"), (6000, "flat"), (3000, "flat")]
    segs, handles = [], []
    disk_rows = datagen.pad(datagen.uniform_rows(9000, dim, 990) * 4, pd)
    for i, (n, kind) in enumerate(sizes):
        if kind == "memory":
            # upserts of disk rows (same external ids, same or moved vectors)
            base = disk_rows[np.random.default_rng(991 + i).integers(0, 9000, n)].copy()
            base[n // 2:, 0] += 0.25
            ext = np.arange(n, dtype=np.uint64) + 5000 * i
        else:
            off = 0 if i == 2 else 6000
            base = disk_rows[off:off + n].copy()
            ext = np.arange(n, dtype=np.uint64) + off
        if kind == "memory":
            ds = vdbg.Dataset.appendable(ctx, dim, "l2", capacity=256)
            for a in range(0, n, 333):
                ds.append(base[a:a + 333], ext[a:a + 333])
        else:
            ds = vdbg.Dataset(ctx, base, dim)
            ds.set_external_ids(ext)
        segs.append({"base": base, "ext": ext, "kind": kind,
                     "deleted": _mask(n, 0.05, 995 + i) if i in (0, 2) else None,
                     "filter": None})
        handles.append(ds)
    q = disk_rows[np.random.default_rng(999).integers(0, 9000, 25)] + np.float32(0.01)
    print("collection with memory parts", flush=True)
    try:
        for filt, kw in ((None, {}), ("f", {}), ("f", {"strategy": "post_filter"})):
            for i, sg in enumerate(segs):
                sg["filter"] = None if filt is None else _mask(sg["base"].shape[0], 0.5, 1000 + i)
            for k in (1, 10, 50):
                gi, gd, gdc, gp = vdbg.collection_search(
                    ctx, [(ds, None, sg["deleted"], sg["filter"], sg["kind"] == "memory")
                          for ds, sg in zip(handles, segs)], dim, "l2", q, k,
                    vdbg.SearchParams(**kw))
                okw = dict(kw)
                okw["strategy"] = vdbg.STRATEGIES[okw.get("strategy", "auto")]
                oi, od, odc, op = oracle.collection_search(segs, dim, "l2", q, k, **okw)
                assert gp == op, (filt, kw, k)
                assert gp[:2] == (["scan"] * 2 if filt is None else ["scan_filter"] * 2)
                assert np.array_equal(gi, oi), (filt, kw, k)
                assert np.array_equal(gd.view(np.uint32), od.view(np.uint32)), (filt, kw, k)
                assert np.array_equal(gdc, odc), (filt, kw, k)
    finally:
        for ds in handles:
            ds.close()


def test_memory_part_appended_without_ids(ctx, oracle):
    """Rows appended without external ids take their row numbers as external ids: an
    in-memory part built that way merges with a disk segment as if its ids were 0..n-1."""
    dim = 32
    pd = vdbg.padded_dim(dim)
    mem = datagen.pad(datagen.uniform_rows(1500, dim, 1010) * 4, pd)
    disk = datagen.pad(datagen.uniform_rows(4000, dim, 1011) * 4, pd)
    ap = vdbg.Dataset.appendable(ctx, dim, "l2", capacity=256)
    for a in range(0, 1500, 500):
        ap.append(mem[a:a + 500])  # no external ids
    ds = vdbg.Dataset(ctx, disk, dim)
    dext = np.arange(4000, dtype=np.uint64) + 1000  # ids 1000..1499 also name memory rows
    ds.set_external_ids(dext)
    segs = [{"base": mem, "ext": np.arange(1500, dtype=np.uint64), "kind": "memory",
             "deleted": None, "filter": None},
            {"base": disk, "ext": dext, "kind": "flat", "deleted": None, "filter": None}]
    q = np.ascontiguousarray(disk[np.random.default_rng(1012).integers(0, 4000, 20)] + np.float32(0.02))
    try:
        for k in (1, 10, 40):
            gi, gd, gdc, gp = vdbg.collection_search(
                ctx, [(ap, None, None, None, True), (ds, None, None, None, False)], dim, "l2",
                q, k, vdbg.SearchParams())
            oi, od, odc, op = oracle.collection_search(segs, dim, "l2", q, k, strategy=0)
            assert gp == op
            assert np.array_equal(gi, oi), k
            assert np.array_equal(gd.view(np.uint32), od.view(np.uint32)), k
    finally:
        ds.close()
        ap.close()


def test_append_errors(ctx):
    rows = np.ones((10, 16), np.float32)
    ds = vdbg.Dataset(ctx, rows, 16)
    with pytest.raises(vdbg.VdbgError) as e:
        ds.append(rows)
    assert e.value.code == 6
    ds.close()
    ap = vdbg.Dataset.appendable(ctx, 16)
    ap.append(rows)
    sq = vdbg.Sq8Index(ap)
    with pytest.raises(vdbg.VdbgError) as e:
        ap.append(rows)
    assert e.value.code == 6
    sq.close()
    ap.append(rows)  # the index is gone: rows are taken again
    assert ap.n == 20
    ids, d = ap.flat_search(np.ones((2, 16), np.float32), 25)
    assert (ids[:, :20] < 20).all() and (ids[:, 20:] == 0xFFFFFFFF).all()
    ap.close()
