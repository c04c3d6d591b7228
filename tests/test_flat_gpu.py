"""Flat exact search on the GPU against the oracle (FlatIndex::search semantics,
src/index/flat_index.cc:11-39): ids bit-exact under the (dist, id) tie rule, distances
bit-exact to the reference's AVX-512 kernel (the oracle restates it lane by lane)."""
import numpy as np
import pytest

import vdbg
from vdbg import datagen

pytestmark = pytest.mark.gpu


def _check_equal(gi, gd, oi, od):
    assert gi.shape == oi.shape
    bad = np.nonzero((gi != oi).any(axis=1) | (gd.view(np.uint32) != od.view(np.uint32)).any(axis=1))[0]
    assert bad.size == 0, (
        f"{bad.size} queries differ; first q={bad[0]} gpu={gi[bad[0]].tolist()} "
        f"{gd[bad[0]].tolist()} oracle={oi[bad[0]].tolist()} {od[bad[0]].tolist()}")


@pytest.mark.parametrize("n,nq,k", [(100, 5, 10), (5000, 40, 10), (20000, 300, 10),
                                    (20000, 300, 100), (4099, 33, 1)])
def test_flat_uniform_matches_oracle(ctx, oracle, n, nq, k):
    print(f"flat uniform n={n} nq={nq} k={k}", flush=True)
    base = datagen.uniform_rows(n, 128, 1001)
    qs = datagen.uniform_rows(nq, 128, 1002)
    ds = vdbg.Dataset(ctx, base, 128)
    gi, gd = ds.flat_search(qs, k)
    od, oi = oracle.flat_search(base, qs, k)
    _check_equal(gi, gd, oi, od)


@pytest.mark.parametrize("n,nq,k", [(50000, 200, 10), (50000, 130, 100)])
def test_flat_sift_like_ties(ctx, oracle, n, nq, k):
    # integer-valued data: exact GEMM arithmetic, many distance ties broken by id
    print(f"flat sift-like n={n} nq={nq} k={k}", flush=True)
    base = datagen.sift_like(n, 128, 2002)
    qs = datagen.sift_like(nq, 128, 2003)
    ds = vdbg.Dataset(ctx, base, 128)
    gi, gd = ds.flat_search(qs, k)
    od, oi = oracle.flat_search(base, qs, k)
    _check_equal(gi, gd, oi, od)
    assert ctx.last_fallbacks() == 0


def test_flat_k_larger_than_rows(ctx, oracle):
    base = datagen.uniform_rows(5, 128, 7)
    ds = vdbg.Dataset(ctx, base, 128)
    gi, gd = ds.flat_search(base[:1], 100)
    assert (gi[0, :5] != vdbg.NO_ID).all() and (gi[0, 5:] == vdbg.NO_ID).all()
    assert gi[0, 0] == 0
    assert np.isinf(gd[0, 5:]).all()


def test_flat_duplicate_rows_tie_by_id(ctx, oracle):
    rng = np.random.default_rng(3)
    uniq = rng.random((50, 128), dtype=np.float32)
    base = uniq[rng.integers(0, 50, 6000)]
    qs = uniq[:40].copy()
    ds = vdbg.Dataset(ctx, base, 128)
    gi, gd = ds.flat_search(qs, 10)
    od, oi = oracle.flat_search(base, qs, 10)
    _check_equal(gi, gd, oi, od)


def test_flat_filter_respected(ctx, oracle):
    base = datagen.uniform_rows(20000, 128, 11)
    qs = datagen.uniform_rows(64, 128, 12)
    allow = np.zeros((20000 + 63) // 64, np.uint64)
    rows = np.arange(1, 20000, 2)
    np.bitwise_or.at(allow, rows // 64, np.uint64(1) << (rows % 64).astype(np.uint64))
    ds = vdbg.Dataset(ctx, base, 128)
    gi, gd = ds.flat_search(qs, 50, allow=allow)
    assert (gi % 2 == 1).all()
    od, oi = oracle.flat_search(base, qs, 50, allow=allow)
    _check_equal(gi, gd, oi, od)


@pytest.mark.parametrize("metric", ["ip", "cosine"])
def test_flat_inner_product(ctx, oracle, metric):
    base = datagen.clustered_unit(20000, 128, 21, 22, 100, 0.5)
    qs = datagen.clustered_unit(100, 128, 23, 22, 100, 0.5)
    ds = vdbg.Dataset(ctx, base, 128, metric=metric)
    gi, gd = ds.flat_search(qs, 10)
    od, oi = oracle.flat_search(base, qs, 10, metric=metric)
    _check_equal(gi, gd, oi, od)


@pytest.mark.parametrize("dim", [7, 37, 100, 384])
def test_flat_other_dims(ctx, oracle, dim):
    pd = vdbg.padded_dim(dim)
    base = datagen.pad(datagen.uniform_rows(6000, dim, 31), pd)
    qs = datagen.pad(datagen.uniform_rows(40, dim, 32), pd)
    ds = vdbg.Dataset(ctx, base, dim)
    gi, gd = ds.flat_search(qs, 10)
    od, oi = oracle.flat_search(base, qs, 10)
    _check_equal(gi, gd, oi, od)


@pytest.mark.parametrize("data", ["sift_like", "uniform"])
def test_flat_large_batch_many_tiles(ctx, oracle, data):
    # many 64-row tiles per block and many query tiles: the GEMM's staged tiles and row-norm
    # slots are reused often while waves drift apart
    n, nq, k = 300000, 1024 if data == "sift_like" else 256, 10
    print(f"flat large {data} n={n} nq={nq}", flush=True)
    gen = datagen.sift_like if data == "sift_like" else datagen.uniform_rows
    base = gen(n, 128, 3101)
    qs = gen(nq, 128, 3102)
    ds = vdbg.Dataset(ctx, base, 128)
    gi, gd = ds.flat_search(qs, k)
    od, oi = oracle.flat_search(base, qs, k)
    _check_equal(gi, gd, oi, od)


def test_dataset_from_device_rows_in_flight(ctx, oracle):
    # rows produced by torch kernels still queued on torch's stream, the source buffer
    # released right after: every dataset must hold its own rows
    import torch

    dev = torch.device("cuda:0")
    hosts, dss = [], []
    for p in range(4):
        rows = datagen.clustered_unit_t(torch, 40000, 96, 7000 + p, 7100, 64, 0.5, dev)
        dss.append(vdbg.Dataset.from_device(ctx, rows.data_ptr(), 40000, 96, 96, "cosine"))
        hosts.append(rows.cpu().numpy())
        del rows
    qs = hosts[0][:64].copy()
    for p in range(4):
        gi, gd = dss[p].flat_search(qs, 10)
        od, oi = oracle.flat_search(hosts[p], qs, 10, metric="cosine")
        _check_equal(gi, gd, oi, od)


@pytest.mark.parametrize("k,metric,frac", [(250, "l2", None), (300, "l2", None),
                                           (1000, "ip", None), (4000, "l2", 0.3),
                                           (10000, "cosine", None)])
def test_flat_large_k(ctx, oracle, k, metric, frac):
    # k beyond the wave top-k, up to vdb's kMaxK = 10,000 (collection_impl.cc:26)
    print(f"flat large k={k} {metric} filter={frac}", flush=True)
    n, nq = 30000, 24
    if metric == "l2":
        base, qs = datagen.uniform_rows(n, 64, 4101), datagen.uniform_rows(nq, 64, 4102)
    else:
        base = datagen.clustered_unit(n, 64, 4103, 4104, 40, 0.5)
        qs = datagen.clustered_unit(nq, 64, 4105, 4104, 40, 0.5)
    allow = None
    if frac is not None:
        rows = np.nonzero(np.random.default_rng(7).random(n) < frac)[0]
        allow = np.zeros((n + 63) // 64, np.uint64)
        np.bitwise_or.at(allow, rows // 64, np.uint64(1) << (rows % 64).astype(np.uint64))
    ds = vdbg.Dataset(ctx, base, 64, metric=metric)
    gi, gd = ds.flat_search(qs, k, allow=allow)
    od, oi = oracle.flat_search(base, qs, k, metric=metric, allow=allow)
    _check_equal(gi, gd, oi, od)


def _sample_aligned_rows(n, dim, near):
    # A threshold sample of S rows takes every (n / S)-th row (its first 2^b positions hold
    # the multiples of n / 2^b).  Here every near row sits on a multiple of n / 2048, so any
    # sample of at least 2,048 rows holds all of them, and every other row is far away: the
    # lower-rank admission threshold then keeps fewer rows than the depth asks for, and the
    # certificate must refuse it and the re-scan answer.
    rng = np.random.default_rng(5151)
    base = (100.0 + rng.random((n, dim), dtype=np.float32)).astype(np.float32)
    at = (n // 2048) * np.arange(near)
    base[at, :] = 0.0
    base[at, 0] = 0.01 * (1 + np.arange(near, dtype=np.float32))
    qs = np.zeros((8, dim), np.float32)
    qs[:, 1] = 1e-3 * np.arange(8, dtype=np.float32)
    return base, qs


@pytest.mark.parametrize("kind", ["flat", "sq8"])
def test_threshold_short_of_depth_falls_back(ctx, oracle, kind):
    n, dim, near = 4 * 65536, 32, 60
    print(f"threshold short of depth: {kind} n={n} near={near}", flush=True)
    base, qs = _sample_aligned_rows(n, dim, near)
    ds = vdbg.Dataset(ctx, base, dim)
    if kind == "flat":
        gi, gd = ds.flat_search(qs, 100)
        od, oi = oracle.flat_search(base, qs, 100)
    else:
        sq = vdbg.Sq8Index(ds)
        gi, gd = sq.search(qs, 10, 100)
        od, oi = oracle.sq8_search(base, sq.codes(), sq.vmin, sq.scale, qs, 10, 100)
    assert ctx.last_fallbacks() > 0
    _check_equal(gi, gd, oi, od)


@pytest.mark.parametrize("gated", [True, False])
@pytest.mark.parametrize("level", [0, 1, 2])
@pytest.mark.parametrize("kind", ["flat_int", "flat_float", "sq8", "filtered"])
def test_fallback_passes_queued_or_read(ctx, oracle, gated, level, kind):
    """The second chance and the exact re-scan, forced for every query (level 1: the first
    certificate fails; 2: the second too), queued for every slot with their counts left on
    the device (gated) or sized from host reads of the counts: the same results as the
    oracle's either way, and the same number of exact re-scans."""
    n, nq, k = 40000, 150, 10
    print(f"fallback passes {kind} level={level} gated={gated}", flush=True)
    if kind == "flat_int":
        base, qs = datagen.sift_like(n, 128, 7101), datagen.sift_like(nq, 128, 7102)
    else:
        base, qs = datagen.uniform_rows(n, 128, 7103), datagen.uniform_rows(nq, 128, 7104)
    allow = None
    if kind == "filtered":  # a third of the rows: the compacted scan
        allow = np.zeros((n + 63) // 64, np.uint64)
        rows = np.arange(0, n, 3)
        np.bitwise_or.at(allow, rows // 64, np.uint64(1) << (rows % 64).astype(np.uint64))
    ds = vdbg.Dataset(ctx, base, 128)
    ctx.set_gated_fallbacks(gated)
    ctx.set_test_fallbacks(level)
    try:
        if kind == "sq8":
            sq = vdbg.Sq8Index(ds)
            gi, gd = sq.search(qs, k, 100)
        else:
            gi, gd = ds.flat_search(qs, k, allow=allow)
        assert ctx.last_fallbacks() == (nq if level == 2 else 0)
    finally:
        ctx.set_test_fallbacks(0)
        ctx.set_gated_fallbacks(True)
    if kind == "sq8":
        od, oi = oracle.sq8_search(base, sq.codes(), sq.vmin, sq.scale, qs, k, 100)
        sq.close()
    else:
        od, oi = oracle.flat_search(base, qs, k, allow=allow)
    _check_equal(gi, gd, oi, od)
    ds.close()
