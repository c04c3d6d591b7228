"""Exact distances under each of vdb's kernel sets (src/distance/cpu_features.cc:33-58):
scalar, AVX2 and AVX-512 sum in different orders, and the GPU follows whichever set the
context selects, bit for bit against the oracle's restatement of that set."""
import numpy as np
import pytest

import vdbg
from ivf_file import parse_ivfpq, synth_ivfpq
from oracle_lib import KSET, METRIC
from vdbg import datagen

pytestmark = pytest.mark.gpu

SETS = ["scalar", "avx2", "avx512"]


@pytest.fixture
def kctx(ctx):
    before = ctx.kernels
    yield ctx
    ctx.set_kernels(before)


def test_default_is_best_host_set(ctx):
    assert ctx.kernels in SETS
    with pytest.raises(vdbg.VdbgError) as e:
        ctx.set_kernels("neon")
    assert e.value.code == 1


@pytest.mark.parametrize("kset", SETS)
@pytest.mark.parametrize("metric", ["l2", "ip"])
def test_flat_follows_kernel_set(kctx, oracle, kset, metric):
    kctx.set_kernels(kset)
    base = datagen.uniform_rows(30000, 96, 6101)
    qs = datagen.uniform_rows(80, 96, 6102)
    ds = vdbg.Dataset(kctx, base, 96, metric=metric)
    gi, gd = ds.flat_search(qs, 10)
    od, oi = oracle.flat_search(base, qs, 10, metric=metric, kset=kset)
    assert np.array_equal(gi, oi)
    assert np.array_equal(gd.view(np.uint32), od.view(np.uint32))
    # the sets do differ in the last bits on this data
    if kset != "avx512":
        od2, _ = oracle.flat_search(base, qs, 10, metric=metric, kset="avx512")
        assert not np.array_equal(od.view(np.uint32), od2.view(np.uint32))


@pytest.mark.parametrize("kset", SETS)
def test_sq8_follows_kernel_set(kctx, oracle, kset):
    kctx.set_kernels(kset)
    base = datagen.uniform_rows(20000, 64, 6201)
    qs = datagen.uniform_rows(40, 64, 6202)
    ds = vdbg.Dataset(kctx, base, 64)
    sq = vdbg.Sq8Index(ds)
    for depth in (0, 40):
        gi, gd = sq.search(qs, 10, depth)
        od, oi = oracle.sq8_search(base, sq.codes(), sq.vmin, sq.scale, qs, 10, depth, kset=kset)
        assert np.array_equal(gi, oi) and np.array_equal(gd.view(np.uint32), od.view(np.uint32))


@pytest.mark.parametrize("kset", SETS)
def test_ivfpq_and_rerank_follow_kernel_set(kctx, oracle, kset):
    # the coarse distances and the rerank use the set; ADC tables use L2SqAny / DotAny
    kctx.set_kernels(kset)
    base = datagen.uniform_rows(20000, 64, 6301)
    qs = datagen.uniform_rows(40, 64, 6302)
    blob = synth_ivfpq(base, 64, 64, 16, seed=3)
    ds = vdbg.Dataset(kctx, base, 64)
    ix = vdbg.IvfPqIndex.load(ds, blob)
    gi, gd, dc = ix.search(qs, 10, 8, 50)
    f = parse_ivfpq(blob)
    nq, k = len(qs), 10
    od = np.empty((nq, k), np.float32)
    oi = np.empty((nq, k), np.uint32)
    odc = np.empty(nq, np.uint64)
    term2 = np.empty(f["nlist"] * f["m"] * 256, np.float32)
    oracle.lib.or_ivfpq_term2(f["coarse"], f["nlist"], f["pd"], f["pq_centroids"], f["m"],
                              f["dim"] // f["m"], term2)
    oracle.lib.or_ivfpq_search_batch(KSET[kset], METRIC["l2"], np.ascontiguousarray(base),
                                     f["dim"], f["pd"], f["coarse"], f["nlist"], f["pq_centroids"],
                                     f["m"], f["list_off"], f["list_ids"], f["list_codes"], term2,
                                     np.ascontiguousarray(qs), nq, k, 8, 50, None, od, oi, odc, 8)
    assert np.array_equal(gi, oi) and np.array_equal(gd.view(np.uint32), od.view(np.uint32))
    assert np.array_equal(dc, odc)
    cand = np.random.default_rng(1).integers(0, 20000, (40, 90)).astype(np.uint32)
    ri, rd, _ = ds.rerank(qs, cand, 10)
    for q in range(40):
        d2 = np.empty(10, np.float32)
        i2 = np.empty(10, np.uint32)
        oracle.lib.or_rerank(KSET[kset], METRIC["l2"], np.ascontiguousarray(base), 64,
                             np.ascontiguousarray(qs[q]), cand[q].copy(), 90, 10, d2, i2)
        assert np.array_equal(ri[q], i2) and np.array_equal(rd[q].view(np.uint32), d2.view(np.uint32))
