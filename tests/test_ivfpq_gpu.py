"""IVF-PQ on the GPU against the reference's own results and the oracle.

The golden index was built and saved by the reference (IvfPqIndex::build + save) and its
search results recorded by IvfPqIndex::search (tests/golden/make_golden.py).  Larger
indexes are synthesised with the oracle's assignment and encoder: search parity only
depends on an index's contents.  Scores follow the reference's arithmetic order, so ids,
distances and distance-computation counts are compared exactly."""
import os

import numpy as np
import pytest

import vdbg
from ivf_file import parse_ivfpq, synth_ivfpq
from oracle_lib import KSET, METRIC
from vdbg import datagen

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _oracle_ivf(oracle, blob, base, qs, k, nprobe, rerank, metric="l2", allow=None):
    ix = parse_ivfpq(blob)
    nq = len(qs)
    od = np.empty((nq, k), np.float32)
    oi = np.empty((nq, k), np.uint32)
    dc = np.empty(nq, np.uint64)
    term2 = None
    if metric == "l2":
        term2 = np.empty(ix["nlist"] * ix["m"] * 256, np.float32)
        oracle.lib.or_ivfpq_term2(ix["coarse"], ix["nlist"], ix["pd"], ix["pq_centroids"],
                                  ix["m"], ix["dim"] // ix["m"], term2)
    oracle.lib.or_ivfpq_search_batch(KSET["avx512"], METRIC[metric], np.ascontiguousarray(base),
                                     ix["dim"], ix["pd"], ix["coarse"], ix["nlist"],
                                     ix["pq_centroids"], ix["m"], ix["list_off"],
                                     ix["list_ids"], ix["list_codes"], term2,
                                     np.ascontiguousarray(qs), nq, k, nprobe, rerank, allow, od,
                                     oi, dc, 8)
    return od, oi, dc


def _eq(gi, gd, oi, od):
    bad = np.nonzero((gi != oi).any(1) | (gd.view(np.uint32) != od.view(np.uint32)).any(1))[0]
    assert bad.size == 0, (f"{bad.size} queries differ; q={bad[0]} gpu={gi[bad[0]].tolist()} "
                           f"{gd[bad[0]].tolist()} oracle={oi[bad[0]].tolist()} "
                           f"{od[bad[0]].tolist()}")


def test_ivfpq_reference_index_matches_reference_results(ctx):
    g = np.load(os.path.join(GOLD, "ivfpq.npz"), allow_pickle=False)
    base, qs = g["base"], g["queries"]
    ds = vdbg.Dataset(ctx, base, 32)
    ix = vdbg.IvfPqIndex.load(ds, g["index_file"].tobytes())
    assert ix.info() == (24, 8, True)
    assert ix.save() == g["index_file"].tobytes()  # save(load(f)) == f
    for nprobe, rr in [(1, 0), (4, 0), (4, -1), (24, 0), (24, 5000)]:
        tag = f"np{nprobe}_r{rr if rr >= 0 else 'auto'}"
        gi, gd, dc = ix.search(qs, 10, nprobe, rr)
        _eq(gi, gd, g[f"{tag}_i"], g[f"{tag}_d"])
        assert np.array_equal(dc, g[f"{tag}_dc"]), tag


@pytest.mark.parametrize("nprobe,rerank,k", [(1, 0, 10), (16, 0, 10), (64, 0, 10), (16, -1, 10),
                                             (64, 100, 10), (32, 0, 100), (8, 200, 50)])
def test_ivfpq_sift_like_matches_oracle(ctx, oracle, nprobe, rerank, k):
    print(f"ivfpq sift-like nprobe={nprobe} rerank={rerank} k={k}", flush=True)
    base = datagen.sift_like(40000, 128, 2002)
    qs = datagen.sift_like(150, 128, 2003)
    blob = synth_ivfpq(base, 128, 256, 16, seed=1)
    ds = vdbg.Dataset(ctx, base, 128)
    ix = vdbg.IvfPqIndex.load(ds, blob)
    gi, gd, dc = ix.search(qs, k, nprobe, rerank)
    od, oi, odc = _oracle_ivf(oracle, blob, base, qs, k, nprobe, rerank)
    _eq(gi, gd, oi, od)
    assert np.array_equal(dc, odc)


@pytest.mark.parametrize("metric", ["ip", "cosine"])
def test_ivfpq_inner_product(ctx, oracle, metric):
    base = datagen.clustered_unit(20000, 64, 61, 62, 50, 0.5)
    qs = datagen.clustered_unit(80, 64, 63, 62, 50, 0.5)
    blob = synth_ivfpq(base, 64, 64, 8, seed=2, metric=metric)
    ds = vdbg.Dataset(ctx, base, 64, metric=metric)
    ix = vdbg.IvfPqIndex.load(ds, blob)
    assert ix.info()[2] is False  # no precomputed tables for inner product
    for rerank in [0, -1]:
        gi, gd, dc = ix.search(qs, 10, 8, rerank)
        od, oi, odc = _oracle_ivf(oracle, blob, base, qs, 10, 8, rerank, metric=metric)
        _eq(gi, gd, oi, od)
        assert np.array_equal(dc, odc)


def test_ivfpq_filter(ctx, oracle):
    base = datagen.sift_like(30000, 128, 71)
    qs = datagen.sift_like(60, 128, 72)
    blob = synth_ivfpq(base, 128, 128, 16, seed=3)
    allow = np.zeros((30000 + 63) // 64, np.uint64)
    rows = np.arange(0, 30000, 3)
    np.bitwise_or.at(allow, rows // 64, np.uint64(1) << (rows % 64).astype(np.uint64))
    ds = vdbg.Dataset(ctx, base, 128)
    ix = vdbg.IvfPqIndex.load(ds, blob)
    gi, gd, dc = ix.search(qs, 10, 16, -1, allow=allow)
    assert ((gi % 3 == 0) | (gi == vdbg.NO_ID)).all()
    od, oi, odc = _oracle_ivf(oracle, blob, base, qs, 10, 16, -1, allow=allow)
    _eq(gi, gd, oi, od)
    assert np.array_equal(dc, odc)


def test_ivfpq_corrupt_file_is_rejected(ctx):
    g = np.load(os.path.join(GOLD, "ivfpq.npz"), allow_pickle=False)
    ds = vdbg.Dataset(ctx, g["base"], 32)
    blob = bytearray(g["index_file"].tobytes())
    blob[100] ^= 0xFF
    with pytest.raises(vdbg.VdbgError) as e:
        vdbg.IvfPqIndex.load(ds, bytes(blob))
    assert e.value.code == 5  # Status::Corruption, as LoadIndex returns
    with pytest.raises(vdbg.VdbgError) as e:
        vdbg.IvfPqIndex.load(ds, g["index_file"].tobytes()[:-10])
    assert e.value.code == 5


@pytest.mark.parametrize("nprobe,rerank,k", [(16, -1, 50), (64, -1, 100), (300, 0, 10),
                                             (40, 1000, 20), (8, 0, 400)])
def test_ivfpq_deep_top_r_matches_oracle(ctx, oracle, nprobe, rerank, k):
    # R = max(rerank depth, k) beyond the wave top-k: the default depth max(10 k, 100) at
    # k >= 26, explicit depths, k itself, and nprobe beyond 256 lists
    print(f"ivfpq deep nprobe={nprobe} rerank={rerank} k={k}", flush=True)
    base = datagen.sift_like(40000, 128, 2002)
    qs = datagen.sift_like(70, 128, 2004)
    blob = synth_ivfpq(base, 128, 512, 16, seed=2)
    ds = vdbg.Dataset(ctx, base, 128)
    ix = vdbg.IvfPqIndex.load(ds, blob)
    gi, gd, dc = ix.search(qs, k, nprobe, rerank)
    od, oi, odc = _oracle_ivf(oracle, blob, base, qs, k, nprobe, rerank)
    _eq(gi, gd, oi, od)
    assert np.array_equal(dc, odc)
