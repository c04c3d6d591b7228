"""Rerank on the GPU (src/index/index.cc:89-95): the float rerank that vdb's CPU HNSW-SQ8
and IVF-PQ searches apply to their candidates, run against the resident rows, compared with
the oracle bit for bit, including duplicate and padded candidates and depths beyond one
wavefront's top-k."""
import numpy as np
import pytest

import vdbg
from oracle_lib import KSET, METRIC
from vdbg import datagen

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("metric,depth,k,data", [("l2", 100, 10, "sift"), ("cosine", 64, 64, "unit"),
                                                 ("ip", 700, 10, "unit"), ("l2", 900, 300, "sift"),
                                                 ("ip", 100, 10, "sift"), ("l2", 64, 10, "mixed")])
def test_rerank_matches_oracle(ctx, oracle, metric, depth, k, data):
    # SIFT-like integer rows and queries (depth <= 256) rerank from the rows' int8 copy in
    # exact integer arithmetic; "mixed" gives every third query a fractional value, so those
    # fall back to the fp32 rows within the same batch
    n, nq = 20000, 40
    rng = np.random.default_rng(depth + k)
    if data in ("sift", "mixed"):
        base, qs = datagen.sift_like(n, 128, 5101), datagen.sift_like(nq, 128, 5102)
        if data == "mixed":
            qs[::3, 5] += np.float32(0.25)
    else:
        base = datagen.clustered_unit(n, 128, 5103, 5104, 30, 0.5)
        qs = datagen.clustered_unit(nq, 128, 5105, 5104, 30, 0.5)
    cand = rng.integers(0, n, (nq, depth)).astype(np.uint32)
    cand[::3, depth // 2:] = vdbg.NO_ID        # short candidate lists
    cand[1::5, :4] = cand[1::5, 4:8]           # duplicates
    ds = vdbg.Dataset(ctx, base, 128, metric=metric)
    gi, gd, dc = ds.rerank(qs, cand, k)
    for q in range(nq):
        c = cand[q][cand[q] != vdbg.NO_ID].copy()
        od = np.full(k, np.inf, np.float32)
        oi = np.full(k, vdbg.NO_ID, np.uint32)
        cnt = oracle.lib.or_rerank(KSET["avx512"], METRIC[metric], np.ascontiguousarray(base), 128,
                                   np.ascontiguousarray(qs[q]), c, c.size, k, od, oi)
        assert cnt == min(k, c.size)
        assert np.array_equal(gi[q], oi), q
        assert np.array_equal(gd[q].view(np.uint32), od.view(np.uint32)), q
        assert dc[q] == c.size


def test_rerank_rejects_rows_out_of_range(ctx):
    base = datagen.uniform_rows(100, 16, 5201)
    ds = vdbg.Dataset(ctx, base, 16)
    cand = np.array([[1, 2, 100]], np.uint32)
    with pytest.raises(vdbg.VdbgError) as e:
        ds.rerank(base[:1], cand, 2)
    assert e.value.code == 1


def test_rerank_depth_zero_returns_nothing(ctx):
    base = datagen.uniform_rows(100, 16, 5202)
    ds = vdbg.Dataset(ctx, base, 16)
    gi, gd, dc = ds.rerank(base[:3], np.zeros((3, 0), np.uint32), 5)
    assert (gi == vdbg.NO_ID).all() and np.isinf(gd).all() and (dc == 0).all()
