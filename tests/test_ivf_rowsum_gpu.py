"""The IVF-PQ L2 scan that ranks rows on their term-2 sums (k_ivf_scan_rs) against the oracle
and against the per-list table scan it replaces.

Rows are ranked on offset + rowsum + sum_j qtab and only the rows near the running threshold
are scored in the reference's order (ivf_pq.cc:197-217), so every returned id, distance and
distance count must equal the oracle's bit for bit: on duplicated rows (equal scores decided
by row id across the block's four waves), on chunks of 64 probed lists and past them, with
sparse filters that leave the top short, and for m = 4 and 8."""
import numpy as np
import pytest

import vdbg
from ivf_file import parse_ivfpq, synth_ivfpq, write_ivfpq
from vdbg import datagen
from test_ivfpq_gpu import _eq, _oracle_ivf

pytestmark = pytest.mark.gpu


def _words(n, rows):
    allow = np.zeros((n + 63) // 64, np.uint64)
    rows = np.asarray(rows, np.int64)
    np.bitwise_or.at(allow, rows // 64, np.uint64(1) << (rows % 64).astype(np.uint64))
    return allow


def _both(ctx, ix, qs, k, nprobe, rerank, allow=None):
    ctx.set_ivf_row_sums(False)
    try:
        ref = ix.search(qs, k, nprobe, rerank, allow=allow)
    finally:
        ctx.set_ivf_row_sums(True)
    got = ix.search(qs, k, nprobe, rerank, allow=allow)
    return got, ref


@pytest.mark.parametrize("nprobe,rerank,k", [(1, 0, 10), (63, 0, 10), (64, 100, 10), (65, 0, 10),
                                             (130, -1, 10), (128, 0, 64), (40, 250, 10)])
def test_rowsum_scan_matches_oracle_and_table_scan(ctx, oracle, nprobe, rerank, k):
    print(f"ivf rowsum nprobe={nprobe} rerank={rerank} k={k}", flush=True)
    base = datagen.sift_like(30000, 128, 3101)
    qs = datagen.sift_like(90, 128, 3102)
    blob = synth_ivfpq(base, 128, 256, 16, seed=5)
    ds = vdbg.Dataset(ctx, base, 128)
    ix = vdbg.IvfPqIndex.load(ds, blob)
    (gi, gd, dc), (ti, td, tdc) = _both(ctx, ix, qs, k, nprobe, rerank)
    od, oi, odc = _oracle_ivf(oracle, blob, base, qs, k, nprobe, rerank)
    _eq(gi, gd, oi, od)
    assert np.array_equal(dc, odc)
    _eq(ti, td, oi, od)
    assert np.array_equal(tdc, odc)


def test_rowsum_scan_ties_decided_by_row_id(ctx, oracle):
    # every row appears eight times: equal codes in one list score equally, and the lowest
    # ids must win wherever the copies land among the block's waves
    print("ivf rowsum duplicated rows", flush=True)
    uniq = datagen.sift_like(2500, 128, 3111)
    base = np.ascontiguousarray(np.tile(uniq, (8, 1)))
    qs = datagen.sift_like(60, 128, 3112)
    blob = synth_ivfpq(base, 128, 64, 16, seed=6)
    ds = vdbg.Dataset(ctx, base, 128)
    ix = vdbg.IvfPqIndex.load(ds, blob)
    for nprobe, rerank, k in [(8, 0, 10), (64, 0, 100), (16, 50, 7)]:
        gi, gd, dc = ix.search(qs, k, nprobe, rerank)
        od, oi, odc = _oracle_ivf(oracle, blob, base, qs, k, nprobe, rerank)
        _eq(gi, gd, oi, od)
        assert np.array_equal(dc, odc)


@pytest.mark.parametrize("frac", [0.001, 0.02, 0.5])
def test_rowsum_scan_with_filter(ctx, oracle, frac):
    print(f"ivf rowsum filter {frac}", flush=True)
    n = 30000
    base = datagen.sift_like(n, 128, 3121)
    qs = datagen.sift_like(70, 128, 3122)
    blob = synth_ivfpq(base, 128, 128, 16, seed=7)
    rng = np.random.default_rng(3123)
    allow = _words(n, np.nonzero(rng.random(n) < frac)[0])
    ds = vdbg.Dataset(ctx, base, 128)
    ix = vdbg.IvfPqIndex.load(ds, blob)
    for nprobe, rerank in [(16, 0), (32, -1)]:
        (gi, gd, dc), (ti, td, tdc) = _both(ctx, ix, qs, 10, nprobe, rerank, allow=allow)
        od, oi, odc = _oracle_ivf(oracle, blob, base, qs, 10, nprobe, rerank, allow=allow)
        _eq(gi, gd, oi, od)
        assert np.array_equal(dc, odc)
        _eq(ti, td, oi, od)


@pytest.mark.parametrize("dim,m", [(64, 4), (64, 8), (128, 4), (96, 8), (48, 16)])
def test_rowsum_scan_other_code_sizes(ctx, oracle, dim, m):
    # sub-vectors of 16, 8 and 32 dims take the table kernel's compiled widths, 12 and 3 its
    # run-time width
    print(f"ivf rowsum dim={dim} m={m}", flush=True)
    base = datagen.sift_like(20000, dim, 3131)
    qs = datagen.sift_like(50, dim, 3132)
    blob = synth_ivfpq(base, dim, 128, m, seed=8)
    ds = vdbg.Dataset(ctx, base, dim)
    ix = vdbg.IvfPqIndex.load(ds, blob)
    for nprobe, rerank, k in [(16, 0, 10), (70, -1, 10), (24, 0, 130)]:
        gi, gd, dc = ix.search(qs, k, nprobe, rerank)
        od, oi, odc = _oracle_ivf(oracle, blob, base, qs, k, nprobe, rerank)
        _eq(gi, gd, oi, od)
        assert np.array_equal(dc, odc)


def test_rowsum_scan_empty_lists_and_fewer_rows_than_r(ctx, oracle):
    # 1,500 rows over 256 lists, each list's centroid repeated by an empty twin: every chunk
    # of 64 probed lists holds empty lists at the same coarse distance as full ones, and the
    # probed rows can number fewer than R (the seed then bounds nothing and answers are padded)
    print("ivf rowsum empty lists", flush=True)
    base = datagen.sift_like(1500, 128, 3141)
    qs = datagen.sift_like(40, 128, 3142)
    ix0 = parse_ivfpq(synth_ivfpq(base, 128, 256, 16, seed=9))
    off = ix0["list_off"].astype(np.int64)
    coarse, ids, codes = [], [], []
    for l in range(ix0["nlist"]):
        for twin in range(2):
            coarse.append(ix0["coarse"][l])
            if twin == 0:
                ids.append(ix0["list_ids"][off[l]:off[l + 1]])
                codes.append(ix0["list_codes"][off[l] * 16:off[l + 1] * 16])
            else:
                ids.append(np.zeros(0, np.uint32))
                codes.append(np.zeros(0, np.uint8))
    blob = write_ivfpq(1500, 128, np.array(coarse), 128, 16, ix0["pq_centroids"], ids, codes)
    ds = vdbg.Dataset(ctx, base, 128)
    ix = vdbg.IvfPqIndex.load(ds, blob)
    for nprobe, rerank, k in [(1, 0, 10), (8, 100, 10), (40, 0, 200), (200, -1, 10), (512, 0, 64)]:
        (gi, gd, dc), (ti, td, tdc) = _both(ctx, ix, qs, k, nprobe, rerank)
        od, oi, odc = _oracle_ivf(oracle, blob, base, qs, k, nprobe, rerank)
        _eq(gi, gd, oi, od)
        assert np.array_equal(dc, odc)
        _eq(ti, td, oi, od)


@pytest.mark.parametrize("rerank,k", [(0, 10), (-1, 10), (0, 300)])
def test_query_with_nan_leaves_the_batch_intact(ctx, oracle, rerank, k):
    # a query whose coarse distances are all NaN can leave no-id probe slots: every scan
    # (row sums, per-list tables, the deep top-R past 256) takes them as empty lists, and the
    # batch's finite queries are answered as the oracle answers them
    print(f"ivf nan query rerank={rerank} k={k}", flush=True)
    base = datagen.sift_like(20000, 128, 3151)
    qs = datagen.sift_like(30, 128, 3152)
    qs[7, :] = np.nan
    finite = np.arange(30) != 7
    blob = synth_ivfpq(base, 128, 128, 16, seed=11)
    ds = vdbg.Dataset(ctx, base, 128)
    ix = vdbg.IvfPqIndex.load(ds, blob)
    od, oi, odc = _oracle_ivf(oracle, blob, base, np.ascontiguousarray(qs[finite]), k, 16, rerank)
    (gi, gd, dc), (ti, td, tdc) = _both(ctx, ix, qs, k, 16, rerank)
    _eq(gi[finite], gd[finite], oi, od)
    assert np.array_equal(dc[finite], odc)
    _eq(ti[finite], td[finite], oi, od)
