"""Concurrent one-query searches through a coalescer (vdbg_coalescer_*), against the oracle.

vdb calls Index::search once per query from its pool workers (src/engine/collection_impl.cc:
1120-1130) and once per segment for each (:1060-1073).  A coalescer gathers such concurrent
calls into device batches; every call must still return exactly the one-query answer:
FlatIndex::search (src/index/flat_index.cc:11-39), Sq8Index's scan with rerank
(src/index/quant/sq8.cc, index.cc:89-95), IvfPqIndex::search (ivf_pq.cc:169-222),
PqFlatIndex::search (ivf_pq.cc:59-79) and HnswSq8Index::search (hnsw_index.cc:82-100), ids,
distances and distance computations, bit for bit with the oracle.  Host threads call through
ctypes (which releases the GIL for the call), and the C++ load driver
(tests/cpp/per_query_load) runs 16 native threads."""
import json
import os
import subprocess
import threading

import numpy as np
import pytest

import vdbg
from ivf_file import synth_ivfpq
from test_ivfpq_gpu import _oracle_ivf
from vdbg import datagen

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden")
DRIVER = os.path.join(HERE, "cpp", "per_query_load")


def _words(n, frac, seed):
    a = np.random.default_rng(seed).random(n) < frac
    w = np.zeros(((n + 63) // 64) * 8, np.uint8)
    b = np.packbits(a, bitorder="little")
    w[:b.size] = b
    return w.view(np.uint64)


def _run_threads(co, qs, calls, nthreads=16):
    """calls: list of (query index, k, param, rerank, allow); returns results in that order."""
    out = [None] * len(calls)
    errs = []

    def work(t):
        try:
            for i in range(t, len(calls), nthreads):
                qi, k, param, rerank, allow = calls[i]
                out[i] = co.search(qs[qi], k, param, rerank, allow)
        except Exception as e:  # surfaced below
            errs.append(e)

    th = [threading.Thread(target=work, args=(t,)) for t in range(nthreads)]
    for t in th:
        t.start()
    for t in th:
        t.join()
    assert not errs, errs[0]
    return out


def _check(got, want_i, want_d, want_dc=None, what=""):
    ids, d, dc = got
    assert np.array_equal(ids, want_i), (what, ids.tolist(), want_i.tolist())
    assert np.array_equal(d.view(np.uint32), want_d.view(np.uint32)), what
    if want_dc is not None:
        assert dc == want_dc, (what, dc, want_dc)


@pytest.mark.parametrize("data", ["int", "float"])
def test_flat_calls_match_oracle(ctx, oracle, data):
    print(f"coalesced flat {data}", flush=True)
    n, dim = 20000, 64
    if data == "int":
        base = datagen.sift_like(n, dim, 3101)
        qs = datagen.sift_like(48, dim, 3102)
    else:
        base = datagen.uniform_rows(n, dim, 3103)
        qs = datagen.uniform_rows(48, dim, 3104)
    ds = vdbg.Dataset(ctx, base, dim)
    allow = _words(n, 0.3, 3105)
    co = vdbg.Coalescer(ds, max_batch=8, max_wait_us=200)
    try:
        calls = [(i, k, 0, 0, a) for i in range(48) for k in (1, 10) for a in (None, allow)]
        got = _run_threads(co, qs, calls)
        for (qi, k, _, _, a), g in zip(calls, got):
            od, oi = oracle.flat_search(base, qs[qi:qi + 1], k, kset=ctx.kernels, allow=a)
            _check(g, oi[0], od[0], n, (data, qi, k, a is not None))
        b, q = co.stats()
        assert q == len(calls) and b <= q
    finally:
        co.close()
        ds.close()


def test_sq8_and_pqflat_calls_match_oracle(ctx, oracle):
    print("coalesced sq8 / pq-flat", flush=True)
    n, dim = 12000, 64
    base = datagen.sift_like(n, dim, 3201)
    qs = datagen.sift_like(32, dim, 3202)
    ds = vdbg.Dataset(ctx, base, dim)
    sq = vdbg.Sq8Index(ds)
    co = vdbg.Coalescer(sq, max_batch=16, max_wait_us=100)
    allow = _words(n, 0.5, 3203)
    try:
        calls = [(i, k, depth, 0, a) for i in range(32) for k, depth in ((10, 100), (5, 0))
                 for a in (None, allow)]
        got = _run_threads(co, qs, calls)
        codes = sq.codes()
        for (qi, k, depth, _, a), g in zip(calls, got):
            od, oi = oracle.sq8_search(base, codes, sq.vmin, sq.scale, qs[qi:qi + 1], k, depth,
                                       kset=ctx.kernels, allow=a)
            _check(g, oi[0], od[0], None, ("sq8", qi, k, depth))
    finally:
        co.close()
        sq.close()
    ix = vdbg.PqFlatIndex.build(ds, 8, seed=42)
    co = vdbg.Coalescer(ix, max_batch=16, max_wait_us=100)
    try:
        calls = [(i, k, 0, rr, a) for i in range(32) for k, rr in ((10, -1), (3, 0))
                 for a in (None, allow)]
        got = _run_threads(co, qs, calls)
        for (qi, k, _, rr, a), g in zip(calls, got):
            wi, wd, wdc = ix.search(qs[qi:qi + 1], k, rr, a)  # the one-query call
            _check(g, wi[0], wd[0], int(wdc[0]), ("pqflat", qi, k, rr))
    finally:
        co.close()
        ix.close()
        ds.close()


def test_ivfpq_calls_match_oracle(ctx, oracle):
    print("coalesced ivf-pq", flush=True)
    base = datagen.sift_like(30000, 128, 2002)
    qs = datagen.sift_like(24, 128, 2003)
    blob = synth_ivfpq(base, 128, 128, 16, seed=1)
    ds = vdbg.Dataset(ctx, base, 128)
    ix = vdbg.IvfPqIndex.load(ds, blob)
    co = vdbg.Coalescer(ix, max_batch=12, max_wait_us=100)
    try:
        calls = [(i, k, nprobe, rr, None) for i in range(24)
                 for k, nprobe, rr in ((10, 16, 0), (10, 8, -1), (20, 32, 100))]
        got = _run_threads(co, qs, calls, nthreads=12)
        for (qi, k, nprobe, rr, _), g in zip(calls, got):
            od, oi, odc = _oracle_ivf(oracle, blob, base, qs[qi:qi + 1], k, nprobe, rr)
            _check(g, oi[0], od[0], int(odc[0]), ("ivfpq", qi, k, nprobe, rr))
    finally:
        co.close()
        ix.close()
        ds.close()


def test_hnsw_calls_match_oracle(ctx, oracle):
    print("coalesced hnsw-sq8", flush=True)
    g = np.load(os.path.join(GOLD, "hnsw.npz"))
    ks = str(g["kernels"])
    ctx.set_kernels(ks)
    rows = np.ascontiguousarray(g["c_rows"], np.float32)
    metric = ["l2", "ip", "cosine"][int(g["c_metric"])]
    dim = int(g["c_dim"])
    f = g["c_file"].tobytes()
    ds = vdbg.Dataset(ctx, rows, dim, metric)
    sq = vdbg.Sq8Index.load(ds, f)
    co = vdbg.Coalescer(sq, max_batch=16, max_wait_us=100, hnsw=True)
    rng = np.random.default_rng(3301)
    n = rows.shape[0]
    qs = rows[rng.integers(0, n, 24)].copy()
    qs[:, :dim] += rng.standard_normal((24, dim)).astype(np.float32) * 0.1
    if metric == "cosine":
        qs /= np.linalg.norm(qs, axis=1, keepdims=True)
    allow = _words(n, 0.5, 3302)
    try:
        calls = [(i, k, ef, rr, a) for i in range(24) for k, ef, rr in ((10, 64, -1), (5, 16, 0))
                 for a in (None, allow)]
        got = _run_threads(co, qs, calls)
        for (qi, k, ef, rr, a), gg in zip(calls, got):
            od, oi, odc = oracle.hnsw_sq8_search(f, rows, qs[qi:qi + 1], k, ef, rr, metric=metric,
                                                 allow=a, kset=ks)
            _check(gg, oi[0], od[0], int(odc[0]), ("hnsw", qi, k, ef, rr))
    finally:
        co.close()
        sq.close()
        ds.close()


def test_coalescer_arguments(ctx):
    ds = vdbg.Dataset(ctx, np.ones((100, 16), np.float32), 16)
    try:
        for mb, w in ((0, 10), (5000, 10), (4, 2_000_000)):
            with pytest.raises(vdbg.VdbgError) as e:
                vdbg.Coalescer(ds, max_batch=mb, max_wait_us=w)
            assert e.value.code == 1
        co = vdbg.Coalescer(ds, max_batch=1, max_wait_us=0)
        ids, d, dc = co.search(np.ones(16, np.float32), 3)
        assert ids.tolist()[:1] == [0] and dc == 100
        with pytest.raises(vdbg.VdbgError) as e:
            co.search(np.ones(16, np.float32), 10001)
        assert e.value.code == 1
        co.close()
    finally:
        ds.close()


def test_load_driver_16_threads_matches_oracle(oracle, tmp_path):
    """The native load driver: 16 threads of one-query calls on 50,000 x 96 integer rows;
    every query's coalesced answer equals the oracle's and the batched call's."""
    print("per_query_load 16 threads", flush=True)
    n, dim, nq, k = 50000, 96, 256, 10
    base = datagen.sift_like(n, dim, 3401)
    qs = datagen.sift_like(nq, dim, 3402)
    data = tmp_path / "rows.f32"
    with open(data, "wb") as fh:
        fh.write(np.ascontiguousarray(base[:, :dim]).tobytes())
        fh.write(np.ascontiguousarray(qs[:, :dim]).tobytes())
    out = tmp_path / "res.bin"
    r = subprocess.run([DRIVER, "--rows", str(n), "--dim", str(dim), "--queries", str(nq),
                        "--threads", "16", "--k", str(k), "--max-batch", "16", "--wait-us", "50",
                        "--seconds", "0.5", "--data", str(data), "--out", str(out)],
                       capture_output=True, text=True, timeout=110)
    assert r.returncode == 0, r.stderr
    rep = json.loads(r.stdout.strip().splitlines()[-1])
    assert rep["differ_from_batch"] == 0 and rep["queries_done"] > 0
    raw = np.fromfile(out, np.uint32)
    ids = raw[:nq * k].reshape(nq, k)
    d = raw[nq * k:].view(np.float32).reshape(nq, k)
    od, oi = oracle.flat_search(base, qs, k)
    assert np.array_equal(ids, oi)
    assert np.array_equal(d.view(np.uint32), od.view(np.uint32))
