"""Concurrent use of the device path and its fallbacks, against the oracle.

vdb calls Index::search concurrently: one call per query from pool workers and one per
segment (src/engine/collection_impl.cc:1069-1073, 1126).  Here several host threads share one
context and queue their searches on two streams, while the certificate fallbacks are forced so
that the exact re-scan of every query is still in flight when each call returns; two
contexts on the device run side by side too.  Every answer must equal the oracle's
FlatIndex::search (src/index/flat_index.cc:11-39) bit for bit.  The forced fallbacks (second
chance, then the exact re-scan) are also checked one by one for flat float rows, integer
rows, SQ8 codes and a filter."""
import threading

import numpy as np
import pytest
import torch

import vdbg
from vdbg import datagen

pytestmark = pytest.mark.gpu


def _eq(gi, gd, oi, od, what=""):
    bad = np.nonzero((gi != oi).any(1) | (gd.view(np.uint32) != od.view(np.uint32)).any(1))[0]
    assert bad.size == 0, (f"{what}: {bad.size} queries differ; q={bad[0]} "
                           f"gpu={gi[bad[0]].tolist()} oracle={oi[bad[0]].tolist()}")


def _launches(c, name):
    return c.profile_get(name)[1]


@pytest.mark.parametrize("data", ["float", "int", "sq8", "filter"])
@pytest.mark.parametrize("level", [1, 2])
def test_forced_fallbacks_match_oracle(oracle, data, level):
    print(f"forced fallbacks data={data} level={level}", flush=True)
    c = vdbg.Context(0)
    try:
        if data == "int":
            base = datagen.sift_like(30000, 128, 2002)
            qs = datagen.sift_like(150, 128, 2003)
        else:
            base = datagen.uniform_rows(30000, 128, 61)
            qs = datagen.uniform_rows(150, 128, 62)
        ds = vdbg.Dataset(c, base, 128)
        allow = None
        if data == "filter":
            allow = np.zeros((30000 + 63) // 64, np.uint64)
            rows = np.arange(0, 30000, 3)
            np.bitwise_or.at(allow, rows // 64, np.uint64(1) << (rows % 64).astype(np.uint64))
        c.profile(True)
        c.profile_reset()
        c.set_test_fallbacks(level)
        if data == "sq8":
            sq = vdbg.Sq8Index(ds)
            gi, gd = sq.search(qs, 10, 100)
            c.set_test_fallbacks(0)
            od, oi = oracle.sq8_search(base, sq.codes(), sq.vmin, sq.scale, qs, 10, 100)
        else:
            gi, gd = ds.flat_search(qs, 10, allow=allow)
            c.set_test_fallbacks(0)
            od, oi = oracle.flat_search(base, qs, 10, allow=allow)
        _eq(gi, gd, oi, od, f"{data} level {level}")
        assert _launches(c, "rescore") >= 1, "the second chance did not run"
        if level == 2:
            assert c.last_fallbacks() == len(qs)
            assert _launches(c, "exact_scan") >= 1
        else:
            assert c.last_fallbacks() == 0
        # and the normal path afterwards still answers the same
        gi2, gd2 = (sq.search(qs, 10, 100) if data == "sq8"
                    else ds.flat_search(qs, 10, allow=allow))
        _eq(gi2, gd2, oi, od, f"{data} after level {level}")
    finally:
        c.close()


def _run_threads(fns):
    errors = []

    def wrap(fn):
        try:
            fn()
        except BaseException as e:  # noqa: BLE001 - reported below
            errors.append(e)

    ts = [threading.Thread(target=wrap, args=(f,)) for f in fns]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    if errors:
        raise errors[0]


def test_one_context_threads_and_two_streams(oracle):
    # 4 threads x 3 calls, alternating between two streams of one context; the exact
    # re-scan is forced so that launches reading the context's scratch are still queued
    # when each call returns and the next call (on the other stream) reuses it
    print("one context, 4 threads, 2 streams, forced exact re-scans", flush=True)
    c = vdbg.Context(0)
    try:
        base = datagen.uniform_rows(40000, 128, 71)
        ds = vdbg.Dataset(c, base, 128)
        c.set_test_fallbacks(2)
        streams = [torch.cuda.Stream(), torch.cuda.Stream()]
        jobs = []
        for t in range(4):
            for r in range(3):
                nq = 40 + 17 * t + 5 * r
                qs = datagen.uniform_rows(nq, 128, 1000 + 10 * t + r)
                jobs.append(dict(qs=qs, nq=nq, stream=streams[(t + r) % 2],
                                 q=torch.from_numpy(qs).cuda(),
                                 ids=torch.empty((nq, 10), dtype=torch.int32, device="cuda"),
                                 d=torch.empty((nq, 10), dtype=torch.float32, device="cuda")))
        torch.cuda.synchronize()

        def worker(mine):
            def run():
                for j in mine:
                    ds.flat_search_device(j["q"].data_ptr(), j["nq"], 10, j["ids"].data_ptr(),
                                          j["d"].data_ptr(), stream=j["stream"].cuda_stream)
            return run

        _run_threads([worker(jobs[3 * t:3 * t + 3]) for t in range(4)])
        torch.cuda.synchronize()
        c.set_test_fallbacks(0)
        for j in jobs:
            od, oi = oracle.flat_search(base, j["qs"], 10)
            gi = j["ids"].cpu().numpy().view(np.uint32)
            gd = j["d"].cpu().numpy()
            _eq(gi, gd, oi, od, f"nq={j['nq']}")
    finally:
        c.close()


def test_two_contexts_side_by_side(oracle):
    print("two contexts in two threads", flush=True)
    ctxs = [vdbg.Context(0), vdbg.Context(0)]
    try:
        bases = [datagen.uniform_rows(25000, 128, 81), datagen.sift_like(25000, 128, 2002)]
        qsets = [datagen.uniform_rows(70, 128, 82), datagen.sift_like(90, 128, 2003)]
        dss = [vdbg.Dataset(ctxs[i], bases[i], 128) for i in range(2)]
        ctxs[0].set_test_fallbacks(2)
        out = [None, None]

        def worker(i):
            def run():
                res = []
                for r in range(3):
                    res.append(dss[i].flat_search(qsets[i], 10))
                out[i] = res
            return run

        _run_threads([worker(0), worker(1)])
        for i in range(2):
            od, oi = oracle.flat_search(bases[i], qsets[i], 10)
            for gi, gd in out[i]:
                _eq(gi, gd, oi, od, f"context {i}")
    finally:
        for c in ctxs:
            c.close()
