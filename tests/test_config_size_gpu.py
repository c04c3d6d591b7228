"""Parity at the bench's own size: 1M x 128 SIFT-like rows and its 10,000 queries (oracle
checks on query subsets where the CPU restatement would take minutes).

- SQ8 training and encoding of all 1M rows, byte for byte against the oracle's encoder
  (Sq8Quantizer::train / encode, src/index/quant/sq8.cc:11-37).
- The IVF-PQ build at nlist 4,096, m 16 (IvfPqIndex::build, src/index/quant/ivf_pq.cc:
  102-149): a strided subset of the rows is re-assigned by the oracle's AssignNearest
  against the built coarse centroids (kmeans.cc:16-55) and re-encoded by its PQ encoder
  on the residual (pq.cc:43-57, ivf_pq.cc:128-139) against the built codebook; both must
  equal what the file holds.  (A reference build of the k-means itself at this size is
  beyond the CPU budget of a test; centroids are pinned bit for bit at the golden size in
  test_build_gpu.py.)
- Every point of the bench's sweeps: flat batches 1, 2, 8, 64, 1,024 at k = 10 and k = 100,
  IVF-PQ nprobe 16 / 32 / 64 / 128 x rerank 0 / 100, ids, distances and distance counts
  against the oracle.
- The bench's own calls at full batch: the flat headline (10,000 queries, k = 10, and the
  k = 100 sweep point) and the SQ8 scan (depth 100, k = 10), each checked on 64 queries
  spread over the whole batch, its last query tile included.
- vdb's own IVF-PQ build at this size (its fixed 25 k-means iterations): the GPU build writes
  the reference's file (tests/golden/ivf1m.npz holds its length, CRC32C and digests).
- A collection shaped as the filtered benchmark: 384-dim cosine rows in 8 segments of
  100,000, 2 % deleted, filters of 1 / 10 / 50 %, merged, against the oracle's composition."""
import os

import numpy as np
import pytest

import vdbg
from ivf_file import parse_ivfpq
from oracle_lib import KSET
from vdbg import datagen

pytestmark = pytest.mark.gpu
N, DIM = 1_000_000, 128


@pytest.fixture(scope="module")
def big(ctx):
    print("config-size: generating 1M x 128 rows", flush=True)
    base = datagen.sift_like(N, DIM, 2002)
    qs = datagen.sift_like(10000, DIM, 2003)
    ds = vdbg.Dataset(ctx, base, DIM)
    yield base, qs, ds
    ds.close()


@pytest.fixture(scope="module")
def ivf(big, oracle):
    base, qs, ds = big
    print("config-size: building IVF-PQ nlist 4096 m 16", flush=True)
    ix = vdbg.IvfPqIndex.build(ds, nlist=4096, m=16, seed=42, max_points=256, iters=20)
    f = parse_ivfpq(ix.save())
    f["term2"] = np.empty(f["nlist"] * f["m"] * 256, np.float32)
    oracle.lib.or_ivfpq_term2(f["coarse"], f["nlist"], f["pd"], f["pq_centroids"], f["m"],
                              DIM // f["m"], f["term2"])
    yield ix, f
    ix.close()


def _eq(gi, gd, oi, od):
    bad = np.nonzero((gi != oi).any(1) | (gd.view(np.uint32) != od.view(np.uint32)).any(1))[0]
    assert bad.size == 0, (f"{bad.size} queries differ; q={bad[0]} gpu={gi[bad[0]].tolist()} "
                           f"oracle={oi[bad[0]].tolist()}")


def test_sq8_encode_1m_matches_oracle(big, oracle):
    base, _, ds = big
    sq = vdbg.Sq8Index(ds)
    vmin, scale = oracle.sq8_train(base, DIM)
    assert np.array_equal(sq.vmin.view(np.uint32), vmin.view(np.uint32))
    assert np.array_equal(sq.scale.view(np.uint32), scale.view(np.uint32))
    codes = oracle.sq8_encode(base, DIM, vmin, scale)
    got = sq.codes()
    bad = np.nonzero((got != codes).any(1))[0]
    assert bad.size == 0, f"{bad.size} rows encode differently, first {bad[:5].tolist()}"
    sq.close()


def test_ivfpq_build_1m_assignment_and_codes(big, ivf, oracle):
    base, _, _ = big
    _, f = ivf
    nlist, m, pd = f["nlist"], f["m"], f["pd"]
    dsub = DIM // m
    off = f["list_off"].astype(np.int64)
    assert off[-1] == N and np.array_equal(np.sort(f["list_ids"]), np.arange(N, dtype=np.uint32))
    pos = np.arange(0, N, 97)  # a strided subset of the CSR positions
    rows = f["list_ids"][pos]
    lists = np.searchsorted(off, pos, side="right") - 1
    sub = np.ascontiguousarray(base[rows])
    assign = np.empty(len(rows), np.uint32)
    oracle.lib.or_assign_nearest(KSET["avx512"], sub, len(rows), DIM, pd,
                                 np.ascontiguousarray(f["coarse"]), nlist, assign, None, 8)
    wrong = np.nonzero(assign != lists)[0]
    assert wrong.size == 0, f"{wrong.size} rows in another list, first row {rows[wrong[0]]}"
    cen = np.ascontiguousarray(f["pq_centroids"])
    code = np.empty(m, np.uint8)
    codes = f["list_codes"].reshape(-1, m)
    for p, r, l in zip(pos, rows, lists):
        resid = np.ascontiguousarray((base[r, :DIM] - f["coarse"][l, :DIM]).astype(np.float32))
        oracle.lib.or_pq_encode(cen, m, dsub, resid, code)
        assert np.array_equal(code, codes[p]), f"row {r}: {code.tolist()} vs {codes[p].tolist()}"


@pytest.mark.parametrize("nq,k", [(1, 10), (2, 10), (8, 10), (64, 10), (1024, 10), (1024, 100)])
def test_flat_sweep_points_match_oracle(big, oracle, nq, k):
    base, qs, ds = big
    q = np.ascontiguousarray(qs[:nq])
    gi, gd = ds.flat_search(q, k)
    s = min(nq, 64)  # the oracle checks up to 64 queries of the batch
    od, oi = oracle.flat_search(base, q[:s], k, threads=16)
    _eq(gi[:s], gd[:s], oi, od)


@pytest.mark.parametrize("nprobe", [16, 32, 64, 128])
@pytest.mark.parametrize("rerank", [0, 100])
def test_ivfpq_sweep_points_match_oracle(big, ivf, oracle, nprobe, rerank):
    base, qs, _ = big
    ix, f = ivf
    q = np.ascontiguousarray(qs[:2000])
    gi, gd, dc = ix.search(q, 10, nprobe, rerank)
    s = 500
    od, oi, odc = oracle.ivfpq_search(f, f["term2"], base, q[:s], 10, nprobe, rerank)
    _eq(gi[:s], gd[:s], oi, od)
    assert np.array_equal(dc[:s], odc)


def _spread(nq, count=64):
    """count query positions over a batch of nq: evenly spaced from the first to the last,
    and the last 8 (the batch's last query tile)."""
    return np.unique(np.concatenate([np.linspace(0, nq - 1, count - 8).astype(np.int64),
                                     np.arange(nq - 8, nq)]))


@pytest.mark.parametrize("k", [10, 100])
def test_flat_headline_batch_matches_oracle(big, oracle, k):
    """The headline call as the bench makes it: all 10,000 queries in one batch."""
    base, qs, ds = big
    print(f"config-size: flat 10,000 queries k={k}", flush=True)
    gi, gd = ds.flat_search(qs, k)
    sel = _spread(len(qs))
    od, oi = oracle.flat_search(base, np.ascontiguousarray(qs[sel]), k, threads=16)
    _eq(gi[sel], gd[sel], oi, od)


def test_sq8_search_1m_matches_oracle(big, oracle):
    """The SQ8 path as the bench runs it: every 1M code scanned for 10,000 queries, the top
    100 reranked to 10 (Sq8Quantizer + TopK + Rerank, index.cc:89-95)."""
    base, qs, ds = big
    print("config-size: SQ8 10,000 queries depth 100", flush=True)
    sq = vdbg.Sq8Index(ds)
    try:
        gi, gd = sq.search(qs, 10, 100)
        sel = _spread(len(qs))
        od, oi = oracle.sq8_search(base, sq.codes(), sq.vmin, sq.scale,
                                   np.ascontiguousarray(qs[sel]), 10, 100, threads=16)
        _eq(gi[sel], gd[sel], oi, od)
    finally:
        sq.close()


def test_ivfpq_build_1m_is_vdbs_own_build(big):
    """IvfPqIndex::build (ivf_pq.cc:102-149) at vdb's fixed 25 k-means iterations
    (kmeans.h:14, kmeans.cc:57-174) over the 1M rows writes the file vdb's own build wrote:
    the same list sizes, coarse centroids, codebook, list ids and codes, length and CRC32C
    (recorded from the reference's build by tests/golden/make_golden.py ivf1m)."""
    import hashlib
    base, _, ds = big
    z = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ivf1m.npz"))
    print("config-size: IVF-PQ build at 25 iterations", flush=True)
    ix = vdbg.IvfPqIndex.build(ds, nlist=4096, m=16, seed=42, max_points=256, iters=25)
    try:
        f = ix.save()
    finally:
        ix.close()
    p = parse_ivfpq(f)
    sha = lambda a: np.frombuffer(hashlib.sha256(np.ascontiguousarray(a).tobytes()).digest(),
                                  np.uint8)
    sizes = np.diff(p["list_off"].astype(np.int64)).astype(np.uint32)
    diff = np.nonzero(sizes != z["list_sizes"])[0]
    assert diff.size == 0, f"{diff.size} lists differ in size, first list {diff[:5].tolist()}"
    assert np.array_equal(sha(p["coarse"]), z["coarse_sha"]), "coarse centroids differ"
    assert np.array_equal(sha(p["pq_centroids"]), z["codebook_sha"]), "codebook differs"
    assert np.array_equal(sha(p["list_ids"]), z["ids_sha"]), "list ids differ"
    assert np.array_equal(sha(p["list_codes"]), z["codes_sha"]), "codes differ"
    assert len(f) == int(z["file_len"])
    assert int.from_bytes(f[-4:], "little") == int(z["file_crc"])


def test_filtered_collection_at_benchmark_shape(ctx, oracle):
    """The filtered benchmark's shape at 100,000 rows per segment: 384-dim unit rows from the
    10,000-centre mixture in 8 segments, 2 % deleted, the bucket filters at 1 / 10 / 50 %
    and no filter, k = 10, 32 raw queries prepared on the device, each segment planned and
    searched, merged by (dist, part, row)."""
    import torch

    dim, nseg, seg_n, nq, k = 384, 8, 100_000, 32, 10
    dev = torch.device("cuda:0")
    print("config-size: filtered collection 8 x 100,000 x 384", flush=True)
    dss, segs = [], []
    N = nseg * seg_n
    deleted = datagen.uniform01(5004, 0, N) < np.float32(0.02)
    bucket = datagen.rand_u64(5006, 0, N) % np.uint64(100)

    def words(bits):
        w = np.zeros((bits.size + 63) // 64 * 8, np.uint8)
        b = np.packbits(bits, bitorder="little")
        w[:b.size] = b
        return w.view(np.uint64)

    try:
        for p in range(nseg):
            rows = datagen.clustered_unit_t(torch, seg_n, dim, 5002, 5001, 10000, 1.0, dev,
                                            start_row=p * seg_n)
            ds = vdbg.Dataset.from_device(ctx, rows.data_ptr(), seg_n, dim, dim, "cosine")
            ext = np.arange(p * seg_n, (p + 1) * seg_n, dtype=np.uint64)
            ds.set_external_ids(ext)
            dss.append(ds)
            segs.append({"base": rows.cpu().numpy(), "ext": ext, "kind": "flat",
                         "deleted": words(deleted[p * seg_n:(p + 1) * seg_n])})
            del rows
        raw = datagen.clustered_unit_t(torch, nq, dim, 5005, 5001, 10000, 1.0, dev,
                                       unit=False).cpu().numpy()
        for sel in (None, 1, 10, 50):
            for p, sg in enumerate(segs):
                sg["filter"] = None if sel is None else words(
                    bucket[p * seg_n:(p + 1) * seg_n] < np.uint64(sel))
            print(f"config-size: filtered collection selectivity {sel}", flush=True)
            gi, gd, gdc, gp = vdbg.collection_search(
                ctx, [(ds, None, sg["deleted"], sg["filter"]) for ds, sg in zip(dss, segs)],
                dim, "cosine", raw, k)
            oi, od, odc, op = oracle.collection_search(segs, dim, "cosine", raw, k)
            assert gp == op
            assert gp == (["index"] if sel is None else ["prefilter_exact"]) * nseg
            bad = np.nonzero((gi != oi).any(1) | (gd.view(np.uint32) != od.view(np.uint32)).any(1))[0]
            assert bad.size == 0, (sel, bad[:5])
            assert np.array_equal(gdc, odc)
    finally:
        for ds in dss:
            ds.close()
