"""HnswSq8Index segments on the GPU backend: the graph of a VDBHSQ81 file walked on the host
(HnswGraph::search, src/index/hnsw/hnsw_graph.h:301-324, 467-548) and each query's beam
reranked on the GPU (hnsw_index.cc:82-100, index.cc:89-95).

Expected results are the reference's own: tests/golden/hnsw.npz holds files its
HnswSq8Index::build + save wrote and the ids, distances and distance computations its
HnswSq8Index::search returned for them, per (k, ef, rerank) setting, without a filter and
under RowFilters allowing ~98 %, ~30 % and ~2 % of the rows.  Random queries beyond those are
compared with the oracle's restatement, which the same fixtures pin."""
import os
import struct

import numpy as np
import pytest

import vdbg

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
METRICS = ["l2", "ip", "cosine"]


def gold():
    return np.load(os.path.join(GOLD, "hnsw.npz"))


def case(g, tag):
    rows = np.ascontiguousarray(g[f"{tag}_rows"], np.float32)
    return (rows, g[f"{tag}_q"], METRICS[int(g[f"{tag}_metric"])], int(g[f"{tag}_dim"]),
            g[f"{tag}_file"].tobytes())


@pytest.fixture(scope="module")
def loaded(ctx):
    g = gold()
    ctx.set_kernels(str(g["kernels"]))
    out = {}
    for tag in ("c", "d", "e"):
        rows, q, metric, dim, f = case(g, tag)
        ds = vdbg.Dataset(ctx, rows, dim, metric)
        sq = vdbg.Sq8Index.load(ds, f)
        out[tag] = (ds, sq)
    yield g, out
    for ds, sq in out.values():
        sq.close()
        ds.close()


@pytest.mark.parametrize("tag", ["c", "d", "e"])
def test_matches_reference_recorded_results(ctx, loaded, tag):
    g, h = loaded
    rows, q, metric, dim, f = case(g, tag)
    ds, sq = h[tag]
    print(f"hnsw golden {tag} n={rows.shape[0]} dim={dim} {metric}", flush=True)
    for fi in range(4):
        allow = g[f"{tag}_allow{fi}"] if fi else None
        for si, (k, ef, rr) in enumerate(g["settings"]):
            ids, d, dc = sq.hnsw_search(q, int(k), int(ef), int(rr), allow)
            key = f"{tag}_f{fi}_s{si}"
            assert np.array_equal(ids, g[key + "_i"]), key
            assert np.array_equal(d.view(np.uint32), g[key + "_d"].view(np.uint32)), key
            assert np.array_equal(dc, g[key + "_dc"]), key


def test_graph_info(loaded):
    g, h = loaded
    for tag, (ds, sq) in h.items():
        n, M, efc, top, ep = sq.graph_info()
        f = g[f"{tag}_file"].tobytes()
        assert n == ds.n and M == {"c": 16, "d": 12, "e": 8}[tag] and top >= 1 and 0 <= ep < n
        assert efc == {"c": 100, "d": 80, "e": 40}[tag]


@pytest.mark.parametrize("tag", ["c", "d", "e"])
def test_random_queries_match_oracle(ctx, oracle, loaded, tag):
    g, h = loaded
    rows, q, metric, dim, f = case(g, tag)
    ds, sq = h[tag]
    rng = np.random.default_rng(77)
    n, pd = rows.shape
    qs = rows[rng.integers(0, n, 64)].copy()
    qs[:, :dim] += rng.standard_normal((64, dim)).astype(np.float32) * (4 if metric == "l2" else 0.1)
    if metric == "cosine":
        qs /= np.linalg.norm(qs, axis=1, keepdims=True)
    ks = str(g["kernels"])
    for k, ef, rr in ((10, 64, -1), (1, 1, -1), (25, 100, 40), (7, 9, 0), (300, 16, -1)):
        allow = None
        for frac in (None, 0.5):
            if frac is not None:
                a = rng.random(n) < frac
                w = np.zeros(((n + 63) // 64) * 8, np.uint8)
                b = np.packbits(a, bitorder="little")
                w[:b.size] = b
                allow = w.view(np.uint64)
            ids, d, dc = sq.hnsw_search(qs, k, ef, rr, allow)
            od, oi, odc = oracle.hnsw_sq8_search(f, rows, qs, k, ef, rr, metric=metric,
                                                 allow=allow, kset=ks)
            assert np.array_equal(ids, oi), (k, ef, rr, frac)
            assert np.array_equal(d.view(np.uint32), od.view(np.uint32)), (k, ef, rr, frac)
            assert np.array_equal(dc, odc), (k, ef, rr, frac)


def test_device_form_and_threads_agree(ctx, loaded):
    import torch
    g, h = loaded
    rows, q, metric, dim, f = case(g, "c")
    ds, sq = h["c"]
    allow = g["c_allow2"]
    want = sq.hnsw_search(q, 10, 32, 50, allow)
    for threads in (1, 3, 0):
        ctx.set_host_threads(threads)
        got = sq.hnsw_search(q, 10, 32, 50, allow)
        assert all(np.array_equal(a, b) for a, b in zip(want, got)), threads
    dev = torch.device("cuda:0")
    qd = torch.from_numpy(q).to(dev)
    ad = torch.from_numpy(allow.view(np.int64)).to(dev)
    for rr in (50, 0):
        wi, wd, wdc = sq.hnsw_search(q, 10, 32, rr, allow)
        ids = torch.empty((len(q), 10), dtype=torch.int32, device=dev)
        dd = torch.empty((len(q), 10), dtype=torch.float32, device=dev)
        dc = torch.empty(len(q), dtype=torch.int64, device=dev)
        sq.hnsw_search_device(qd.data_ptr(), len(q), 10, 32, rr, ids.data_ptr(), dd.data_ptr(),
                              allow_ptr=ad.data_ptr(), dc_ptr=dc.data_ptr(),
                              stream=torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert np.array_equal(ids.cpu().numpy().view(np.uint32), wi)
        assert np.array_equal(dd.cpu().numpy().view(np.uint32), wd.view(np.uint32))
        assert np.array_equal(dc.cpu().numpy().view(np.uint64), wdc)


def test_every_kernel_set(ctx, oracle, loaded):
    g, h = loaded
    rows, q, metric, dim, f = case(g, "d")
    ds, sq = h["d"]
    try:
        for ks in ("scalar", "avx2", "avx512"):
            ctx.set_kernels(ks)
            ids, d, dc = sq.hnsw_search(q, 10, 40, -1)
            od, oi, odc = oracle.hnsw_sq8_search(f, rows, q, 10, 40, -1, metric=metric, kset=ks)
            assert np.array_equal(ids, oi) and np.array_equal(d.view(np.uint32), od.view(np.uint32))
            assert np.array_equal(dc, odc), ks
    finally:
        ctx.set_kernels(str(g["kernels"]))


def test_created_index_has_no_graph(ctx, loaded):
    g, h = loaded
    rows, q, metric, dim, f = case(g, "e")
    ds, _ = h["e"]
    sq = vdbg.Sq8Index(ds)
    with pytest.raises(vdbg.VdbgError) as e:
        sq.hnsw_search(q, 10)
    assert e.value.code == 6
    with pytest.raises(vdbg.VdbgError) as e:
        sq.graph_info()
    assert e.value.code == 6
    sq.close()


def test_bad_graphs_are_corruption(ctx):
    """HnswGraph::Deserialize's checks (hnsw_graph.h:368-413) and their messages."""
    g = gold()
    rows, q, metric, dim, f = case(g, "e")
    n, pd = rows.shape
    ds = vdbg.Dataset(ctx, rows, dim, metric)
    gs = 8 + 8 + 8 + 8 * pd + n * pd  # where the graph starts
    body = bytearray(f[:-4])
    hdr = struct.unpack_from("<QQIIQII", body, gs)
    lvl0 = gs + 40

    def refile(b):
        b = bytes(b)
        return b + struct.pack("<I", vdbg.crc32c(b))

    def expect(b, msg):
        with pytest.raises(vdbg.VdbgError) as e:
            vdbg.Sq8Index.load(ds, refile(b))
        assert e.value.code == 5 and msg in str(e.value), str(e.value)

    expect(body[:gs + 20], "truncated hnsw header")
    b = bytearray(body)
    struct.pack_into("<I", b, gs + 16, 1)  # M = 1
    expect(b, "hnsw header does not match the segment")
    b = bytearray(body)
    struct.pack_into("<I", b, gs + 36, n)  # entry point past the rows
    expect(b, "bad hnsw entry point")
    b = bytearray(body)
    struct.pack_into("<I", b, gs + 32, 16)  # top layer above kMaxLevel
    expect(b, "bad hnsw entry point")
    expect(body[:lvl0 + n // 2], "truncated hnsw levels")
    expect(body[:lvl0 + n + 100], "truncated hnsw layer 0")
    M0 = 2 * hdr[2]
    b = bytearray(body)
    struct.pack_into("<I", b, lvl0 + n, M0 + 1)  # node 0 with more links than M0
    expect(b, "bad link count")
    b = bytearray(body)
    struct.pack_into("<I", b, lvl0 + n, 1)
    struct.pack_into("<I", b, lvl0 + n + 4, n + 5)  # a link past the rows
    expect(b, "bad link target")
    top = max(1, hdr[5])
    lv = np.frombuffer(bytes(body[lvl0:lvl0 + n]), np.uint8)
    b = bytearray(body)
    b[lvl0 + int(np.argmax(lv == 0))] = top + 1  # a node above the top layer
    expect(b, "node above the top layer")
    up = lvl0 + n + n * (1 + M0) * 4
    expect(body[:up + 8], "truncated hnsw upper layers")
    ds.close()
