"""PqFlatIndex on the GPU (vdbg_pqflat_*): src/index/quant/ivf_pq.cc:41-98.

Files and results come from the reference (tests/golden/pqflat.npz: VDBPQFL1 files its
PqFlatIndex::build + save wrote, and what its PqFlatIndex::search returned on them).  A GPU
build over the same rows must write the same file byte for byte; searches must return the
recorded ids, distances and distance computations; random cases are compared with the
oracle's restatement, which the same fixtures pin."""
import os
import struct

import numpy as np
import pytest

import vdbg
from ivf_file import parse_pqflat

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def gold():
    return np.load(os.path.join(GOLD, "pqflat.npz"))


@pytest.mark.parametrize("tag", ["a", "b", "c"])
def test_loaded_file_matches_reference_results(ctx, tag):
    g = gold()
    ctx.set_kernels(str(g["kernels"]))
    rows, q, metric = g[f"{tag}_rows"], g[f"{tag}_q"], str(g[f"{tag}_metric"])
    dim = int(g[f"{tag}_dim"])
    print(f"pqflat golden {tag} n={rows.shape[0]} dim={dim} {metric}", flush=True)
    ds = vdbg.Dataset(ctx, rows, dim, metric)
    ix = vdbg.PqFlatIndex.load(ds, g[f"{tag}_file"].tobytes())
    assert np.array_equal(ix.codes(), parse_pqflat(g[f"{tag}_file"].tobytes())["codes"])
    for fi, allow in enumerate((None, g[f"{tag}_allow"])):
        for si, (k, rr) in enumerate(g["settings"]):
            ids, d, dc = ix.search(q, int(k), int(rr), allow)
            key = f"{tag}_f{fi}_s{si}"
            assert np.array_equal(ids, g[key + "_i"]), key
            assert np.array_equal(d.view(np.uint32), g[key + "_d"].view(np.uint32)), key
            assert np.array_equal(dc, g[key + "_dc"]), key
    assert ix.save() == g[f"{tag}_file"].tobytes()
    ix.close()
    ds.close()


@pytest.mark.parametrize("tag", ["a", "b", "c"])
def test_gpu_build_writes_the_reference_file(ctx, tag):
    """ProductQuantizer::train (the same libstdc++ sampling, k-means on the GPU) and encode:
    the VDBPQFL1 file of a GPU build is the reference's byte for byte."""
    g = gold()
    rows, metric, dim = g[f"{tag}_rows"], str(g[f"{tag}_metric"]), int(g[f"{tag}_dim"])
    m = parse_pqflat(g[f"{tag}_file"].tobytes())["m"]
    print(f"pqflat build {tag} m={m}", flush=True)
    ds = vdbg.Dataset(ctx, rows, dim, metric)
    ix = vdbg.PqFlatIndex.build(ds, m, seed=42)
    assert ix.save() == g[f"{tag}_file"].tobytes()
    ix.close()
    ds.close()


def test_random_queries_match_oracle(ctx, oracle):
    g = gold()
    ks = str(g["kernels"])
    ctx.set_kernels(ks)
    rng = np.random.default_rng(5)
    for tag in ("a", "b", "c"):
        rows, metric, dim = g[f"{tag}_rows"], str(g[f"{tag}_metric"]), int(g[f"{tag}_dim"])
        f = g[f"{tag}_file"].tobytes()
        pix = parse_pqflat(f)
        n, pd = rows.shape
        ds = vdbg.Dataset(ctx, rows, dim, metric)
        ix = vdbg.PqFlatIndex.load(ds, f)
        q = rows[rng.integers(0, n, 40)] + np.float32(0.05) * (np.arange(pd) < dim)
        for k, rr in ((10, -1), (1, 0), (25, -1), (7, 300), (100, 0), (40, 2000)):
            for frac in (None, 0.3, 0.002):
                allow = None
                if frac is not None:
                    a = rng.random(n) < frac
                    w = np.zeros(((n + 63) // 64) * 8, np.uint8)
                    b = np.packbits(a, bitorder="little")
                    w[:b.size] = b
                    allow = w.view(np.uint64)
                ids, d, dc = ix.search(q, k, rr, allow)
                od, oi, odc = oracle.pqflat_search(pix, rows, q, k, rr, metric, allow, kset=ks)
                assert np.array_equal(ids, oi), (tag, k, rr, frac)
                assert np.array_equal(d.view(np.uint32), od.view(np.uint32)), (tag, k, rr, frac)
                assert np.array_equal(dc, odc), (tag, k, rr, frac)
        ix.close()
        ds.close()


def test_bad_files_and_arguments(ctx):
    g = gold()
    rows, dim = g["a_rows"], int(g["a_dim"])
    f = g["a_file"].tobytes()
    ds = vdbg.Dataset(ctx, rows, dim)
    other = vdbg.Dataset(ctx, rows[:-1], dim)

    def expect(d, data, msg):
        with pytest.raises(vdbg.VdbgError) as e:
            vdbg.PqFlatIndex.load(d, data)
        assert e.value.code == 5 and msg in str(e.value), str(e.value)

    def refile(b):
        return b + struct.pack("<I", vdbg.crc32c(b))

    expect(ds, f[:11], "too short")
    expect(ds, f[:-1] + bytes([f[-1] ^ 1]), "checksum mismatch")
    expect(ds, refile(b"VDBIVFP1" + f[8:-4]), "not a pq-flat index file")
    expect(other, f, "does not match the segment")
    expect(ds, refile(f[:24 + 100]), "does not match the segment")  # codebook cut
    expect(ds, refile(f[:-4 - 10]), "truncated pq codes")
    b = bytearray(f[:-4])
    struct.pack_into("<I", b, 20, 0)  # m = 0
    expect(ds, refile(bytes(b)), "does not match the segment")
    with pytest.raises(vdbg.VdbgError) as e:
        vdbg.PqFlatIndex.build(ds, 7)  # 7 does not divide 32
    assert e.value.code == 1 and "pq_m must divide" in str(e.value)
    ds.close()
    other.close()


def test_empty_segment(ctx):
    ds = vdbg.Dataset(ctx, np.zeros((0, 32), np.float32), 32)
    ix = vdbg.PqFlatIndex.build(ds, 8)
    ids, d, dc = ix.search(np.ones((3, 32), np.float32), 5)
    assert (ids == 0xFFFFFFFF).all() and np.isinf(d).all() and (dc == 0).all()
    ix.close()
    ds.close()
