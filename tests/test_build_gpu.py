"""Index construction on the GPU against the reference: KMeans and AssignNearest
(src/index/quant/kmeans.cc), ProductQuantizer::train and IvfPqIndex::build
(ivf_pq.cc:102-149).  The reference's seeded construction is deterministic, so the GPU
build must reproduce the reference's centroids and index file bit for bit."""
import os

import numpy as np
import pytest

import vdbg
from ivf_file import parse_ivfpq
from vdbg import datagen

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def bits(x):
    return np.asarray(x, np.float32).view(np.uint32)


def test_assign_nearest_matches_reference(ctx):
    g = np.load(os.path.join(GOLD, "kmeans.npz"), allow_pickle=False)
    a, d = vdbg.assign_nearest(ctx, g["data"], g["centroids_pp"].reshape(40, 16))
    assert np.array_equal(a, g["assign"]) and np.array_equal(bits(d), bits(g["dist"]))


def test_kmeans_matches_reference(ctx):
    g = np.load(os.path.join(GOLD, "kmeans.npz"), allow_pickle=False)
    cen, inertia, _ = vdbg.kmeans(ctx, g["data"], 40, iters=25, seed=1234, max_points=256,
                                  kmeanspp=True)
    assert np.array_equal(bits(cen.ravel()), bits(g["centroids_pp"]))
    cen, _, _ = vdbg.kmeans(ctx, g["data"], 40, iters=10, seed=99, max_points=32, kmeanspp=False)
    assert np.array_equal(bits(cen.ravel()), bits(g["centroids_rand"]))


def test_kmeans_empty_clusters_reseeded(ctx):
    # tests/pq_test.cc:37-50: 3 distinct points, 16 centroids
    n, d = 1000, 4
    data = np.array([[i % 3 + 0.1 * j for j in range(d)] for i in range(n)], np.float32)
    cen, _, reseeds = vdbg.kmeans(ctx, data, 16, kmeanspp=False)
    assert np.isfinite(cen).all() and reseeds > 0


def test_kmeans_fewer_points_than_centroids(ctx):
    data = np.array([[0, 0], [1, 1], [2, 2]], np.float32)
    cen, _, _ = vdbg.kmeans(ctx, data, 8)
    assert cen.shape == (8, 2) and np.array_equal(cen[3], data[0])


def test_ivfpq_build_reproduces_reference_index_file(ctx):
    g = np.load(os.path.join(GOLD, "ivfpq.npz"), allow_pickle=False)
    ds = vdbg.Dataset(ctx, g["base"], 32)
    ix = vdbg.IvfPqIndex.build(ds, nlist=24, m=8, seed=42, max_points=64, iters=25)
    blob = ix.save()
    want = g["index_file"].tobytes()
    if blob != want:
        a, b = parse_ivfpq(blob), parse_ivfpq(want)
        assert np.array_equal(bits(a["coarse"]), bits(b["coarse"])), "coarse centroids differ"
        assert np.array_equal(a["list_off"], b["list_off"]), "list sizes differ"
        assert np.array_equal(bits(a["pq_centroids"]), bits(b["pq_centroids"])), "codebook differs"
        assert np.array_equal(a["list_codes"], b["list_codes"]), "codes differ"
    assert blob == want


def test_ivfpq_build_small_segment_shrinks_nlist(ctx):
    # tests/pq_test.cc:149-157
    base = datagen.pad(np.random.default_rng(10).normal(size=(500, 16)).astype(np.float32), 16)
    ds = vdbg.Dataset(ctx, base, 16)
    ix = vdbg.IvfPqIndex.build(ds, nlist=4096, m=4)
    assert ix.info()[0] == 500 // 39
    assert int(ix.list_sizes().sum()) == 500
