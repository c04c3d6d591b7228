"""The host side of the HNSW-SQ8 path, checked without a GPU: the SQ8 distance the graph
walk computes on the CPU (vdbg_host_sq8_distance), for every kernel set and metric, in both
its instruction and its lane-by-lane form, against bit patterns the reference's own kernels
wrote (src/distance/scalar.cc:25-41, avx2.cc:48-74, avx512.cc:48-64)."""
import os

import numpy as np
import pytest

import vdbg

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.mark.parametrize("portable", [False, True])
@pytest.mark.parametrize("kset", ["scalar", "avx2", "avx512"])
def test_host_sq8_distance_matches_reference_bits(kset, portable):
    g = np.load(os.path.join(GOLD, "distances.npz"))
    for i, d in enumerate(g["dims"]):
        a = g["a"][i, :d].copy()
        c, vm, sc = g["codes"][i, :d].copy(), g["vmin"][i, :d].copy(), g["scale"][i, :d].copy()
        l2 = vdbg.host_sq8_distance(kset, "l2", a, c, vm, sc, portable)
        ip = vdbg.host_sq8_distance(kset, "ip", a, c, vm, sc, portable)
        assert np.float32(l2).view(np.uint32) == g[f"sq8l2_{kset}"][i].view(np.uint32), (kset, i)
        # the reference's sq8_ip_* return minus the dot product
        assert np.float32(ip).view(np.uint32) == g[f"sq8ip_{kset}"][i].view(np.uint32), (kset, i)


def test_host_sq8_distance_rejects_unknown_sets():
    x = np.zeros(16, np.float32)
    c = np.zeros(16, np.uint8)
    assert np.isnan(vdbg.host_sq8_distance("neon", "l2", x, c, x, x))
    assert np.isnan(vdbg.host_sq8_distance("avx2", "l2", x[:8], c[:8], x[:8], x[:8]))
