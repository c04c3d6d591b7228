"""IVF-PQ shapes past the scan's table staging and 64-dim sub-vectors: m = 64 over 64 dims,
m = 48 over 96 (inner product), m = 2 over 136 (68-dim sub-vectors).  vdb accepts any pq_m
that divides the dimension (src/index/index.cc:27-29).  The reference built these indexes and
recorded its IvfPqIndex::search results (tests/golden/ivf_shapes.npz); the GPU must return
them from the same files, and its own build over the same rows must write the same files."""
import os
import sys

import numpy as np
import pytest

import vdbg

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLD)
from make_golden import ivf_shape_rows  # noqa: E402


def case(g, tag):
    n, dim, m, nlist, seed = (int(v) for v in g[f"{tag}_shape"])
    return ivf_shape_rows(n, dim, seed), ivf_shape_rows(20, dim, seed + 100), dim, m, nlist


@pytest.mark.parametrize("tag", ["w", "x", "y"])
def test_reference_files_give_reference_results(ctx, tag):
    g = np.load(os.path.join(GOLD, "ivf_shapes.npz"))
    ctx.set_kernels(str(g["kernels"]))
    base, q, dim, m, nlist = case(g, tag)
    metric = str(g[f"{tag}_metric"])
    print(f"ivf shape {tag}: dim {dim} m {m} nlist {nlist} {metric}", flush=True)
    ds = vdbg.Dataset(ctx, base, dim, metric)
    ix = vdbg.IvfPqIndex.load(ds, g[f"{tag}_file"].tobytes())
    for si, (nprobe, rr) in enumerate(g["settings"]):
        ids, d, dc = ix.search(q, 10, int(nprobe), int(rr))
        key = f"{tag}_s{si}"
        assert np.array_equal(ids, g[key + "_i"]), key
        assert np.array_equal(d.view(np.uint32), g[key + "_d"].view(np.uint32)), key
        assert np.array_equal(dc, g[key + "_dc"]), key
    ix.close()
    ds.close()


@pytest.mark.parametrize("tag", ["w", "x", "y"])
def test_gpu_build_writes_the_reference_file(ctx, tag):
    g = np.load(os.path.join(GOLD, "ivf_shapes.npz"))
    base, q, dim, m, nlist = case(g, tag)
    metric = str(g[f"{tag}_metric"])
    print(f"ivf shape build {tag}", flush=True)
    ds = vdbg.Dataset(ctx, base, dim, metric)
    ix = vdbg.IvfPqIndex.build(ds, nlist=nlist, m=m, seed=42, max_points=256, iters=25)
    assert ix.save() == g[f"{tag}_file"].tobytes()
    ix.close()
    ds.close()
