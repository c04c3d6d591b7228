"""The synthetic-workload generators: the torch (device) streams reproduce the numpy ones."""
import numpy as np
import torch

from vdbg import datagen


def test_rand_u64_torch_matches_numpy():
    a = datagen.rand_u64(77, 5, 5000)
    b = datagen.rand_u64_t(torch, 77, 5, 5000, "cpu").numpy().view(np.uint64)
    assert np.array_equal(a, b)
    m = datagen.umod_t(torch.from_numpy(b.view(np.int64)), 10000).numpy()
    assert np.array_equal((a % np.uint64(10000)).astype(np.int64), m)


def test_normal_torch_matches_numpy():
    x = datagen.normal(9, 3, 1001)
    y = datagen.normal_t(torch, 9, 3, 1001, "cpu").numpy()
    assert np.allclose(x, y, rtol=0, atol=1e-12)


def test_clustered_unit_torch_rows_and_offsets():
    c1 = datagen.clustered_unit(3000, 96, 11, 12, 50, 0.5)
    c2 = datagen.clustered_unit_t(torch, 3000, 96, 11, 12, 50, 0.5, "cpu").numpy()
    assert np.abs(c1 - c2).max() < 1e-6
    c3 = datagen.clustered_unit_t(torch, 1000, 96, 11, 12, 50, 0.5, "cpu", start_row=2000)
    assert np.array_equal(c3.numpy(), c2[2000:])
    n = np.linalg.norm(c2.astype(np.float64), axis=1)
    assert np.abs(n - 1).max() < 1e-6
