"""The exact-integer ranking GEMM: rows and queries whose values are all integers of magnitude
<= 2048, with every partial sum below 2^24, rank through fp16 MFMA (each product and sum is
exact, so the ranking values equal the fp32 GEMM's bit for bit).  Results must stay bit-exact
to the oracle (FlatIndex::search, src/index/flat_index.cc:11-39), and batches or datasets
outside those bounds must take the fp32 GEMM."""
import numpy as np
import pytest

import vdbg
from vdbg import datagen

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _fp16_not_int8(ctx):
    # datasets created here keep no int8 copy, so integer rows rank on the fp16 GEMM
    ctx.set_int8_gemm(False)
    yield
    ctx.set_int8_gemm(True)


def _check_equal(gi, gd, oi, od):
    assert gi.shape == oi.shape
    bad = np.nonzero((gi != oi).any(axis=1) | (gd.view(np.uint32) != od.view(np.uint32)).any(axis=1))[0]
    assert bad.size == 0, (
        f"{bad.size} queries differ; first q={bad[0]} gpu={gi[bad[0]].tolist()} "
        f"{gd[bad[0]].tolist()} oracle={oi[bad[0]].tolist()} {od[bad[0]].tolist()}")


def _int_rows(n, dim, seed, hi):
    return np.random.default_rng(seed).integers(0, hi + 1, size=(n, dim)).astype(np.float32)


@pytest.mark.parametrize("n,nq,k", [(50000, 200, 10), (120000, 300, 100), (4100, 7, 1)])
def test_sift_like_takes_fp16(ctx, oracle, n, nq, k):
    print(f"gemm16 sift-like n={n} nq={nq} k={k}", flush=True)
    base = datagen.sift_like(n, 128, 5001)
    qs = datagen.sift_like(nq, 128, 5002)
    ds = vdbg.Dataset(ctx, base, 128)
    gi, gd = ds.flat_search(qs, k)
    assert ctx.last_gemm_bits() == 16
    od, oi = oracle.flat_search(base, qs, k)
    _check_equal(gi, gd, oi, od)
    assert ctx.last_fallbacks() == 0


@pytest.mark.parametrize("dim,hi,bits", [(960, 30, 16), (40, 255, 16), (16, 400, 16),
                                         (16, 1000, 32), (300, 60, 0)])
def test_integer_other_dims(ctx, oracle, dim, hi, bits):
    # K chunking (960 -> 15 chunks of 64 dims), a ragged 48-dim pad, one 16-dim K block;
    # 16 dims of values up to 1000 keep every element-wise partial sum below 2^24 but not
    # (|q| + max |x|)^2, so they rank on the fp32 GEMM; 304 dims have no GEMM kernel
    print(f"gemm16 dim={dim} values 0..{hi}", flush=True)
    pd = vdbg.padded_dim(dim)
    base = datagen.pad(_int_rows(9000, dim, 5101 + dim, hi), pd)
    qs = datagen.pad(_int_rows(70, dim, 5201 + dim, hi), pd)
    ds = vdbg.Dataset(ctx, base, dim)
    gi, gd = ds.flat_search(qs, 10)
    od, oi = oracle.flat_search(base, qs, 10)
    _check_equal(gi, gd, oi, od)
    assert ctx.last_gemm_bits() == bits


def test_integer_inner_product(ctx, oracle):
    base = (_int_rows(30000, 128, 5301, 40) - 20).astype(np.float32)
    qs = (_int_rows(100, 128, 5302, 40) - 20).astype(np.float32)
    ds = vdbg.Dataset(ctx, base, 128, metric="ip")
    gi, gd = ds.flat_search(qs, 10)
    assert ctx.last_gemm_bits() == 16
    od, oi = oracle.flat_search(base, qs, 10, metric="ip")
    _check_equal(gi, gd, oi, od)


def test_one_fractional_query_takes_fp32(ctx, oracle):
    base = datagen.sift_like(30000, 128, 5401)
    qs = datagen.sift_like(64, 128, 5402)
    qs[17, 3] += 0.5
    ds = vdbg.Dataset(ctx, base, 128)
    gi, gd = ds.flat_search(qs, 10)
    assert ctx.last_gemm_bits() == 32
    od, oi = oracle.flat_search(base, qs, 10)
    _check_equal(gi, gd, oi, od)
    # the same dataset with an all-integer batch goes back to fp16
    gi, gd = ds.flat_search(np.delete(qs, 17, axis=0), 10)
    assert ctx.last_gemm_bits() == 16
    od, oi = oracle.flat_search(base, np.delete(qs, 17, axis=0), 10)
    _check_equal(gi, gd, oi, od)


def test_fractional_rows_take_split_operands(ctx, oracle):
    # float rows rank on fp16 MFMA with both operands split in two parts (not exact: the
    # bound is widened and the exact re-scoring decides), integer queries included
    base = datagen.uniform_rows(20000, 128, 5501)
    qs = np.rint(datagen.uniform_rows(32, 128, 5502) * 10).astype(np.float32)
    ds = vdbg.Dataset(ctx, base, 128)
    gi, gd = ds.flat_search(qs, 10)
    assert ctx.last_gemm_bits() == 16
    od, oi = oracle.flat_search(base, qs, 10)
    _check_equal(gi, gd, oi, od)


@pytest.mark.parametrize("frac", [0.2, 0.7])
def test_integer_filtered(ctx, oracle, frac):
    # 0.2: allowed rows are compacted (fp32 and fp16 copies); 0.7: the mask is tested per row
    n = 60000
    base = datagen.sift_like(n, 128, 5601)
    qs = datagen.sift_like(96, 128, 5602)
    rows = np.nonzero(np.random.default_rng(5603).random(n) < frac)[0]
    allow = np.zeros((n + 63) // 64, np.uint64)
    np.bitwise_or.at(allow, rows // 64, np.uint64(1) << (rows % 64).astype(np.uint64))
    ds = vdbg.Dataset(ctx, base, 128)
    gi, gd = ds.flat_search(qs, 20, allow=allow)
    assert ctx.last_gemm_bits() == 16
    od, oi = oracle.flat_search(base, qs, 20, allow=allow)
    _check_equal(gi, gd, oi, od)


def test_fp32_switch_gives_identical_results(ctx):
    base = datagen.sift_like(40000, 128, 5801)
    qs = datagen.sift_like(300, 128, 5802)
    ds = vdbg.Dataset(ctx, base, 128)
    gi16, gd16 = ds.flat_search(qs, 50)
    assert ctx.last_gemm_bits() == 16
    ctx.set_fp16_gemm(False)
    try:
        gi32, gd32 = ds.flat_search(qs, 50)
        assert ctx.last_gemm_bits() == 32
    finally:
        ctx.set_fp16_gemm(True)
    assert np.array_equal(gi16, gi32)
    assert np.array_equal(gd16.view(np.uint32), gd32.view(np.uint32))


def test_owner_closes_before_children(oracle):
    # closing a context first closes its datasets and their indexes; the library refuses to
    # destroy a context or dataset that still has children
    ctx2 = vdbg.Context(0)
    base = datagen.sift_like(5000, 128, 5701)
    ds = vdbg.Dataset(ctx2, base, 128)
    sq = vdbg.Sq8Index(ds)
    assert vdbg.lib.vdbg_ctx_destroy(ctx2.h) != 0
    assert vdbg.lib.vdbg_dataset_destroy(ds.h) != 0
    gi, gd = ds.flat_search(base[:3], 5)
    assert (gi[:, 0] == np.arange(3)).all()
    ctx2.close()
    assert sq.h is None and ds.h is None and ctx2.h is None
    ds.close()
    sq.close()
