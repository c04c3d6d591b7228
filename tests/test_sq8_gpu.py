"""SQ8 on the GPU against the oracle: training and encoding byte-identical to
Sq8Quantizer (src/index/quant/sq8.cc:9-37); the exhaustive SQ8 scan into the top
max(depth, k) plus fp32 Rerank (src/index/hnsw/hnsw_index.cc:82-100, src/index/index.cc:
89-95) with ids and distances bit-exact."""
import numpy as np
import pytest

import vdbg
from vdbg import datagen

pytestmark = pytest.mark.gpu


def _eq(gi, gd, oi, od):
    bad = np.nonzero((gi != oi).any(1) | (gd.view(np.uint32) != od.view(np.uint32)).any(1))[0]
    assert bad.size == 0, (f"{bad.size} queries differ; q={bad[0]} gpu={gi[bad[0]].tolist()} "
                           f"{gd[bad[0]].tolist()} oracle={oi[bad[0]].tolist()} "
                           f"{od[bad[0]].tolist()}")


@pytest.mark.parametrize("n,dim,seed", [(3000, 100, 1), (20000, 128, 2), (100, 7, 3)])
def test_sq8_train_encode_byte_identical(ctx, oracle, n, dim, seed):
    print(f"sq8 train/encode n={n} dim={dim}", flush=True)
    pd = vdbg.padded_dim(dim)
    rng = np.random.default_rng(seed)
    base = datagen.pad(rng.normal(0, 3, (n, dim)).astype(np.float32), pd)
    base[:, min(3, dim - 1)] = 0.5  # a constant column: scale 0
    ds = vdbg.Dataset(ctx, base, dim)
    vmin, scale = ds.sq8_train()
    ov, osc = oracle.sq8_train(base, dim)
    assert np.array_equal(vmin.view(np.uint32), ov.view(np.uint32))
    assert np.array_equal(scale.view(np.uint32), osc.view(np.uint32))
    sq = vdbg.Sq8Index(ds, vmin, scale)
    assert np.array_equal(sq.codes(), oracle.sq8_encode(base, dim, ov, osc))


def test_sq8_train_sift_like_full_size_invariants(ctx):
    # 1M x 128 SIFT-like: min/max are exact values of the data, codes decode within half
    # a step (tests/distance_test.cc:106-126), checked on a strided subset
    base = datagen.sift_like(1_000_000, 128, 2002)
    ds = vdbg.Dataset(ctx, base, 128)
    vmin, scale = ds.sq8_train()
    assert np.array_equal(vmin, base.min(0))
    assert np.array_equal(scale, (base.max(0) - vmin) / np.float32(255))
    sq = vdbg.Sq8Index(ds, vmin, scale)
    codes = sq.codes()
    sub = slice(0, None, 997)
    back = vmin + codes[sub].astype(np.float32) * scale
    assert (np.abs(back - base[sub]) <= scale * 0.5 * 1.0001 + 1e-6).all()


@pytest.mark.parametrize("n,nq,k,depth", [(20000, 100, 10, 100), (20000, 64, 10, 0),
                                          (5000, 10, 10, 50), (30000, 200, 100, 100)])
def test_sq8_search_matches_oracle(ctx, oracle, n, nq, k, depth):
    print(f"sq8 search n={n} nq={nq} k={k} depth={depth}", flush=True)
    base = datagen.sift_like(n, 128, 2002)
    qs = datagen.sift_like(nq, 128, 2003)
    ds = vdbg.Dataset(ctx, base, 128)
    sq = vdbg.Sq8Index(ds)
    gi, gd = sq.search(qs, k, depth)
    od, oi = oracle.sq8_search(base, sq.codes(), sq.vmin, sq.scale, qs, k, depth)
    _eq(gi, gd, oi, od)


@pytest.mark.parametrize("metric", ["ip", "cosine"])
def test_sq8_inner_product(ctx, oracle, metric):
    base = datagen.clustered_unit(20000, 128, 41, 42, 100, 0.5)
    qs = datagen.clustered_unit(64, 128, 43, 42, 100, 0.5)
    ds = vdbg.Dataset(ctx, base, 128, metric=metric)
    sq = vdbg.Sq8Index(ds)
    gi, gd = sq.search(qs, 10, 64)
    od, oi = oracle.sq8_search(base, sq.codes(), sq.vmin, sq.scale, qs, 10, 64, metric=metric)
    _eq(gi, gd, oi, od)


def test_sq8_filter(ctx, oracle):
    base = datagen.uniform_rows(20000, 128, 51)
    qs = datagen.uniform_rows(40, 128, 52)
    allow = np.zeros((20000 + 63) // 64, np.uint64)
    rows = np.arange(0, 20000, 5)
    np.bitwise_or.at(allow, rows // 64, np.uint64(1) << (rows % 64).astype(np.uint64))
    ds = vdbg.Dataset(ctx, base, 128)
    sq = vdbg.Sq8Index(ds)
    gi, gd = sq.search(qs, 10, 40, allow=allow)
    assert (gi % 5 == 0).all()
    od, oi = oracle.sq8_search(base, sq.codes(), sq.vmin, sq.scale, qs, 10, 40, allow=allow)
    _eq(gi, gd, oi, od)


@pytest.mark.parametrize("k,depth", [(10, 500), (300, 0), (100, 1000)])
def test_sq8_deep(ctx, oracle, k, depth):
    # SQ8 scan depth or k beyond the wave top-k, then the float rerank
    base = datagen.sift_like(30000, 128, 4201)
    qs = datagen.sift_like(20, 128, 4202)
    ds = vdbg.Dataset(ctx, base, 128)
    sq = vdbg.Sq8Index(ds)
    gi, gd = sq.search(qs, k, depth)
    od, oi = oracle.sq8_search(base, sq.codes(), sq.vmin, sq.scale, qs, k, depth)
    _eq(gi, gd, oi, od)


def _wide_range_rows(n, dim, seed):
    # per-dimension scales from 1e-3 to 1e3 and signs: the split fp16 query operand spans
    # many binades (small parts fall below fp16's normal range)
    rng = np.random.default_rng(seed)
    scales = np.float32(10.0) ** rng.uniform(-3, 3, dim).astype(np.float32)
    return (rng.normal(0, 1, (n, dim)).astype(np.float32) * scales).astype(np.float32)


@pytest.mark.parametrize("data,metric,nq,k,depth", [
    ("sift_like", "l2", 300, 10, 100), ("uniform", "l2", 200, 10, 0),
    ("unit", "cosine", 150, 10, 64), ("unit", "ip", 150, 20, 0),
    ("wide", "l2", 130, 10, 100), ("wide", "ip", 100, 10, 50)])
@pytest.mark.parametrize("dim", [128, 96, 384])
def test_sq8_int8_fp16_fp32_match_oracle(ctx, oracle, data, metric, nq, k, depth, dim):
    # the SQ8 scan ranks on int8 MFMA (codes - 128 exact, the query operand rounded to
    # integers in two int8 parts under a widened bound), on fp16 MFMA with the int8 GEMM off
    # (codes exact, query operand split in two fp16 parts), or on the fp32 GEMM; results must
    # be the same bit for bit and the oracle's
    print(f"sq8 int8/fp16/fp32 {data} {metric} dim={dim} nq={nq} k={k} depth={depth}", flush=True)
    n = 40000 if dim <= 128 else 12000
    if data == "sift_like":
        base, qs = datagen.sift_like(n, dim, 6101), datagen.sift_like(nq, dim, 6102)
    elif data == "uniform":
        base, qs = datagen.uniform_rows(n, dim, 6103), datagen.uniform_rows(nq, dim, 6104)
    elif data == "unit":
        base = datagen.clustered_unit(n, dim, 6105, 6106, 200, 0.5)
        qs = datagen.clustered_unit(nq, dim, 6107, 6106, 200, 0.5)
    else:
        base, qs = _wide_range_rows(n, dim, 6108), _wide_range_rows(nq, dim, 6108 + 1)
    ds = vdbg.Dataset(ctx, base, dim, metric=metric)
    sq = vdbg.Sq8Index(ds)
    gi, gd = sq.search(qs, k, depth)
    assert ctx.last_gemm_bits() == 8
    ctx.set_int8_gemm(False)
    try:
        gi16, gd16 = sq.search(qs, k, depth)
        assert ctx.last_gemm_bits() == 16
    finally:
        ctx.set_int8_gemm(True)
    ctx.set_fp16_gemm(False)
    try:
        gi32, gd32 = sq.search(qs, k, depth)
        assert ctx.last_gemm_bits() == 32
    finally:
        ctx.set_fp16_gemm(True)
    _eq(gi, gd, gi16, gd16)
    _eq(gi, gd, gi32, gd32)
    od, oi = oracle.sq8_search(base, sq.codes(), sq.vmin, sq.scale, qs, k, depth, metric=metric)
    _eq(gi, gd, oi, od)


@pytest.mark.parametrize("int8", [True, False])
def test_sq8_large_batch_filtered(ctx, oracle, int8):
    n, nq = 120000, 700
    base, qs = datagen.sift_like(n, 128, 6201), datagen.sift_like(nq, 128, 6202)
    rows = np.nonzero(np.random.default_rng(6203).random(n) < 0.6)[0]
    allow = np.zeros((n + 63) // 64, np.uint64)
    np.bitwise_or.at(allow, rows // 64, np.uint64(1) << (rows % 64).astype(np.uint64))
    ds = vdbg.Dataset(ctx, base, 128)
    sq = vdbg.Sq8Index(ds)
    ctx.set_int8_gemm(int8)
    try:
        gi, gd = sq.search(qs, 10, 100, allow=allow)
        assert ctx.last_gemm_bits() == (8 if int8 else 16)
        assert ctx.last_fallbacks() == 0
    finally:
        ctx.set_int8_gemm(True)
    od, oi = oracle.sq8_search(base, sq.codes(), sq.vmin, sq.scale, qs, 10, 100, allow=allow)
    _eq(gi, gd, oi, od)


@pytest.mark.parametrize("nq,k,depth", [(600, 10, 20), (600, 10, 100), (100, 10, 100)])
def test_sq8_int8_sample_passes(ctx, oracle, nq, k, depth):
    # 600 queries take the int8 GEMM's compact sample pass; 100 queries (one tile, the
    # sample spread over 512 chunks) the one keeping every group minimum
    base, qs = datagen.sift_like(90000, 128, 6301), datagen.sift_like(nq, 128, 6302)
    ds = vdbg.Dataset(ctx, base, 128)
    sq = vdbg.Sq8Index(ds)
    gi, gd = sq.search(qs, k, depth)
    assert ctx.last_gemm_bits() == 8
    assert ctx.last_fallbacks() == 0
    od, oi = oracle.sq8_search(base, sq.codes(), sq.vmin, sq.scale, qs, k, depth)
    _eq(gi, gd, oi, od)


def test_sq8_int8_falls_back_when_row_starts_overflow(ctx, oracle):
    # queries within 1e-3 of the quantizer's minimum: the batch's query operand is so small
    # that its scale exponent would push the L2 row starts past 2^27, so the batch takes the
    # fp16 split GEMM, and the answers stay the oracle's
    base = datagen.sift_like(20000, 128, 6401)
    ds = vdbg.Dataset(ctx, base, 128)
    sq = vdbg.Sq8Index(ds)
    rng = np.random.default_rng(6402)
    qs = (sq.vmin[None, :128] + rng.uniform(0, 1e-3, (40, 128))).astype(np.float32)
    gi, gd = sq.search(qs, 10, 50)
    assert ctx.last_gemm_bits() == 16
    od, oi = oracle.sq8_search(base, sq.codes(), sq.vmin, sq.scale, qs, 10, 50)
    _eq(gi, gd, oi, od)
