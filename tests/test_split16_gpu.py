"""Float rows on the two-part GEMMs, and on the high fp16 halves alone (the default, last
tests).  With the high-half ranking off and the int8 GEMM on, rows and queries
scaled by powers of two are rounded to integers and split into int8 h + l parts, ranked by
2^16 h.h + 2^8 (h.l + l.h) + l.l under a bound widened for the rounding; with it off, they
are split into fp16 h + l parts and ranked by x_h q_h + x_h q_l + x_l q_h.  Returned ids and
distances must equal the fp32 GEMM's and the oracle's (FlatIndex::search,
src/index/flat_index.cc:11-39) bit for bit, across K-chunk shapes, metrics, value ranges,
filters and batch sizes."""
import numpy as np
import pytest

import vdbg
from vdbg import datagen

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _int8_at_any_size(ctx):
    # the two-part paths: the high-half fp16 ranking off (datasets then keep an int8 copy),
    # and the test batches take the int8 two-part GEMM whatever their size
    ctx.set_fp16_single(False)
    ctx.set_int8_float_min_work(0)
    yield
    ctx.set_int8_float_min_work(2e10)
    ctx.set_fp16_single(True)


def _check_equal(gi, gd, oi, od):
    assert gi.shape == oi.shape
    bad = np.nonzero((gi != oi).any(axis=1) | (gd.view(np.uint32) != od.view(np.uint32)).any(axis=1))[0]
    assert bad.size == 0, (
        f"{bad.size} queries differ; first q={bad[0]} gpu={gi[bad[0]].tolist()} "
        f"{gd[bad[0]].tolist()} ref={oi[bad[0]].tolist()} {od[bad[0]].tolist()}")


def _data(kind, n, nq, dim, seed):
    if kind == "uniform":
        return datagen.uniform_rows(n, dim, seed), datagen.uniform_rows(nq, dim, seed + 1)
    if kind == "unit":
        return (datagen.clustered_unit(n, dim, seed, seed + 7, 300, 0.5),
                datagen.clustered_unit(nq, dim, seed + 1, seed + 7, 300, 0.5))
    rng = np.random.default_rng(seed)
    if kind == "normal":
        return (rng.normal(0, 1, (n, dim)).astype(np.float32),
                rng.normal(0, 1, (nq, dim)).astype(np.float32))
    # per-dimension scales over six decades: small parts fall below fp16's normal range
    scales = (np.float32(10.0) ** rng.uniform(-3, 3, dim)).astype(np.float32)
    return ((rng.normal(0, 1, (n, dim)) * scales).astype(np.float32),
            (rng.normal(0, 1, (nq, dim)) * scales).astype(np.float32))


def _search_both(ctx, ds, qs, k, allow=None, expect8=None):
    # default (int8 two-part where the padded dim and the batch allow it), fp16 two-part, fp32
    gi, gd = ds.flat_search(qs, k, allow=allow)
    bits = ctx.last_gemm_bits()
    assert bits in (8, 16)
    if expect8 is not None:
        assert bits == (8 if expect8 else 16)
    ctx.set_int8_gemm(False)
    try:
        gi16, gd16 = ds.flat_search(qs, k, allow=allow)
        assert ctx.last_gemm_bits() == 16
    finally:
        ctx.set_int8_gemm(True)
    ctx.set_fp16_gemm(False)
    try:
        gi32, gd32 = ds.flat_search(qs, k, allow=allow)
        assert ctx.last_gemm_bits() == 32
    finally:
        ctx.set_fp16_gemm(True)
    _check_equal(gi, gd, gi16, gd16)
    _check_equal(gi, gd, gi32, gd32)
    return gi, gd


@pytest.mark.parametrize("kind,metric,dim,n,nq,k", [
    ("uniform", "l2", 128, 30000, 200, 10),     # K chunk 64, two chunks
    ("unit", "cosine", 384, 30000, 150, 10),    # the filtered benchmark's shape, six chunks
    ("normal", "l2", 96, 20000, 130, 50),       # chunk 48
    ("unit", "ip", 112, 20000, 100, 10),        # chunk 16, seven chunks
    ("wide", "l2", 64, 20000, 100, 10),
    ("wide", "ip", 128, 20000, 100, 20),
    ("normal", "l2", 1024, 8000, 64, 10),
    ("uniform", "l2", 16, 5000, 40, 5),
    ("normal", "ip", 37, 20000, 64, 20),        # padded to 48: one chunk of [h | l] 96 wide
    ("unit", "cosine", 256, 20000, 100, 10),    # four chunks of 64, next chunk's queries ahead
])
def test_split_matches_fp32_and_oracle(ctx, oracle, kind, metric, dim, n, nq, k):
    print(f"split16 {kind} {metric} dim={dim} n={n} nq={nq} k={k}", flush=True)
    base, qs = _data(kind, n, nq, dim, 7001 + dim)
    pd = vdbg.padded_dim(dim)
    base, qs = datagen.pad(base, pd), datagen.pad(qs, pd)
    ds = vdbg.Dataset(ctx, base, dim, metric=metric)
    # unit rows whose padded dim is a multiple of 32 must take the int8 two-part GEMM
    gi, gd = _search_both(ctx, ds, qs, k, expect8=True if kind == "unit" and pd % 32 == 0 else None)
    od, oi = oracle.flat_search(base, qs, k, metric=metric)
    _check_equal(gi, gd, oi, od)
    assert ctx.last_fallbacks() == 0


@pytest.mark.parametrize("frac", [0.15, 0.7])
def test_split_filtered(ctx, oracle, frac):
    # 0.15: allowed rows compacted (fp32 rows and fp16 pairs); 0.7: NaN starts per filtered row
    n, dim = 40000, 384
    base, qs = _data("unit", n, 128, dim, 7101)
    rows = np.nonzero(np.random.default_rng(7102).random(n) < frac)[0]
    allow = np.zeros((n + 63) // 64, np.uint64)
    np.bitwise_or.at(allow, rows // 64, np.uint64(1) << (rows % 64).astype(np.uint64))
    ds = vdbg.Dataset(ctx, base, dim, metric="cosine")
    gi, gd = _search_both(ctx, ds, qs, 10, allow=allow, expect8=True)
    od, oi = oracle.flat_search(base, qs, 10, metric="cosine", allow=allow)
    _check_equal(gi, gd, oi, od)


@pytest.mark.parametrize("kind,metric", [("normal", "l2"), ("unit", "cosine")])
def test_split_large_batch(ctx, oracle, kind, metric):
    n, nq, dim = 150000, 1100, 128
    base, qs = _data(kind, n, nq, dim, 7201)
    ds = vdbg.Dataset(ctx, base, dim, metric=metric)
    gi, gd = ds.flat_search(qs, 10)
    assert ctx.last_gemm_bits() in (8, 16)
    assert ctx.last_fallbacks() == 0
    od, oi = oracle.flat_search(base, qs, 10, metric=metric)
    _check_equal(gi, gd, oi, od)


@pytest.fixture
def single(ctx):
    ctx.set_fp16_single(True)
    yield ctx
    ctx.set_fp16_single(False)


_CASES = [("uniform", "l2", 128, 30000, 200, 10), ("unit", "cosine", 384, 30000, 150, 10),
          ("normal", "l2", 96, 20000, 130, 50), ("unit", "ip", 112, 20000, 100, 10),
          ("wide", "l2", 64, 20000, 100, 10), ("wide", "ip", 128, 20000, 100, 20),
          ("normal", "l2", 1024, 8000, 64, 10), ("normal", "ip", 37, 20000, 64, 20),
          ("unit", "cosine", 256, 20000, 300, 10)]


@pytest.mark.parametrize("kind,metric,dim,n,nq,k", _CASES)
def test_single_part_matches_oracle(single, oracle, kind, metric, dim, n, nq, k):
    # float rows ranked on the high fp16 halves alone (one MFMA per product), the bound
    # widened by (2^-10 + 2^-21) |q||x|: same ids and distances as the oracle
    ctx = single
    print(f"single16 {kind} {metric} dim={dim} n={n} nq={nq} k={k}", flush=True)
    base, qs = _data(kind, n, nq, dim, 7301 + dim)
    pd = vdbg.padded_dim(dim)
    base, qs = datagen.pad(base, pd), datagen.pad(qs, pd)
    ds = vdbg.Dataset(ctx, base, dim, metric=metric)
    gi, gd = ds.flat_search(qs, k)
    assert ctx.last_gemm_bits() == 16
    od, oi = oracle.flat_search(base, qs, k, metric=metric)
    _check_equal(gi, gd, oi, od)


@pytest.mark.parametrize("frac", [0.15, 0.7])
def test_single_part_filtered(single, oracle, frac):
    ctx = single
    n, dim = 40000, 384
    base, qs = _data("unit", n, 128, dim, 7111)
    rows = np.nonzero(np.random.default_rng(7112).random(n) < frac)[0]
    allow = np.zeros((n + 63) // 64, np.uint64)
    np.bitwise_or.at(allow, rows // 64, np.uint64(1) << (rows % 64).astype(np.uint64))
    ds = vdbg.Dataset(ctx, base, dim, metric="cosine")
    gi, gd = ds.flat_search(qs, 10, allow=allow)
    assert ctx.last_gemm_bits() == 16
    od, oi = oracle.flat_search(base, qs, 10, metric="cosine", allow=allow)
    _check_equal(gi, gd, oi, od)
