"""The int8 ranking GEMM (gemm8.hip): integer rows spanning at most 256 values and queries in
the same int8 window (after one per-dataset shift) rank on int8 MFMA with exact int32
products and sums.  Inner product values equal the fp32 GEMM's; L2 values exceed them by at
most 1 (the half row norm rounded up) and the exact re-scoring decides.  Results must stay
bit-exact to the oracle (FlatIndex::search, src/index/flat_index.cc:11-39), and batches or
datasets outside the window must take the fp16 or fp32 GEMM."""
import numpy as np
import pytest

import vdbg
from vdbg import datagen

pytestmark = pytest.mark.gpu


def _check_equal(gi, gd, oi, od):
    assert gi.shape == oi.shape
    bad = np.nonzero((gi != oi).any(axis=1) | (gd.view(np.uint32) != od.view(np.uint32)).any(axis=1))[0]
    assert bad.size == 0, (
        f"{bad.size} queries differ; first q={bad[0]} gpu={gi[bad[0]].tolist()} "
        f"{gd[bad[0]].tolist()} oracle={oi[bad[0]].tolist()} {od[bad[0]].tolist()}")


def _ints(n, dim, seed, lo, hi):
    return np.random.default_rng(seed).integers(lo, hi + 1, size=(n, dim)).astype(np.float32)


@pytest.mark.parametrize("n,nq,k", [(50000, 200, 10), (120000, 300, 100), (4100, 7, 1),
                                    (70000, 1500, 10), (30000, 40, 200)])
def test_sift_like_takes_int8(ctx, oracle, n, nq, k):
    print(f"gemm8 sift-like n={n} nq={nq} k={k}", flush=True)
    base = datagen.sift_like(n, 128, 6001)
    qs = datagen.sift_like(nq, 128, 6002)
    ds = vdbg.Dataset(ctx, base, 128)
    gi, gd = ds.flat_search(qs, k)
    assert ctx.last_gemm_bits() == 8
    assert ctx.last_fallbacks() == 0  # the int8 candidates certify without exact re-scans
    od, oi = oracle.flat_search(base, qs, k)
    _check_equal(gi, gd, oi, od)


@pytest.mark.parametrize("dim,lo,hi,bits", [(960, 0, 30, 8), (64, 0, 255, 8), (96, -128, 127, 8),
                                            (32, 5, 260, 8), (256, -3, 17, 8), (40, 0, 255, 16),
                                            (100, 0, 255, 16), (64, 0, 300, 16)])
def test_integer_dims_and_ranges(ctx, oracle, dim, lo, hi, bits):
    # pd multiple of 32 and a value range of at most 256 take the int8 GEMM; a 48- or
    # 112-dim pad, or rows spanning 301 values, the fp16 GEMM
    print(f"gemm8 dim={dim} values {lo}..{hi}", flush=True)
    pd = vdbg.padded_dim(dim)
    base = datagen.pad(_ints(9000, dim, 6101 + dim, lo, hi), pd)
    qs = datagen.pad(_ints(70, dim, 6201 + dim, lo, hi), pd)
    ds = vdbg.Dataset(ctx, base, dim)
    gi, gd = ds.flat_search(qs, 10)
    assert ctx.last_gemm_bits() == bits
    assert ctx.last_fallbacks() == 0
    od, oi = oracle.flat_search(base, qs, 10)
    _check_equal(gi, gd, oi, od)


def test_inner_product(ctx, oracle):
    base = _ints(30000, 128, 6301, -20, 20)
    qs = _ints(100, 128, 6302, -20, 20)
    ds = vdbg.Dataset(ctx, base, 128, metric="ip")
    gi, gd = ds.flat_search(qs, 10)
    assert ctx.last_gemm_bits() == 8
    assert ctx.last_fallbacks() == 0
    od, oi = oracle.flat_search(base, qs, 10, metric="ip")
    _check_equal(gi, gd, oi, od)


def test_query_window(ctx, oracle):
    # rows in [0, 100] centre at shift 51: queries may range over [-77, 178]
    base = _ints(20000, 64, 6401, 0, 100)
    ds = vdbg.Dataset(ctx, base, 64)
    inside = _ints(50, 64, 6402, -77, 178)
    gi, gd = ds.flat_search(inside, 10)
    assert ctx.last_gemm_bits() == 8
    od, oi = oracle.flat_search(base, inside, 10)
    _check_equal(gi, gd, oi, od)
    outside = inside.copy()
    outside[13, 7] = 179  # one value past the window
    # a batch of at most 128 queries chooses on the device between int8 and fp32
    gi, gd = ds.flat_search(outside, 10)
    assert ctx.last_gemm_bits() == 32
    od, oi = oracle.flat_search(base, outside, 10)
    _check_equal(gi, gd, oi, od)
    # a larger batch reads the flags on the host and takes the fp16 GEMM
    big = np.ascontiguousarray(np.concatenate([outside, inside, inside, inside])[:180])
    gi, gd = ds.flat_search(big, 10)
    assert ctx.last_gemm_bits() == 16
    od, oi = oracle.flat_search(base, big, 10)
    _check_equal(gi, gd, oi, od)
    frac = inside.copy()
    frac[3, 3] += 0.5  # a fractional query value: the fp32 GEMM
    gi, gd = ds.flat_search(frac, 10)
    assert ctx.last_gemm_bits() == 32
    od, oi = oracle.flat_search(base, frac, 10)
    _check_equal(gi, gd, oi, od)


@pytest.mark.parametrize("frac", [0.05, 0.2, 0.7])
def test_filtered(ctx, oracle, frac):
    # 0.05 / 0.2: the allowed rows are compacted (fp32, fp16 and int8 copies); 0.7: the mask
    # is tested per row, in the sample pass too
    n = 60000
    base = datagen.sift_like(n, 128, 6501)
    qs = datagen.sift_like(96, 128, 6502)
    rows = np.nonzero(np.random.default_rng(6503).random(n) < frac)[0]
    allow = np.zeros((n + 63) // 64, np.uint64)
    np.bitwise_or.at(allow, rows // 64, np.uint64(1) << (rows % 64).astype(np.uint64))
    ds = vdbg.Dataset(ctx, base, 128)
    gi, gd = ds.flat_search(qs, 20, allow=allow)
    assert ctx.last_gemm_bits() == 8
    assert ctx.last_fallbacks() == 0
    od, oi = oracle.flat_search(base, qs, 20, allow=allow)
    _check_equal(gi, gd, oi, od)


def test_duplicate_rows_tie_by_id(ctx, oracle):
    # every row four times: equal distances order by row id
    one = _ints(5000, 128, 6601, 0, 255)
    base = np.repeat(one, 4, axis=0)
    qs = _ints(64, 128, 6602, 0, 255)
    ds = vdbg.Dataset(ctx, base, 128)
    gi, gd = ds.flat_search(qs, 17)
    assert ctx.last_gemm_bits() == 8
    od, oi = oracle.flat_search(base, qs, 17)
    _check_equal(gi, gd, oi, od)


def test_switches_give_identical_results(ctx):
    base = datagen.sift_like(40000, 128, 6701)
    qs = datagen.sift_like(300, 128, 6702)
    ds = vdbg.Dataset(ctx, base, 128)
    gi8, gd8 = ds.flat_search(qs, 50)
    assert ctx.last_gemm_bits() == 8
    ctx.set_int8_gemm(False)
    try:
        gi16, gd16 = ds.flat_search(qs, 50)
        assert ctx.last_gemm_bits() == 16
    finally:
        ctx.set_int8_gemm(True)
    ctx.set_fp16_gemm(False)
    try:
        gi32, gd32 = ds.flat_search(qs, 50)
        assert ctx.last_gemm_bits() == 32
    finally:
        ctx.set_fp16_gemm(True)
    for gi, gd in ((gi16, gd16), (gi32, gd32)):
        assert np.array_equal(gi8, gi)
        assert np.array_equal(gd8.view(np.uint32), gd.view(np.uint32))


@pytest.mark.parametrize("nq,k", [(1100, 10), (1100, 33), (200, 150)])
def test_compact_and_full_sample(ctx, oracle, nq, k):
    # the int8 GEMM's sample pass keeps the 8 smallest group minima per lane and chunk half
    # while those lists hold at least 3 k entries and at most 4096 in all (1100 queries), and
    # every group minimum otherwise (200 queries: one query tile spreads the 65,536 sample
    # rows over 512 chunks); both thresholds certify
    print(f"gemm8 sample pass nq={nq} k={k}", flush=True)
    base = datagen.sift_like(150000, 128, 6801)
    qs = datagen.sift_like(nq, 128, 6802)
    ds = vdbg.Dataset(ctx, base, 128)
    gi, gd = ds.flat_search(qs, k)
    assert ctx.last_gemm_bits() == 8
    assert ctx.last_fallbacks() == 0
    od, oi = oracle.flat_search(base, qs, k)
    _check_equal(gi, gd, oi, od)


def test_unit_neighbours_tie_within_the_bound(ctx, oracle):
    # each query is a row, and 256 rows sit at squared distance 1 from it (+-1 on one dim):
    # int8 L2 values run up to 1 above the GEMM value, so the staged re-scoring cannot
    # certify from the GEMM order and the chain falls through to the exact scan; the answer
    # (the query's row, then distance-1 rows by id) must still be the oracle's
    rng = np.random.default_rng(6901)
    centres = rng.integers(20, 200, size=(40, 128)).astype(np.float32)
    eye = np.eye(128, dtype=np.float32)
    rows = [centres]
    for c in centres:
        rows.append(c + eye)
        rows.append(c - eye)
    base = np.concatenate(rows + [rng.integers(0, 255, size=(30000, 128)).astype(np.float32)])
    qs = np.concatenate([centres] * 4)  # 160 queries: the 256-query tile path
    ds = vdbg.Dataset(ctx, base, 128)
    for k in (10, 40):
        gi, gd = ds.flat_search(qs, k)
        assert ctx.last_gemm_bits() == 8
        od, oi = oracle.flat_search(base, qs, k)
        _check_equal(gi, gd, oi, od)
        assert np.all(gd[:, 1:] == 1.0)


@pytest.mark.parametrize("nq,k,metric", [(1, 10, "l2"), (2, 1, "l2"), (1, 48, "l2"),
                                         (2, 10, "ip"), (7, 100, "l2"), (5, 48, "l2"),
                                         (8, 10, "ip"), (64, 10, "l2"), (128, 20, "l2"),
                                         (1, 10, "ip"), (33, 10, "ip")])
def test_small_batches_choose_on_device(ctx, oracle, nq, k, metric):
    # up to 32 queries and k <= 48: the tiny-batch path (one pass over the int8 rows keeping
    # each chunk's best keys, one merge with the exact re-score and certificate; k_tiny_scan
    # up to 2 queries, k_small_scan above); up to 128 queries: the int8 / fp32 main pass
    # chosen on the device, no host read before it
    base = datagen.sift_like(60000, 128, 6601)
    qs = datagen.sift_like(nq, 128, 6602)
    ds = vdbg.Dataset(ctx, base, 128, metric=metric)
    gi, gd = ds.flat_search(qs, k)
    assert ctx.last_gemm_bits() == 8
    assert ctx.last_fallbacks() == 0
    od, oi = oracle.flat_search(base, qs, k, metric=metric)
    _check_equal(gi, gd, oi, od)
    # one fractional query value: on the tiny-batch path that query alone is re-scanned
    # exactly; other small batches move to the fp32 pass
    qf = qs.copy()
    qf[nq - 1, 5] += 0.25
    gi, gd = ds.flat_search(qf, k)
    if nq <= 32 and k <= 48:
        assert ctx.last_gemm_bits() == 8 and ctx.last_fallbacks() == 1
    else:
        assert ctx.last_gemm_bits() == 32
    od, oi = oracle.flat_search(base, qf, k, metric=metric)
    _check_equal(gi, gd, oi, od)


@pytest.mark.parametrize("frac", [0.002, 0.3])
def test_small_batches_filtered(ctx, oracle, frac):
    # the fused thresholds skip sampled rows the filter rejects; at 0.2 % fewer than k of
    # the 4096 sampled rows may pass, and the threshold is then open
    n = 80000
    base = datagen.sift_like(n, 128, 6611)
    qs = datagen.sift_like(5, 128, 6612)
    rng = np.random.default_rng(6613)
    rows = np.sort(rng.choice(n, size=max(1, int(n * frac)), replace=False))
    allow = np.zeros((n + 63) // 64, np.uint64)
    np.bitwise_or.at(allow, rows // 64, np.uint64(1) << (rows % 64).astype(np.uint64))
    ds = vdbg.Dataset(ctx, base, 128)
    gi, gd = ds.flat_search(qs, 10, allow=allow)
    od, oi = oracle.flat_search(base, qs, 10, allow=allow)
    _check_equal(gi, gd, oi, od)


@pytest.mark.parametrize("nq", [1, 2])
def test_tiny_batches_forced_fallback_and_filter(ctx, oracle, nq):
    # the tiny-batch path with its certificate failed on purpose (every query re-scanned
    # exactly) and with a filter that leaves whole chunks empty
    n = 50000
    base = datagen.sift_like(n, 128, 6621)
    qs = datagen.sift_like(nq, 128, 6622)
    ds = vdbg.Dataset(ctx, base, 128)
    try:
        ctx.set_test_fallbacks(1)
        gi, gd = ds.flat_search(qs, 10)
        assert ctx.last_fallbacks() == nq
    finally:
        ctx.set_test_fallbacks(0)
    od, oi = oracle.flat_search(base, qs, 10)
    _check_equal(gi, gd, oi, od)
    allowed = np.zeros(n, bool)
    allowed[20000:20500] = True  # one stretch: most chunks hold no allowed row
    allowed[::97] = True
    words = np.zeros((n + 63) // 64, np.uint64)
    rows = np.nonzero(allowed)[0]
    np.bitwise_or.at(words, rows // 64, np.uint64(1) << (rows % 64).astype(np.uint64))
    gi, gd = ds.flat_search(qs, 10, allow=words)
    od, oi = oracle.flat_search(base, qs, 10, allow=words)
    _check_equal(gi, gd, oi, od)


@pytest.mark.parametrize("pick", [(0, -1), (-1, 0), (-1, -2)])
def test_tiny_two_queries_edge_chunks(ctx, oracle, pick):
    # two queries on the tiny-batch path whose nearest rows sit in the first and the last
    # row chunk: each query's chunk lists and bounds must be the ones the merge reads
    base = datagen.sift_like(60000, 128, 6621)
    qs = np.ascontiguousarray(base[list(pick)])
    ds = vdbg.Dataset(ctx, base, 128)
    gi, gd = ds.flat_search(qs, 10)
    assert ctx.last_gemm_bits() == 8
    assert ctx.last_fallbacks() == 0
    od, oi = oracle.flat_search(base, qs, 10)
    _check_equal(gi, gd, oi, od)


@pytest.mark.parametrize("pd,nq,k,metric", [(128, 3, 10, "l2"), (128, 16, 10, "l2"),
                                            (128, 32, 48, "l2"), (128, 17, 1, "ip"),
                                            (64, 9, 10, "l2"), (256, 32, 20, "ip"),
                                            (64, 32, 48, "ip"), (256, 5, 1, "l2")])
def test_small_scan_shapes(ctx, oracle, pd, nq, k, metric):
    # k_small_scan: 3..32 queries scored together on int8 MFMA, every lane a chunk of four
    # keys for the merge; rows not a multiple of 32 (the last wave's block runs past them)
    print(f"small scan pd={pd} nq={nq} k={k} {metric}", flush=True)
    n = 50003
    base = datagen.sift_like(n, pd, 6631 + pd)
    qs = datagen.sift_like(nq, pd, 6632 + nq)
    ds = vdbg.Dataset(ctx, base, pd, metric=metric)
    gi, gd = ds.flat_search(qs, k)
    assert ctx.last_gemm_bits() == 8
    assert ctx.last_fallbacks() == 0
    od, oi = oracle.flat_search(base, qs, k, metric=metric)
    _check_equal(gi, gd, oi, od)


def test_small_scan_edges_filter_and_fallback(ctx, oracle):
    # nearest rows in the first and the last wave's rows, a filter that leaves most waves
    # without an allowed row, and the certificate failed on purpose
    n = 70001
    base = datagen.sift_like(n, 128, 6641)
    qs = np.ascontiguousarray(np.concatenate([base[[0, 1, n - 1, n - 2, n // 2]],
                                              datagen.sift_like(7, 128, 6642)]))
    ds = vdbg.Dataset(ctx, base, 128)
    gi, gd = ds.flat_search(qs, 10)
    assert ctx.last_gemm_bits() == 8 and ctx.last_fallbacks() == 0
    od, oi = oracle.flat_search(base, qs, 10)
    _check_equal(gi, gd, oi, od)
    allowed = np.zeros(n, bool)
    allowed[30000:30300] = True
    allowed[::211] = True
    words = np.zeros((n + 63) // 64, np.uint64)
    rows = np.nonzero(allowed)[0]
    np.bitwise_or.at(words, rows // 64, np.uint64(1) << (rows % 64).astype(np.uint64))
    gi, gd = ds.flat_search(qs, 10, allow=words)
    od, oi = oracle.flat_search(base, qs, 10, allow=words)
    _check_equal(gi, gd, oi, od)
    try:
        ctx.set_test_fallbacks(1)
        gi, gd = ds.flat_search(qs, 10)
        assert ctx.last_fallbacks() == len(qs)
    finally:
        ctx.set_test_fallbacks(0)
    od, oi = oracle.flat_search(base, qs, 10)
    _check_equal(gi, gd, oi, od)
