"""The ranking bound of the IVF-PQ row-sum scan (k_ivf_scan_rs), checked in float32 on the CPU.

The scan ranks a code of probed list l by A = offset + (rowsum + sum_j qtab[j][c_j]), rowsum =
sum_j term2[l][j][c_j] summed once per row, while the reference scores it as E = offset +
adc(table) with table[j][c] = fl(term2 + qtab) and four accumulators over j mod 4
(src/index/quant/ivf_pq.cc:203-214, src/index/quant/pq.h:36-46).  The kernel claims
|A - E| < 2^-19 S with S = |offset| + sum_j max_c |term2[l][j][c]| + sum_j max_c |qtab[j][c]|
(each sum raised by 2^-16), and skips a row only when
    rowsum + table sum > fl(tau + 2^-17 |tau|) + fl(2^-17 S - offset),
which must imply E > tau.  numpy float32 operations round each result to float32, so the
kernel's and the reference's operation orders are reproduced exactly here, over magnitudes
spread across many binades with strong cancellation (E far below S)."""
import numpy as np
import pytest

F = np.float32
M = 16


def _reference_score(off, t2, qt, codes):
    # table entries rounded once, four accumulators over j mod 4, (s0 + s1) + (s2 + s3)
    n = codes.shape[0]
    s = [np.zeros(n, F) for _ in range(4)]
    for j in range(M):
        e = (t2[j, codes[:, j]] + qt[j, codes[:, j]]).astype(F)
        s[j % 4] = (s[j % 4] + e).astype(F)
    adc = ((s[0] + s[1]).astype(F) + (s[2] + s[3]).astype(F)).astype(F)
    return (F(off) + adc).astype(F)


def _ranking_terms(t2, qt, codes):
    n = codes.shape[0]
    rs = np.zeros(n, F)
    for j in range(M):  # k_ivf_rowsum: j ascending from 0
        rs = (rs + t2[j, codes[:, j]]).astype(F)
    q = [qt[j, codes[:, j]].astype(F) for j in range(4)]  # the first four start the sums
    for j in range(4, M):
        q[j % 4] = (q[j % 4] + qt[j, codes[:, j]]).astype(F)
    qs = ((q[0] + q[1]).astype(F) + (q[2] + q[3]).astype(F)).astype(F)
    return (rs + qs).astype(F)


def _bound_terms(off, t2, qt):
    t2abs = F(0)
    for j in range(M):
        t2abs = F(t2abs + F(np.abs(t2[j]).max()))
    t2abs = F(t2abs * F(1 + 2.0 ** -16))
    bq = F(0)
    for j in range(M):
        bq = F(bq + F(np.abs(qt[j]).max()))
    bq = F(bq * F(1 + 2.0 ** -16))
    return F(F(F(abs(off)) + t2abs) + bq)


@pytest.mark.parametrize("seed", range(12))
def test_rowsum_ranking_bound_and_skip_rule(seed):
    rng = np.random.default_rng(seed)
    scale = 10.0 ** rng.uniform(-3, 6)
    # entries over eight binades, term2 and qtab of opposite signs so the scores cancel
    t2 = (rng.uniform(1, 2, (M, 256)) * 2.0 ** rng.integers(-4, 4, (M, 256)) * scale).astype(F)
    qt = (-t2 * rng.uniform(0.9, 1.1, (M, 256)).astype(F)).astype(F)
    off = F(rng.uniform(-1, 1) * scale * 16)
    codes = rng.integers(0, 256, (20000, M)).astype(np.int64)
    e = _reference_score(off, t2, qt, codes)
    rq = _ranking_terms(t2, qt, codes)
    s_bound = _bound_terms(off, t2, qt)
    err = np.abs(np.float64(off) + rq.astype(np.float64) - e.astype(np.float64))
    assert (err <= 2.0 ** -19 * np.float64(s_bound)).all(), (err.max(), s_bound)
    # the data exercises the rounding: without its margin the rule drops rows that belong
    bad = sum(int((e[rq > F(tau - off)] <= tau).sum()) for tau in e[:400])
    assert bad > 0
    # the skip rule at thresholds right at, just above and just below the scores
    k_rel = F(2.0 ** -17)
    c_s = F(F(k_rel * s_bound) - off)
    for tau in np.concatenate([e[:400], np.nextafter(e[:400], F(np.inf)),
                               np.nextafter(e[:400], F(-np.inf))]).astype(F):
        t0 = F(tau + F(k_rel * F(abs(tau))))
        skip = rq > F(t0 + c_s)
        assert (e[skip] > tau).all(), (tau, e[skip].min())
