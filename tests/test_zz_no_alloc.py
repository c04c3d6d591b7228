"""vdbg_flat_search_device_noalloc (scratch in a static device array, nothing allocated)
against vdbg_flat_search_device on the same inputs: ids and distances bit for bit, on two
calls in a row with the second batch smaller, for the GEMM paths (int8 integer rows, fp16
split float rows), a filter, the forced exact re-scan (the array's second part) and the
exact scan without a GEMM; plus its refusals (k above 240, a batch beyond the array)."""
import numpy as np
import pytest
import torch

import vdbg
from vdbg import datagen

pytestmark = pytest.mark.gpu


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _run(ds, fn, q, k, allow=None):
    nq = q.shape[0]
    ids = torch.full((nq, k), -7, dtype=torch.int32, device="cuda")
    d = torch.full((nq, k), -7.0, dtype=torch.float32, device="cuda")
    fn(q.data_ptr(), nq, k, ids.data_ptr(), d.data_ptr(),
       allow_ptr=None if allow is None else allow.data_ptr())
    torch.cuda.synchronize()
    return ids.cpu().numpy().view(np.uint32), d.cpu().numpy()


def _same(a, b, what):
    ai, ad = a
    bi, bd = b
    bad = np.nonzero((ai != bi).any(1) | (ad.view(np.uint32) != bd.view(np.uint32)).any(1))[0]
    assert bad.size == 0, f"{what}: {bad.size} queries differ, first {bad[0]}"


CASES = [
    # name, rows, dim, queries (first call, second call), k
    ("int8 sift-like", lambda: datagen.sift_like(200_000, 128, 2002),
     lambda n, s: datagen.sift_like(n, 128, s), 128, (300, 37), 10),
    ("fp16 split float", lambda: datagen.uniform_rows(60_000, 128, 91),
     lambda n, s: datagen.uniform_rows(n, 128, s), 128, (257, 64), 100),
    ("exact scan, no GEMM", lambda: datagen.uniform_rows(900, 208, 92),
     lambda n, s: datagen.uniform_rows(n, 208, s), 208, (70, 3), 10),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("fallbacks", [0, 2])
def test_noalloc_equals_device_entry(ctx, oracle, case, fallbacks):
    name, make_base, make_q, dim, sizes, k = case
    print(f"noalloc {name} fallbacks={fallbacks}", flush=True)
    base = make_base()
    ds = vdbg.Dataset(ctx, base, dim)
    try:
        ctx.set_test_fallbacks(fallbacks)
        for call, nq in enumerate(sizes):
            qs = make_q(nq, 5000 + call)
            q = _dev(qs)
            want = _run(ds, ds.flat_search_device, q, k)
            got = _run(ds, ds.flat_search_device_noalloc, q, k)
            _same(got, want, f"{name} call {call} nq={nq}")
            if call == 0:
                od, oi = oracle.flat_search(base, qs, k)
                _same(got, (oi, od), f"{name} vs oracle")
    finally:
        ctx.set_test_fallbacks(0)
        ds.close()


def test_noalloc_filter(ctx):
    print("noalloc filter", flush=True)
    base = datagen.uniform_rows(50_000, 128, 93)
    ds = vdbg.Dataset(ctx, base, 128)
    words = np.zeros((50_000 + 63) // 64, np.uint64)
    rows = np.arange(0, 50_000, 7)
    np.bitwise_or.at(words, rows // 64, np.uint64(1) << (rows % 64).astype(np.uint64))
    allow = _dev(words.view(np.int64))
    for call, nq in enumerate((200, 20)):
        q = _dev(datagen.uniform_rows(nq, 128, 6000 + call))
        want = _run(ds, ds.flat_search_device, q, 10, allow)
        got = _run(ds, ds.flat_search_device_noalloc, q, 10, allow)
        _same(got, want, f"filter call {call}")
        assert (got[0] % 7 == 0).all()
    ds.close()


def test_noalloc_refusals(ctx):
    print("noalloc refusals", flush=True)
    base = datagen.sift_like(1_000_000, 128, 2002)
    ds = vdbg.Dataset(ctx, base, 128)
    q = _dev(datagen.sift_like(64, 128, 2003))
    with pytest.raises(vdbg.VdbgError) as e:
        _run(ds, ds.flat_search_device_noalloc, q, 241)
    assert e.value.code == 1
    # a batch beyond the array is refused before anything is queued: the outputs stay
    # untouched and the next call still works
    big = 65536
    qq = _dev(datagen.sift_like(big, 128, 2005))
    ids = torch.full((big, 10), -7, dtype=torch.int32, device="cuda")
    d = torch.zeros((big, 10), dtype=torch.float32, device="cuda")
    with pytest.raises(vdbg.VdbgError) as e:
        ds.flat_search_device_noalloc(qq.data_ptr(), big, 10, ids.data_ptr(), d.data_ptr())
    assert e.value.code == 7
    torch.cuda.synchronize()
    assert (ids == -7).all().item()
    q2 = _dev(datagen.sift_like(33, 128, 2006))
    _same(_run(ds, ds.flat_search_device_noalloc, q2, 10),
          _run(ds, ds.flat_search_device, q2, 10), "after a refusal")
    # about the largest batch the array serves at 1M x 128, k = 10 (bisection over calls
    # that either run or are refused before anything is queued)
    lo, hi = 1, 8192
    while lo < hi:
        mid = (lo + hi + 1) // 2
        qq = _dev(datagen.sift_like(mid, 128, 2004))
        try:
            _run(ds, ds.flat_search_device_noalloc, qq, 10)
            lo = mid
        except vdbg.VdbgError as err:
            assert err.code == 7, err
            hi = mid - 1
    print(f"noalloc: largest batch at 1M x 128, k=10: about {lo} queries", flush=True)
    assert lo >= 256
    ds.close()
