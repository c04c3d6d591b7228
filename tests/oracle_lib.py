"""ctypes bindings for the oracle libraries (test infrastructure only).

liboracle.so is the C restatement of vdb's hot path (oracle/vdb_oracle.c); libvdbref.so
(oracle/_ref/, present only where it was built from the reference's sources) is the
reference's own code behind a C driver.  Both are test oracles: product code never loads them.
"""
import ctypes as C
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "liboracle.so")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libvdbref.so")

KSET = {"scalar": 0, "avx2": 1, "avx512": 2}
METRIC = {"l2": 0, "ip": 1, "cosine": 2}

f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
u64p = np.ctypeslib.ndpointer(np.uint64, flags="C_CONTIGUOUS")
u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
sz = C.c_size_t


def _opt(ptr_type):
    """Argument type that also accepts None (a null pointer)."""

    class _Opt:
        @classmethod
        def from_param(cls, obj):
            if obj is None:
                return None
            return ptr_type.from_param(obj)

    return _Opt


def _sig(lib, name, res, args):
    f = getattr(lib, name)
    f.restype = res
    f.argtypes = args
    return f


class Oracle:
    def __init__(self, path=ORACLE_SO):
        self.lib = lib = C.CDLL(path)
        _sig(lib, "or_l2", C.c_float, [C.c_int, f32p, f32p, sz])
        _sig(lib, "or_dot", C.c_float, [C.c_int, f32p, f32p, sz])
        _sig(lib, "or_metric_dist", C.c_float, [C.c_int, C.c_int, f32p, f32p, sz])
        _sig(lib, "or_sq8_l2", C.c_float, [C.c_int, f32p, u8p, f32p, f32p, sz])
        _sig(lib, "or_sq8_ip", C.c_float, [C.c_int, f32p, u8p, f32p, f32p, sz])
        _sig(lib, "or_l2sq_any", C.c_float, [f32p, f32p, sz])
        _sig(lib, "or_dot_any", C.c_float, [f32p, f32p, sz])
        _sig(lib, "or_topk", sz, [f32p, u32p, sz, sz, f32p, u32p])
        _sig(lib, "or_flat_search_batch", None,
             [C.c_int, C.c_int, f32p, sz, sz, f32p, sz, sz, _opt(u64p), f32p, u32p, C.c_int])
        _sig(lib, "or_rerank", sz, [C.c_int, C.c_int, f32p, sz, f32p, u32p, sz, sz, f32p, u32p])
        _sig(lib, "or_sq8_train", None, [f32p, sz, sz, sz, f32p, f32p])
        _sig(lib, "or_sq8_encode_rows", None, [f32p, sz, sz, sz, f32p, f32p, u8p])
        _sig(lib, "or_sq8_decode", None, [u8p, sz, f32p, f32p, f32p])
        _sig(lib, "or_sq8_search_batch", None,
             [C.c_int, C.c_int, f32p, u8p, sz, sz, f32p, f32p, f32p, sz, sz, sz, _opt(u64p),
              f32p, u32p, C.c_int])
        _sig(lib, "or_pq_encode", None, [f32p, sz, sz, f32p, u8p])
        _sig(lib, "or_pq_compute_table", None, [f32p, sz, sz, f32p, C.c_int, f32p])
        _sig(lib, "or_pq_adc", C.c_float, [f32p, sz, u8p])
        _sig(lib, "or_assign_nearest", None,
             [C.c_int, f32p, sz, sz, sz, f32p, sz, u32p, _opt(f32p), C.c_int])
        _sig(lib, "or_ivfpq_term2", None, [f32p, sz, sz, f32p, sz, sz, f32p])
        _sig(lib, "or_ivfpq_search_batch", None,
             [C.c_int, C.c_int, f32p, sz, sz, f32p, sz, f32p, sz, u64p, u32p, u8p, _opt(f32p),
              f32p, sz, sz, sz, C.c_int, _opt(u64p), f32p, u32p, _opt(u64p), C.c_int])
        _sig(lib, "or_normalize", C.c_int, [f32p, sz])
        _sig(lib, "or_merge_parts", sz, [sz, sz, f32p, u32p, u64p, u64p, f32p, u64p])
        _sig(lib, "or_plan_segment", C.c_int,
             [C.c_int, sz, sz, sz, C.c_int, C.c_int, sz, sz, sz, sz, C.POINTER(C.c_size_t)])
        _sig(lib, "or_crc32c", C.c_uint32, [C.c_uint32, C.c_char_p, sz])
        _sig(lib, "or_pqflat_search_batch", None,
             [C.c_int, C.c_int, f32p, sz, sz, f32p, sz, sz, u8p, f32p, sz, sz, C.c_int,
              _opt(u64p), f32p, u32p, _opt(u64p), C.c_int])
        _sig(lib, "or_hnsw_sq8_search_file", C.c_int,
             [C.c_int, C.c_int, C.c_char_p, sz, f32p, sz, sz, f32p, sz, sz, sz, C.c_int,
              _opt(u64p), f32p, u32p, _opt(u64p), C.c_int])

    # -- convenience wrappers (numpy in, numpy out)
    def flat_search(self, base, queries, k, metric="l2", kset="avx512", allow=None,
                    threads=8):
        base = np.ascontiguousarray(base, np.float32)
        queries = np.ascontiguousarray(queries, np.float32)
        nq, pd = queries.shape
        od = np.empty((nq, k), np.float32)
        oi = np.empty((nq, k), np.uint32)
        self.lib.or_flat_search_batch(KSET[kset], METRIC[metric], base, base.shape[0], pd,
                                      queries, nq, k, allow, od, oi, threads)
        return od, oi

    def sq8_train(self, base, dim):
        rows, pd = base.shape
        vmin = np.empty(pd, np.float32)
        scale = np.empty(pd, np.float32)
        self.lib.or_sq8_train(np.ascontiguousarray(base, np.float32), rows, dim, pd, vmin,
                              scale)
        return vmin, scale

    def sq8_encode(self, base, dim, vmin, scale):
        rows, pd = base.shape
        codes = np.empty((rows, pd), np.uint8)
        self.lib.or_sq8_encode_rows(np.ascontiguousarray(base, np.float32), rows, dim, pd,
                                    vmin, scale, codes)
        return codes

    def sq8_search(self, base, codes, vmin, scale, queries, k, depth, metric="l2",
                   kset="avx512", allow=None, threads=8):
        nq, pd = queries.shape
        od = np.empty((nq, k), np.float32)
        oi = np.empty((nq, k), np.uint32)
        self.lib.or_sq8_search_batch(KSET[kset], METRIC[metric],
                                     np.ascontiguousarray(base, np.float32),
                                     np.ascontiguousarray(codes), base.shape[0], pd, vmin,
                                     scale, np.ascontiguousarray(queries, np.float32), nq, k,
                                     depth, allow, od, oi, threads)
        return od, oi


    def pqflat_search(self, ix, base, queries, k, rerank=-1, metric="l2", allow=None,
                      kset="avx512", threads=8):
        """PqFlatIndex::search over an index parsed with ivf_file.parse_pqflat."""
        base = np.ascontiguousarray(base, np.float32)
        queries = np.ascontiguousarray(queries, np.float32)
        nq, pd = queries.shape
        od = np.empty((nq, k), np.float32)
        oi = np.empty((nq, k), np.uint32)
        dc = np.empty(nq, np.uint64)
        self.lib.or_pqflat_search_batch(KSET[kset], METRIC[metric], base, base.shape[0], pd,
                                        ix["pq_centroids"], ix["m"], ix["dim"] // ix["m"],
                                        ix["codes"], queries, nq, k, rerank, allow, od, oi, dc,
                                        threads)
        return od, oi, dc

    def hnsw_sq8_search(self, file, base, queries, k, ef=64, rerank=-1, metric="l2",
                        allow=None, kset="avx512", threads=8):
        """HnswSq8Index::search per query over a VDBHSQ81 file's quantizer, codes and graph,
        reranked on base.  Returns (dists, ids, distance computations)."""
        base = np.ascontiguousarray(base, np.float32)
        queries = np.ascontiguousarray(queries, np.float32)
        nq, pd = queries.shape
        od = np.empty((nq, k), np.float32)
        oi = np.empty((nq, k), np.uint32)
        dc = np.empty(nq, np.uint64)
        file = bytes(file)
        rc = self.lib.or_hnsw_sq8_search_file(KSET[kset], METRIC[metric], file, len(file), base,
                                              base.shape[0], pd, queries, nq, k, ef, rerank,
                                              allow, od, oi, dc, threads)
        if rc != 0:
            raise ValueError("the index file does not parse")
        return od, oi, dc

    def ivfpq_search(self, ix, term2, base, queries, k, nprobe, rerank, metric="l2",
                     allow=None, kset="avx512"):
        """IvfPqIndex::search over an index parsed with ivf_file.parse_ivfpq."""
        nq = len(queries)
        od = np.empty((nq, k), np.float32)
        oi = np.empty((nq, k), np.uint32)
        dc = np.empty(nq, np.uint64)
        self.lib.or_ivfpq_search_batch(KSET[kset], METRIC[metric], np.ascontiguousarray(base),
                                       ix["dim"], ix["pd"], ix["coarse"], ix["nlist"],
                                       ix["pq_centroids"], ix["m"], ix["list_off"],
                                       ix["list_ids"], ix["list_codes"], term2,
                                       np.ascontiguousarray(queries, np.float32), nq, k,
                                       nprobe, rerank, allow, od, oi, dc, 8)
        return od, oi, dc

    def segment_hits(self, sg, metric, q, k, ef=64, nprobe=16, rerank=-1, strategy=0,
                     prefilter_threshold=10000, post_filter_alpha=10, kset="avx512"):
        """SearchDiskSegment (planner.cc:42-129) of one segment of collection_search on
        prepared queries q (nq, pd): (dists, rows) [nq, k], distance computations per query
        and the plan name.  A "host" segment returns its given hits; an "hnsw" one (vdb's
        HnswIndex over a VDBHNSW1 file) takes each HnswIndex::search from sg["recorded"],
        keyed by (k, ef, allowed words or None as bytes)."""
        nq = q.shape[0]
        names = ["index", "empty", "prefilter_exact", "filtered_index",
                 "filtered_index+exact_fallback", "post_filter", "scan", "scan_filter", "host"]
        if sg["kind"] == "host":
            od, oi, dc = sg["hits"]
            return od, oi, np.asarray(dc, np.uint64), "host"

        def count(words, n):
            bits = np.unpackbits(np.ascontiguousarray(words, np.uint64).view(np.uint8),
                                 bitorder="little")[:n]
            return int(bits.sum())

        def clip(words, n):
            w = np.ascontiguousarray(words, np.uint64).copy()
            if n % 64:
                w[-1] &= np.uint64((1 << (n % 64)) - 1)
            return w

        base = np.ascontiguousarray(sg["base"], np.float32)
        n = base.shape[0]
        deleted = sg.get("deleted")
        filt = sg.get("filter")
        ndel = 0 if deleted is None else count(deleted, n)
        live = n - min(n, ndel)
        del_allow = None if ndel == 0 else clip(~np.asarray(deleted, np.uint64), n)
        bm, matches = None, 0
        if filt is not None:
            bm = np.asarray(filt, np.uint64).copy()
            if ndel > 0:
                bm &= ~np.asarray(deleted, np.uint64)
            bm = clip(bm, n)
            matches = count(bm, n)
        if sg["kind"] == "memory":
            # SearchMutable (planner.cc:131-151) -> MutableSegment::Search
            # (mutable_segment.cc:46-64): the rows not deleted and matching the filter,
            # exactly, counted as distance computations
            allow = None
            if filt is not None or ndel > 0:
                allow = np.full((n + 63) // 64, np.iinfo(np.uint64).max, np.uint64)
                if filt is not None:
                    allow &= np.asarray(filt, np.uint64)
                if ndel > 0:
                    allow &= ~np.asarray(deleted, np.uint64)
                allow = clip(allow, n)
            matches = n if allow is None else count(allow, n)
            od, oi = self.flat_search(base, q, k, metric=metric, kset=kset, allow=allow)
            return od, oi, np.full(nq, matches, np.uint64), names[7 if filt is not None else 6]
        npb = C.c_size_t()
        plan = self.lib.or_plan_segment(1 if filt is not None else 0, n, ndel, matches,
                                        1 if sg["kind"] == "flat" else 0, strategy, ef, k,
                                        nprobe, prefilter_threshold, C.byref(npb))

        def index_search(kk, allow, ef_=ef):
            if sg["kind"] == "hnsw":
                key = (int(kk), int(max(ef_, kk)),
                       None if allow is None else np.ascontiguousarray(allow, np.uint64).tobytes())
                if key not in sg["recorded"]:
                    raise KeyError(f"no recorded HnswIndex::search for k={kk}, ef={ef_}")
                od, oi, dc = sg["recorded"][key]
                return od.copy(), oi.copy(), dc.copy()
            if sg["kind"] == "pqflat":
                return self.pqflat_search(sg["pq"], base, q, kk, rerank, metric, allow,
                                          kset=kset)
            if sg["kind"] == "hnsw_sq8":
                od, oi, dc = self.hnsw_sq8_search(sg["file"], base, q, kk, ef_, rerank,
                                                  metric=metric, allow=allow, kset=kset)
                return od, oi, dc
            if sg["kind"] == "ivf":
                od, oi, dc = self.ivfpq_search(sg["ix"], sg["term2"], base, q, kk,
                                               npb.value, rerank, metric, allow, kset=kset)
                return od, oi, dc
            if sg["kind"] == "sq8":
                depth = max(ef_, kk) if rerank < 0 else rerank
                od, oi = self.sq8_search(base, sg["codes"], sg["vmin"], sg["scale"], q, kk,
                                         depth, metric=metric, kset=kset, allow=allow)
                extra = min(max(depth, kk), n) if depth > 0 else 0
                return od, oi, np.full(nq, n + extra, np.uint64)
            od, oi = self.flat_search(base, q, kk, metric=metric, kset=kset, allow=allow)
            return od, oi, np.full(nq, n, np.uint64)

        if plan == 0:
            od, oi, dc = index_search(k, del_allow)
        elif plan == 1:
            od = np.full((nq, k), np.inf, np.float32)
            oi = np.full((nq, k), 0xFFFFFFFF, np.uint32)
            dc = np.zeros(nq, np.uint64)
        elif plan == 2:
            od, oi = self.flat_search(base, q, k, metric=metric, kset=kset, allow=bm)
            dc = np.full(nq, matches, np.uint64)
        elif plan == 3:
            od, oi, dc = index_search(k, bm)
            if strategy == 0:
                hits = (oi != 0xFFFFFFFF).sum(axis=1)
                short = np.nonzero(hits < min(k, matches))[0]
                if short.size:
                    plan = 4
                    xd, xi = self.flat_search(base, q, k, metric=metric, kset=kset,
                                              allow=bm)
                    od[short], oi[short] = xd[short], xi[short]
                    dc = dc.copy()
                    dc[short] += np.uint64(matches)
        else:
            kk = min(max(live, 1), k * max(1, post_filter_alpha))
            wd, wi, dc = index_search(kk, del_allow, max(ef, kk))  # pp.ef (:113-114)
            od = np.full((nq, k), np.inf, np.float32)
            oi = np.full((nq, k), 0xFFFFFFFF, np.uint32)
            for i in range(nq):
                out = 0
                for j in range(kk):
                    r = int(wi[i, j])
                    if r == 0xFFFFFFFF or out >= k:
                        break
                    if (int(bm[r >> 6]) >> (r & 63)) & 1:
                        oi[i, out], od[i, out] = r, wd[i, j]
                        out += 1
        return od, oi, dc.astype(np.uint64), names[plan]

    def collection_search(self, segments, dim, metric, raw, k, ef=64, nprobe=16, rerank=-1,
                          strategy=0, prefilter_threshold=10000, post_filter_alpha=10,
                          kset="avx512"):
        """CollectionImpl::SearchBatch (src/engine/collection_impl.cc:1036-1135) over disk
        segments, composed from the oracle's parts: PrepareQuery (:1023-1034, or_normalize),
        each segment's plan (SearchDiskSegment, planner.cc:42-129: or_plan_segment, the
        index searches, the exact fallback of :103-108, the post filter of :110-127), and
        the merge (:1076-1112, or_merge_parts), one query at a time.

        segments: dicts with base (n, pd) fp32, ext (n,) uint64, kind "flat" | "sq8" |
        "hnsw_sq8" | "ivf", deleted / filter (dense words or None); sq8 (the GPU's exhaustive
        SQ8 scan index, built from rows, no graph): codes, vmin, scale; hnsw_sq8 (vdb's
        HnswSq8Index): file (the VDBHSQ81 bytes); ivf: ix (parsed VDBIVFP1) and term2 (or
        None); pqflat: pq (a parsed VDBPQFL1); memory: an in-memory part (the active or a
        frozen mutable segment, listed first), scanned exactly; hnsw (vdb's HnswIndex over a
        VDBHNSW1 file): recorded, its HnswIndex::search results (segment_hits); host: hits,
        (dists, rows, dist comps) of a segment already searched.  Returns (ext ids, dists,
        dist comps, plan names)."""
        nq = raw.shape[0]
        pd = (dim + 15) // 16 * 16
        q = np.zeros((nq, pd), np.float32)
        q[:, :dim] = raw
        if not np.isfinite(raw).all():
            raise ValueError("query has a NaN or infinite value")
        if metric == "cosine":
            for i in range(nq):
                if self.lib.or_normalize(q[i], dim) != 1:
                    raise ValueError("a zero query cannot be normalized for cosine")
        np_ = len(segments)
        pdist = np.full((max(np_, 1), nq, k), np.inf, np.float32)
        prow = np.full((max(np_, 1), nq, k), 0xFFFFFFFF, np.uint32)
        dcs = np.zeros(nq, np.uint64)
        plans = []
        for p, sg in enumerate(segments):
            od, oi, dc, plan = self.segment_hits(sg, metric, q, k, ef, nprobe, rerank, strategy,
                                                 prefilter_threshold, post_filter_alpha, kset)
            pdist[p], prow[p] = od, oi
            dcs += np.asarray(dc).astype(np.uint64)
            plans.append(plan)
        ext = np.ascontiguousarray(np.concatenate([sg["ext"] for sg in segments])
                                   if segments else np.zeros(1, np.uint64), np.uint64)
        off = np.concatenate([[0], np.cumsum([sg["base"].shape[0] for sg in segments])[:-1]]
                             ).astype(np.uint64) if segments else np.zeros(1, np.uint64)
        oe = np.full((nq, k), np.iinfo(np.uint64).max, np.uint64)
        odd = np.full((nq, k), np.inf, np.float32)
        for i in range(nq):
            e = np.empty(k, np.uint64)
            dd = np.empty(k, np.float32)
            cnt = self.lib.or_merge_parts(max(np_, 1), k, np.ascontiguousarray(pdist[:, i, :]),
                                          np.ascontiguousarray(prow[:, i, :]), ext, off, dd, e)
            oe[i, :cnt], odd[i, :cnt] = e[:cnt], dd[:cnt]
        return oe, odd, dcs, plans


class Reference:
    """The reference's own code (oracle/_ref/libvdbref.so); None when not built."""

    def __init__(self, path=REF_SO):
        self.lib = lib = C.CDLL(path)
        cs = C.c_char_p
        _sig(lib, "ref_best_kernels", cs, [])
        _sig(lib, "ref_has_kernels", C.c_int, [cs])
        _sig(lib, "ref_l2", C.c_float, [cs, f32p, f32p, sz])
        _sig(lib, "ref_dot", C.c_float, [cs, f32p, f32p, sz])
        _sig(lib, "ref_sq8_l2", C.c_float, [cs, f32p, u8p, f32p, f32p, sz])
        _sig(lib, "ref_sq8_ip", C.c_float, [cs, f32p, u8p, f32p, f32p, sz])
        _sig(lib, "ref_l2sq_any", C.c_float, [f32p, f32p, sz])
        _sig(lib, "ref_dot_any", C.c_float, [f32p, f32p, sz])
        _sig(lib, "ref_topk", sz, [f32p, u32p, sz, sz, f32p, u32p])
        _sig(lib, "ref_flat_search_batch", None,
             [cs, C.c_int, f32p, sz, sz, sz, f32p, sz, sz, _opt(u64p), f32p, u32p, C.c_int])
        _sig(lib, "ref_flat_index_batch", None,
             [C.c_int, f32p, sz, sz, sz, f32p, sz, sz, f32p, u32p, C.c_int])
        _sig(lib, "ref_flat_search_blocked", None,
             [cs, C.c_int, f32p, sz, sz, sz, f32p, sz, sz, f32p, u32p, C.c_int])
        _sig(lib, "ref_rerank", None,
             [cs, C.c_int, f32p, sz, sz, sz, f32p, u32p, sz, sz, f32p, u32p])
        _sig(lib, "ref_sq8_train_encode", None, [f32p, sz, sz, sz, f32p, f32p, _opt(u8p)])
        _sig(lib, "ref_sq8_search_batch", None,
             [cs, C.c_int, f32p, u8p, sz, sz, sz, f32p, f32p, f32p, sz, sz, sz, f32p, u32p,
              C.c_int])
        _sig(lib, "ref_pq_train", C.c_int, [f32p, sz, sz, sz, sz, C.c_uint64, sz, f32p])
        _sig(lib, "ref_pq_encode", C.c_int, [f32p, sz, sz, f32p, sz, sz, u8p])
        _sig(lib, "ref_pq_table", C.c_int, [f32p, sz, sz, f32p, C.c_int, f32p])
        _sig(lib, "ref_pq_adc", C.c_float, [f32p, sz, sz, f32p, u8p])
        _sig(lib, "ref_kmeans", C.c_int,
             [f32p, sz, sz, sz, sz, sz, C.c_uint64, sz, C.c_int, f32p])
        _sig(lib, "ref_assign_nearest", None, [f32p, sz, sz, sz, f32p, sz, u32p, _opt(f32p)])
        _sig(lib, "ref_ivfpq_build", C.c_int,
             [C.c_int, f32p, sz, sz, sz, sz, sz, C.c_uint64, sz, C.POINTER(C.c_void_p),
              C.POINTER(C.c_size_t), C.c_int])
        _sig(lib, "ref_ivfpq_search_batch", C.c_int,
             [C.c_int, C.c_char_p, sz, f32p, sz, sz, sz, f32p, sz, sz, sz, C.c_int, _opt(u64p),
              f32p, u32p, _opt(u64p), C.c_int])
        _sig(lib, "ref_normalize", C.c_int, [f32p, sz])
        _sig(lib, "ref_crc32c", C.c_uint32, [C.c_char_p, sz])
        _sig(lib, "ref_hnsw_sq8_file", sz,
             [C.c_int, f32p, sz, sz, sz, sz, sz, C.c_uint64, C.c_void_p, sz])
        _sig(lib, "ref_pqflat_file", sz,
             [C.c_int, f32p, sz, sz, sz, sz, C.c_uint64, sz, C.c_void_p, sz])
        _sig(lib, "ref_pqflat_search_batch", C.c_int,
             [C.c_int, C.c_char_p, sz, f32p, sz, sz, sz, f32p, sz, sz, C.c_int, _opt(u64p),
              f32p, u32p, _opt(u64p), C.c_int])
        _sig(lib, "ref_hnsw_sq8_search_batch", C.c_int,
             [C.c_int, C.c_char_p, sz, f32p, sz, sz, sz, f32p, sz, sz, sz, C.c_int, _opt(u64p),
              f32p, u32p, _opt(u64p), C.c_int])
        _sig(lib, "ref_hnsw_sq8_file_mt", sz,
             [C.c_int, f32p, sz, sz, sz, sz, sz, C.c_uint64, C.c_int, C.c_void_p])
        _sig(lib, "ref_hnsw_file", sz,
             [C.c_int, f32p, sz, sz, sz, sz, sz, C.c_uint64, C.c_void_p, sz])
        _sig(lib, "ref_hnsw_search_batch", C.c_int,
             [C.c_int, C.c_char_p, sz, f32p, sz, sz, sz, f32p, sz, sz, sz, _opt(u64p),
              f32p, u32p, _opt(u64p), C.c_int])
        _sig(lib, "ref_filtered_collection_search", C.c_int,
             [C.c_int, C.c_void_p, C.c_void_p, sz, sz, sz, C.c_void_p, u64p, f32p, sz, sz,
              u64p, f32p, C.c_int])

    def filtered_collection_search(self, segs, dim, allows, ext, raw, k, metric="cosine",
                                   threads=8):
        """CollectionImpl::Search over flat segments with a filter: segs are (n_p, pd)
        arrays, allows their dense words, ext the concatenated external ids, raw the
        unprepared queries (nq, dim).  Returns (ext ids, dists), nq x k."""
        nseg = len(segs)
        pd = segs[0].shape[1]
        segs = [np.ascontiguousarray(s, np.float32) for s in segs]
        allows = [np.ascontiguousarray(a, np.uint64) for a in allows]
        rows_p = (C.c_void_p * nseg)(*[s.ctypes.data for s in segs])
        n_p = (C.c_size_t * nseg)(*[s.shape[0] for s in segs])
        allow_p = (C.c_void_p * nseg)(*[a.ctypes.data for a in allows])
        raw = np.ascontiguousarray(raw, np.float32)
        nq = raw.shape[0]
        oe = np.empty((nq, k), np.uint64)
        od = np.empty((nq, k), np.float32)
        rc = self.lib.ref_filtered_collection_search(
            METRIC[metric], C.cast(rows_p, C.c_void_p), C.cast(n_p, C.c_void_p), nseg, dim, pd,
            C.cast(allow_p, C.c_void_p), np.ascontiguousarray(ext, np.uint64), raw, nq, k, oe,
            od, threads)
        if rc != 0:
            raise ValueError("a query was rejected by PrepareQuery")
        return oe, od

    def pqflat_file(self, base, dim, m, metric="l2", seed=42, max_points=256):
        base = np.ascontiguousarray(base, np.float32)
        n, pd = base.shape
        size = self.lib.ref_pqflat_file(METRIC[metric], base, n, dim, pd, m, seed, max_points,
                                        None, 0)
        if size == 0:
            raise RuntimeError("ref_pqflat_file failed")
        buf = C.create_string_buffer(size)
        self.lib.ref_pqflat_file(METRIC[metric], base, n, dim, pd, m, seed, max_points, buf, size)
        return buf.raw

    def pqflat_search(self, file, base, dim, queries, k, rerank=-1, metric="l2", allow=None,
                      threads=8):
        base = np.ascontiguousarray(base, np.float32)
        queries = np.ascontiguousarray(queries, np.float32)
        nq, pd = queries.shape
        od = np.empty((nq, k), np.float32)
        oi = np.empty((nq, k), np.uint32)
        dc = np.empty(nq, np.uint64)
        file = bytes(file)
        rc = self.lib.ref_pqflat_search_batch(METRIC[metric], file, len(file), base,
                                              base.shape[0], dim, pd, queries, nq, k, rerank,
                                              allow, od, oi, dc, threads)
        if rc != 0:
            raise ValueError("LoadIndex refused the file")
        return od, oi, dc

    def hnsw_sq8_file(self, base, dim, M=16, ef_construction=200, seed=42, metric="l2",
                      threads=8):
        """HnswSq8Index::build on a pool of threads + save: the VDBHSQ81 file bytes."""
        base = np.ascontiguousarray(base, np.float32)
        n, pd = base.shape
        p = C.c_void_p()
        size = self.lib.ref_hnsw_sq8_file_mt(METRIC[metric], base, n, dim, pd, M,
                                             ef_construction, seed, threads, C.byref(p))
        if size == 0:
            raise RuntimeError("HnswSq8Index::build failed")
        return C.string_at(p.value, size)

    def hnsw_file(self, base, dim, M=16, ef_construction=100, seed=42, metric="l2"):
        """HnswIndex::build (single-threaded) + save: the VDBHNSW1 file bytes."""
        base = np.ascontiguousarray(base, np.float32)
        n, pd = base.shape
        size = self.lib.ref_hnsw_file(METRIC[metric], base, n, dim, pd, M, ef_construction,
                                      seed, None, 0)
        buf = C.create_string_buffer(size)
        assert self.lib.ref_hnsw_file(METRIC[metric], base, n, dim, pd, M, ef_construction,
                                      seed, buf, size) == size
        return buf.raw

    def hnsw_search(self, file, base, dim, queries, k, ef=64, metric="l2", allow=None,
                    threads=8):
        """LoadIndex of a VDBHNSW1 file and HnswIndex::search per query.  Returns (dists,
        ids, distance computations)."""
        base = np.ascontiguousarray(base, np.float32)
        queries = np.ascontiguousarray(queries, np.float32)
        nq, pd = queries.shape
        od = np.empty((nq, k), np.float32)
        oi = np.empty((nq, k), np.uint32)
        dc = np.empty(nq, np.uint64)
        file = bytes(file)
        rc = self.lib.ref_hnsw_search_batch(METRIC[metric], file, len(file), base, base.shape[0],
                                            dim, pd, queries, nq, k, ef, allow, od, oi, dc,
                                            threads)
        if rc != 0:
            raise ValueError("LoadIndex refused the file")
        return od, oi, dc

    def hnsw_sq8_search(self, file, base, dim, queries, k, ef=64, rerank=-1, metric="l2",
                        allow=None, threads=8):
        """LoadIndex of a VDBHSQ81 file and HnswSq8Index::search per query, with the
        reference's own kernel set.  Returns (dists, ids, distance computations)."""
        base = np.ascontiguousarray(base, np.float32)
        queries = np.ascontiguousarray(queries, np.float32)
        nq, pd = queries.shape
        od = np.empty((nq, k), np.float32)
        oi = np.empty((nq, k), np.uint32)
        dc = np.empty(nq, np.uint64)
        file = bytes(file)
        rc = self.lib.ref_hnsw_sq8_search_batch(METRIC[metric], file, len(file), base,
                                                base.shape[0], dim, pd, queries, nq, k, ef,
                                                rerank, allow, od, oi, dc, threads)
        if rc != 0:
            raise ValueError("LoadIndex refused the file")
        return od, oi, dc

    def flat_search(self, base, dim, queries, k, metric="l2", kset="avx512", allow=None,
                    threads=8):
        base = np.ascontiguousarray(base, np.float32)
        queries = np.ascontiguousarray(queries, np.float32)
        nq, pd = queries.shape
        od = np.empty((nq, k), np.float32)
        oi = np.empty((nq, k), np.uint32)
        self.lib.ref_flat_search_batch(kset.encode(), METRIC[metric], base, base.shape[0],
                                       dim, pd, queries, nq, k, allow, od, oi, threads)
        return od, oi

    def ivfpq_build(self, base, dim, nlist, m, seed=42, max_points=256, metric="l2",
                    threads=8):
        base = np.ascontiguousarray(base, np.float32)
        p = C.c_void_p()
        n = C.c_size_t()
        rc = self.lib.ref_ivfpq_build(METRIC[metric], base, base.shape[0], dim, base.shape[1],
                                      nlist, m, seed, max_points, C.byref(p), C.byref(n),
                                      threads)
        if rc != 0:
            raise RuntimeError(f"ref_ivfpq_build failed: {rc}")
        return C.string_at(p.value, n.value)


def load_oracle():
    return Oracle()


def load_reference():
    if not os.path.exists(REF_SO):
        return None
    return Reference()
