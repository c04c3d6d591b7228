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
        _sig(lib, "or_crc32c", C.c_uint32, [C.c_uint32, C.c_char_p, sz])

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
