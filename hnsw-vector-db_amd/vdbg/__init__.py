"""vdbg: Python bindings (ctypes) for the gfx950 search backend in libvdbg.so.

The product is the C ABI in include/vdbg.h; this module is a thin host-side mirror used by
the tests and the benchmark.  Importing it loads libvdbg.so from this directory and fails
loudly when the library is missing: there is no CPU fallback.
"""
import ctypes as C
import os
import weakref

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libvdbg.so")

METRICS = {"l2": 0, "ip": 1, "cosine": 2}
NO_ID = 0xFFFFFFFF

# Status::Code names (include/vdb/status.h:14-26)
CODE_NAMES = {
    0: "OK", 1: "InvalidArgument", 2: "NotFound", 3: "AlreadyExists", 4: "IOError",
    5: "Corruption", 6: "FailedPrecondition", 7: "ResourceExhausted", 8: "Unavailable",
    9: "NotSupported", 10: "Internal",
}


class VdbgError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"{CODE_NAMES.get(code, code)}: {msg}")
        self.code = code


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"libvdbg.so is not built ({LIB_PATH}); run __graft_entry__.build() first")
    # PyTorch-ROCm carries its own libamdhip64.so.7.  Loaded first, it also serves
    # libvdbg.so (same soname); loaded second, it would bring a second HIP/HSA runtime into
    # the process that finds no GPU.  So when torch is installed it is imported first.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    return C.CDLL(LIB_PATH)


lib = _load()

_vp = C.c_void_p
_sz = C.c_size_t
_SIGS = {
    "vdbg_version": (C.c_int, []),
    "vdbg_last_error": (C.c_char_p, []),
    "vdbg_ctx_create": (C.c_int, [C.c_int, C.POINTER(_vp)]),
    "vdbg_ctx_destroy": (C.c_int, [_vp]),
    "vdbg_ctx_stream": (_vp, [_vp]),
    "vdbg_ctx_synchronize": (C.c_int, [_vp]),
    "vdbg_ctx_set_kernels": (C.c_int, [_vp, C.c_char_p]),
    "vdbg_ctx_kernels": (C.c_char_p, [_vp]),
    "vdbg_ctx_set_fp16_gemm": (C.c_int, [_vp, C.c_int]),
    "vdbg_ctx_set_int8_gemm": (C.c_int, [_vp, C.c_int]),
    "vdbg_ctx_set_ivf_row_sums": (C.c_int, [_vp, C.c_int]),
    "vdbg_ctx_set_int8_float_min_work": (C.c_int, [_vp, C.c_double]),
    "vdbg_ctx_set_test_fallbacks": (C.c_int, [_vp, C.c_int]),
    "vdbg_ctx_set_gated_fallbacks": (C.c_int, [_vp, C.c_int]),
    "vdbg_ctx_set_collection_schedule": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int]),
    "vdbg_profile_enable": (C.c_int, [_vp, C.c_int]),
    "vdbg_profile_reset": (C.c_int, [_vp]),
    "vdbg_profile_get": (C.c_int, [_vp, C.c_char_p, C.POINTER(C.c_double),
                                   C.POINTER(C.c_uint64)]),
    "vdbg_dataset_create": (C.c_int, [_vp, _vp, _sz, _sz, _sz, C.c_int, C.POINTER(_vp)]),
    "vdbg_dataset_create_device": (C.c_int, [_vp, _vp, _sz, _sz, _sz, C.c_int,
                                             C.POINTER(_vp)]),
    "vdbg_dataset_open_vectors": (C.c_int, [_vp, C.c_char_p, _sz, _sz, C.c_int, C.c_uint64,
                                            C.c_int, C.POINTER(_vp)]),
    "vdbg_crc32c_extend": (C.c_uint32, [C.c_uint32, C.c_char_p, _sz]),
    "vdbg_blob_decode": (C.c_int, [C.c_char_p, _sz, C.c_char_p, C.POINTER(_sz),
                                   C.POINTER(_sz)]),
    "vdbg_deletes_decode": (C.c_int, [C.c_char_p, _sz, _sz, _vp, C.POINTER(C.c_uint64)]),
    "vdbg_sq8_load": (C.c_int, [_vp, C.c_char_p, _sz, C.POINTER(_vp)]),
    "vdbg_dataset_set_external_ids": (C.c_int, [_vp, _vp]),
    "vdbg_collection_search_host": (C.c_int, [_vp, _vp, _sz, _sz, C.c_int, _vp, _sz, _sz, _vp,
                                              _vp, _vp, _vp, _vp]),
    "vdbg_collection_search_device": (C.c_int, [_vp, _vp, _sz, _sz, C.c_int, _vp, _sz, _sz,
                                                _vp, _vp, _vp, _vp, _vp, _vp]),
    "vdbg_dataset_destroy": (C.c_int, [_vp]),
    "vdbg_dataset_rows": (_vp, [_vp]),
    "vdbg_flat_search_host": (C.c_int, [_vp, _vp, _sz, _sz, _vp, _vp, _vp,
                                        C.POINTER(C.c_uint64)]),
    "vdbg_flat_search_device": (C.c_int, [_vp, _vp, _sz, _sz, _vp, _vp, _vp, _vp]),
    "vdbg_flat_search_device_noalloc": (C.c_int, [_vp, _vp, _sz, _sz, _vp, _vp, _vp, _vp]),
    "vdbg_last_fallbacks": (C.c_int, [_vp, C.POINTER(C.c_uint64)]),
    "vdbg_last_gemm_bits": (C.c_int, [_vp]),
    "vdbg_sq8_train": (C.c_int, [_vp, _vp, _vp]),
    "vdbg_sq8_create": (C.c_int, [_vp, _vp, _vp, C.POINTER(_vp)]),
    "vdbg_sq8_destroy": (C.c_int, [_vp]),
    "vdbg_sq8_codes": (C.c_int, [_vp, _vp]),
    "vdbg_sq8_search_host": (C.c_int, [_vp, _vp, _sz, _sz, _sz, _vp, _vp, _vp,
                                       C.POINTER(C.c_uint64)]),
    "vdbg_sq8_search_device": (C.c_int, [_vp, _vp, _sz, _sz, _sz, _vp, _vp, _vp, _vp]),
    "vdbg_sq8_graph_info": (C.c_int, [_vp, _vp]),
    "vdbg_sq8_hnsw_search_host": (C.c_int, [_vp, _vp, _sz, _sz, _sz, C.c_int, _vp, _vp, _vp,
                                            _vp]),
    "vdbg_sq8_hnsw_search_device": (C.c_int, [_vp, _vp, _sz, _sz, _sz, C.c_int, _vp, _vp, _vp,
                                              _vp, _vp]),
    "vdbg_ctx_set_host_threads": (C.c_int, [_vp, C.c_int]),
    "vdbg_ctx_set_fp16_single": (C.c_int, [_vp, C.c_int]),
    "vdbg_dataset_create_appendable": (C.c_int, [_vp, _sz, _sz, C.c_int, _sz, C.POINTER(_vp)]),
    "vdbg_dataset_append": (C.c_int, [_vp, _vp, _sz, _vp, C.POINTER(C.c_uint64)]),
    "vdbg_dataset_size": (C.c_int, [_vp, C.POINTER(C.c_uint64)]),
    "vdbg_pqflat_build": (C.c_int, [_vp, _sz, C.c_uint64, _sz, _sz, C.POINTER(_vp)]),
    "vdbg_pqflat_load": (C.c_int, [_vp, C.c_char_p, _sz, C.POINTER(_vp)]),
    "vdbg_pqflat_save": (C.c_int, [_vp, _vp, _sz, C.POINTER(_sz)]),
    "vdbg_pqflat_destroy": (C.c_int, [_vp]),
    "vdbg_pqflat_info": (C.c_int, [_vp, C.POINTER(_sz), _vp]),
    "vdbg_pqflat_codes": (C.c_int, [_vp, _vp]),
    "vdbg_pqflat_search_host": (C.c_int, [_vp, _vp, _sz, _sz, C.c_int, _vp, _vp, _vp, _vp]),
    "vdbg_pqflat_search_device": (C.c_int, [_vp, _vp, _sz, _sz, C.c_int, _vp, _vp, _vp, _vp,
                                            _vp]),
    "vdbg_host_sq8_distance": (C.c_float, [C.c_char_p, C.c_int, _vp, _vp, _vp, _vp, _sz,
                                           C.c_int]),
    "vdbg_ivfpq_load": (C.c_int, [_vp, C.c_char_p, _sz, C.POINTER(_vp)]),
    "vdbg_ivfpq_build": (C.c_int, [_vp, _sz, _sz, C.c_uint64, _sz, _sz, C.POINTER(_vp)]),
    "vdbg_kmeans": (C.c_int, [_vp, _vp, _sz, _sz, _sz, _sz, _sz, C.c_uint64, _sz, C.c_int, _vp,
                              C.POINTER(C.c_double), C.POINTER(_sz)]),
    "vdbg_assign_nearest": (C.c_int, [_vp, _vp, _sz, _sz, _sz, _vp, _sz, _vp, _vp]),
    "vdbg_ivfpq_save": (C.c_int, [_vp, _vp, _sz, C.POINTER(_sz)]),
    "vdbg_ivfpq_destroy": (C.c_int, [_vp]),
    "vdbg_ivfpq_info": (C.c_int, [_vp, C.POINTER(_sz), C.POINTER(_sz), C.POINTER(C.c_int)]),
    "vdbg_ivfpq_list_sizes": (C.c_int, [_vp, _vp]),
    "vdbg_ivfpq_search_host": (C.c_int, [_vp, _vp, _sz, _sz, _sz, C.c_int, _vp, _vp, _vp, _vp]),
    "vdbg_ivfpq_search_device": (C.c_int, [_vp, _vp, _sz, _sz, _sz, C.c_int, _vp, _vp, _vp, _vp,
                                           _vp]),
    "vdbg_rerank_host": (C.c_int, [_vp, _vp, _sz, _vp, _sz, _sz, _vp, _vp, _vp]),
    "vdbg_rerank_device": (C.c_int, [_vp, _vp, _sz, _vp, _sz, _sz, _vp, _vp, _vp, _vp]),
    "vdbg_prepare_queries_host": (C.c_int, [_vp, _vp, _sz, _sz, _sz, C.c_int, _vp]),
    "vdbg_prepare_queries_device": (C.c_int, [_vp, _vp, _sz, _sz, _sz, C.c_int, _vp, _vp]),
    "vdbg_merge_parts_host": (C.c_int, [_vp, _sz, _sz, _sz, _vp, _vp, _vp, _sz, _vp, _vp, _vp]),
    "vdbg_merge_parts_device": (C.c_int, [_vp, _sz, _sz, _sz, _vp, _vp, _vp, _vp, _vp, _vp,
                                          _vp]),
    "vdbg_coalescer_create_flat": (C.c_int, [_vp, _sz, C.c_uint32, C.POINTER(_vp)]),
    "vdbg_coalescer_create_sq8": (C.c_int, [_vp, _sz, C.c_uint32, C.POINTER(_vp)]),
    "vdbg_coalescer_create_sq8_hnsw": (C.c_int, [_vp, _sz, C.c_uint32, C.POINTER(_vp)]),
    "vdbg_coalescer_create_ivfpq": (C.c_int, [_vp, _sz, C.c_uint32, C.POINTER(_vp)]),
    "vdbg_coalescer_create_pqflat": (C.c_int, [_vp, _sz, C.c_uint32, C.POINTER(_vp)]),
    "vdbg_coalescer_search": (C.c_int, [_vp, _vp, _sz, _sz, C.c_int, _vp, _vp, _vp, _vp]),
    "vdbg_coalescer_stats": (C.c_int, [_vp, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
    "vdbg_coalescer_destroy": (C.c_int, [_vp]),
}
for _name, (_res, _args) in _SIGS.items():
    _f = getattr(lib, _name)
    _f.restype = _res
    _f.argtypes = _args


def _check(rc):
    if rc != 0:
        raise VdbgError(rc, lib.vdbg_last_error().decode(errors="replace"))


def _ptr(a):
    return None if a is None else a.ctypes.data_as(_vp)


def padded_dim(dim):
    """PaddedDim (include/vdb/types.h:30-32): a multiple of 16 floats."""
    return (dim + 15) // 16 * 16


def pad_rows(x, pd=None):
    x = np.asarray(x, np.float32)
    n, d = x.shape
    pd = padded_dim(d) if pd is None else pd
    if pd == d:
        return np.ascontiguousarray(x)
    out = np.zeros((n, pd), np.float32)
    out[:, :d] = x
    return out


class Context:
    """A device, its stream and workspace (vdbg_ctx)."""

    def __init__(self, device=0):
        h = _vp()
        _check(lib.vdbg_ctx_create(device, C.byref(h)))
        self.h = h
        self._children = weakref.WeakSet()  # live datasets: closed before the context

    def close(self):
        if self.h:
            for ch in list(self._children):
                ch.close()
            _check(lib.vdbg_ctx_destroy(self.h))
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def stream(self):
        return lib.vdbg_ctx_stream(self.h)

    def synchronize(self):
        _check(lib.vdbg_ctx_synchronize(self.h))

    @property
    def kernels(self):
        """The distance kernel set exact distances follow: scalar, avx2 or avx512."""
        return lib.vdbg_ctx_kernels(self.h).decode()

    def set_kernels(self, name):
        _check(lib.vdbg_ctx_set_kernels(self.h, name.encode()))

    def set_fp16_gemm(self, enable=True):
        """Let flat and SQ8 scans rank on fp16 MFMA (the default): integer rows exactly,
        SQ8 codes and float rows on split fp16 operands.  False always ranks on the fp32
        GEMM.  Results are identical."""
        _check(lib.vdbg_ctx_set_fp16_gemm(self.h, 1 if enable else 0))

    def set_int8_gemm(self, enable=True):
        """Let integer flat rows spanning at most 256 values rank on int8 MFMA (the
        default).  Results are identical."""
        _check(lib.vdbg_ctx_set_int8_gemm(self.h, 1 if enable else 0))

    def set_ivf_row_sums(self, enable=True):
        """Let IVF-PQ L2 scans with precomputed tables rank rows on their per-row term-2
        sums (the default); False builds each probed list's table per query.  Results are
        identical."""
        _check(lib.vdbg_ctx_set_ivf_row_sums(self.h, 1 if enable else 0))

    def set_int8_float_min_work(self, work):
        """Smallest rows x queries x padded_dim of a float-row batch that ranks on the int8
        GEMM (default 2e10).  Results are identical either way."""
        _check(lib.vdbg_ctx_set_int8_float_min_work(self.h, float(work)))

    def set_host_threads(self, n):
        _check(lib.vdbg_ctx_set_host_threads(self.h, n))

    def set_fp16_single(self, enable):
        """Float datasets created from now on hold their high fp16 halves alone (one MFMA
        per product) instead of two-part pairs."""
        _check(lib.vdbg_ctx_set_fp16_single(self.h, 1 if enable else 0))

    def set_test_fallbacks(self, level):
        """Testing: 1 fails every first certificate of the flat / SQ8 scans (second chance),
        2 also every second one (exact re-scan); 0 is the normal path.  Results are
        identical."""
        _check(lib.vdbg_ctx_set_test_fallbacks(self.h, int(level)))

    def set_collection_schedule(self, combine=True, lanes=2, threaded=True):
        """How a collection search schedules its segments' flat scans: one combined scan
        where it applies, else each segment on its own, side by side on `lanes` streams
        (0/1: in turn), each lane issued by its own host thread when threaded."""
        _check(lib.vdbg_ctx_set_collection_schedule(self.h, 1 if combine else 0, int(lanes),
                                                    1 if threaded else 0))

    def set_gated_fallbacks(self, enable=True):
        """Fallback passes queued without host reads (on) or sized from host reads of their
        counts (off); results are identical."""
        _check(lib.vdbg_ctx_set_gated_fallbacks(self.h, 1 if enable else 0))

    def profile(self, enable=True):
        _check(lib.vdbg_profile_enable(self.h, 1 if enable else 0))

    def profile_reset(self):
        _check(lib.vdbg_profile_reset(self.h))

    def profile_get(self, name):
        ms = C.c_double()
        n = C.c_uint64()
        _check(lib.vdbg_profile_get(self.h, name.encode(), C.byref(ms), C.byref(n)))
        return ms.value, n.value

    def last_gemm_bits(self):
        """Input width of the last scan's ranking GEMM: 32, 16, 8 (integers) or 0."""
        return lib.vdbg_last_gemm_bits(self.h)

    def last_fallbacks(self):
        n = C.c_uint64()
        _check(lib.vdbg_last_fallbacks(self.h, C.byref(n)))
        return n.value


class Dataset:
    """A segment's rows resident in HBM (vdbg_dataset)."""

    def __init__(self, ctx, rows, dim, metric="l2"):
        rows = np.ascontiguousarray(rows, np.float32)
        n, pd = rows.shape
        h = _vp()
        _check(lib.vdbg_dataset_create(ctx.h, _ptr(rows), n, dim, pd, METRICS[metric],
                                       C.byref(h)))
        self.ctx, self.h, self.n, self.dim, self.pd = ctx, h, n, dim, pd
        self.metric = metric
        self._children = weakref.WeakSet()  # live SQ8 / IVF-PQ indexes
        ctx._children.add(self)

    @classmethod
    def from_device(cls, ctx, rows_ptr, n, dim, pd, metric="l2"):
        self = cls.__new__(cls)
        h = _vp()
        _check(lib.vdbg_dataset_create_device(ctx.h, rows_ptr, n, dim, pd, METRICS[metric],
                                              C.byref(h)))
        self.ctx, self.h, self.n, self.dim, self.pd = ctx, h, n, dim, pd
        self.metric = metric
        self._children = weakref.WeakSet()
        ctx._children.add(self)
        return self

    @classmethod
    def appendable(cls, ctx, dim, metric="l2", capacity=1024):
        """An empty dataset that takes rows by append (vdb's MutableSegment)."""
        self = cls.__new__(cls)
        h = _vp()
        pd = padded_dim(dim)
        _check(lib.vdbg_dataset_create_appendable(ctx.h, dim, pd, METRICS[metric], capacity,
                                                  C.byref(h)))
        self.ctx, self.h, self.n, self.dim, self.pd = ctx, h, 0, dim, pd
        self.metric = metric
        self._children = weakref.WeakSet()
        ctx._children.add(self)
        return self

    def append(self, rows, ext_ids=None):
        """MutableSegment::Append of rows (n x padded_dim) and their external ids; returns
        the first new row's number."""
        rows = np.ascontiguousarray(rows, np.float32)
        assert rows.ndim == 2 and rows.shape[1] == self.pd
        if ext_ids is not None:
            ext_ids = np.ascontiguousarray(ext_ids, np.uint64)
            assert ext_ids.shape == (rows.shape[0],)
        first = C.c_uint64()
        _check(lib.vdbg_dataset_append(self.h, _ptr(rows), rows.shape[0], _ptr(ext_ids),
                                       C.byref(first)))
        n = C.c_uint64()
        _check(lib.vdbg_dataset_size(self.h, C.byref(n)))
        self.n = n.value
        return first.value

    @classmethod
    def open_vectors(cls, ctx, data, dim, metric="l2", rows=None, verify_crc=True):
        """A segment's vectors.f32 file (bytes) made resident, checked as Segment::Open
        checks it; rows = the manifest's row count (None: the header's)."""
        data = bytes(data)
        self = cls.__new__(cls)
        h = _vp()
        _check(lib.vdbg_dataset_open_vectors(ctx.h, data, len(data), dim, METRICS[metric],
                                             2**64 - 1 if rows is None else rows,
                                             1 if verify_crc else 0, C.byref(h)))
        pd = padded_dim(dim)
        self.ctx, self.h, self.dim, self.pd = ctx, h, dim, pd
        self.n = int.from_bytes(data[16:24], "little")
        self.metric = metric
        self._children = weakref.WeakSet()
        ctx._children.add(self)
        return self

    def close(self):
        if self.h:
            for ch in list(self._children):
                ch.close()
            _check(lib.vdbg_dataset_destroy(self.h))
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_external_ids(self, ids):
        """The segment's external ids (ids.u64), resident for collection_search."""
        ids = np.ascontiguousarray(ids, np.uint64)
        assert ids.shape == (self.n,)
        _check(lib.vdbg_dataset_set_external_ids(self.h, _ptr(ids)))

    def flat_search(self, queries, k, allow=None):
        """Host arrays in and out: (ids uint32 [nq, k], dists float32 [nq, k])."""
        q = np.ascontiguousarray(queries, np.float32)
        nq = q.shape[0]
        assert q.shape[1] == self.pd
        ids = np.empty((nq, k), np.uint32)
        dists = np.empty((nq, k), np.float32)
        if allow is not None:
            allow = np.ascontiguousarray(allow, np.uint64)
        dc = C.c_uint64()
        _check(lib.vdbg_flat_search_host(self.h, _ptr(q), nq, k, _ptr(allow), _ptr(ids),
                                         _ptr(dists), C.byref(dc)))
        return ids, dists

    def rerank(self, queries, cand, k):
        """Rerank: exact distances of each query's candidate rows (cand: (nq, depth) uint32,
        UINT32_MAX = none), top k.  Returns (ids, dists, dist_comps)."""
        q = np.ascontiguousarray(queries, np.float32)
        cand = np.ascontiguousarray(cand, np.uint32)
        nq, depth = cand.shape
        assert q.shape == (nq, self.pd)
        ids = np.empty((nq, k), np.uint32)
        d = np.empty((nq, k), np.float32)
        dc = np.empty(nq, np.uint64)
        _check(lib.vdbg_rerank_host(self.h, _ptr(q), nq, _ptr(cand), depth, k, _ptr(ids), _ptr(d),
                                    _ptr(dc)))
        return ids, d, dc

    def flat_search_device(self, q_ptr, nq, k, ids_ptr, dists_ptr, allow_ptr=None,
                           stream=None):
        """Device pointers (ints), queued on `stream` (None = the context's stream)."""
        _check(lib.vdbg_flat_search_device(self.h, q_ptr, nq, k, allow_ptr, ids_ptr,
                                           dists_ptr, stream))

    def flat_search_device_noalloc(self, q_ptr, nq, k, ids_ptr, dists_ptr, allow_ptr=None,
                                   stream=None):
        """The allocation-free variant (vdbg_flat_search_device_noalloc): k <= 240, scratch
        in a static device array of fixed size."""
        _check(lib.vdbg_flat_search_device_noalloc(self.h, q_ptr, nq, k, allow_ptr, ids_ptr,
                                                   dists_ptr, stream))


class Sq8Index:
    """SQ8 codes of a dataset's rows, resident in HBM (vdbg_sq8)."""

    def __init__(self, ds, vmin=None, scale=None):
        if vmin is None:
            vmin, scale = ds.sq8_train()
        self.vmin = np.ascontiguousarray(vmin, np.float32)
        self.scale = np.ascontiguousarray(scale, np.float32)
        h = _vp()
        _check(lib.vdbg_sq8_create(ds.h, _ptr(self.vmin), _ptr(self.scale), C.byref(h)))
        self.ds, self.h = ds, h
        ds._children.add(self)

    @classmethod
    def load(cls, ds, data):
        """A segment's VDBHSQ81 index file (bytes): quantizer and codes made resident as
        they are."""
        data = bytes(data)
        self = cls.__new__(cls)
        h = _vp()
        _check(lib.vdbg_sq8_load(ds.h, data, len(data), C.byref(h)))
        q = np.frombuffer(data, np.uint8)
        pd = ds.pd
        self.vmin = q[24:24 + 4 * pd].view(np.float32).copy()
        self.scale = q[24 + 4 * pd:24 + 8 * pd].view(np.float32).copy()
        self.ds, self.h = ds, h
        ds._children.add(self)
        return self

    def close(self):
        if self.h:
            lib.vdbg_sq8_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def codes(self):
        out = np.empty((self.ds.n, self.ds.pd), np.uint8)
        _check(lib.vdbg_sq8_codes(self.h, _ptr(out)))
        return out

    def search(self, queries, k, depth, allow=None):
        q = np.ascontiguousarray(queries, np.float32)
        nq = q.shape[0]
        ids = np.empty((nq, k), np.uint32)
        dists = np.empty((nq, k), np.float32)
        if allow is not None:
            allow = np.ascontiguousarray(allow, np.uint64)
        dc = C.c_uint64()
        _check(lib.vdbg_sq8_search_host(self.h, _ptr(q), nq, k, depth, _ptr(allow), _ptr(ids),
                                        _ptr(dists), C.byref(dc)))
        return ids, dists

    def search_device(self, q_ptr, nq, k, depth, ids_ptr, dists_ptr, allow_ptr=None,
                      stream=None):
        _check(lib.vdbg_sq8_search_device(self.h, q_ptr, nq, k, depth, allow_ptr, ids_ptr,
                                          dists_ptr, stream))

    def graph_info(self):
        """(nodes, M, ef_construction, top layer, entry point) of a loaded graph."""
        out = np.empty(5, np.int64)
        _check(lib.vdbg_sq8_graph_info(self.h, _ptr(out)))
        return tuple(int(v) for v in out)

    def hnsw_search(self, queries, k, ef=64, rerank=-1, allow=None):
        """HnswSq8Index::search for a batch: the graph walk on the host, the rerank on the
        GPU.  Returns (ids, dists, distance computations)."""
        q = np.ascontiguousarray(queries, np.float32)
        nq = q.shape[0]
        ids = np.empty((nq, k), np.uint32)
        dists = np.empty((nq, k), np.float32)
        dc = np.empty(nq, np.uint64)
        if allow is not None:
            allow = np.ascontiguousarray(allow, np.uint64)
        _check(lib.vdbg_sq8_hnsw_search_host(self.h, _ptr(q), nq, k, ef, rerank, _ptr(allow),
                                             _ptr(ids), _ptr(dists), _ptr(dc)))
        return ids, dists, dc

    def hnsw_search_device(self, q_ptr, nq, k, ef, rerank, ids_ptr, dists_ptr, allow_ptr=None,
                           dc_ptr=None, stream=None):
        _check(lib.vdbg_sq8_hnsw_search_device(self.h, q_ptr, nq, k, ef, rerank, allow_ptr,
                                               ids_ptr, dists_ptr, dc_ptr, stream))


def host_sq8_distance(kernels, metric, q, codes, vmin, scale, portable=False):
    """The SQ8 distance the HNSW walk computes on the host (pure host code)."""
    q = np.ascontiguousarray(q, np.float32)
    c = np.ascontiguousarray(codes, np.uint8)
    vmin = np.ascontiguousarray(vmin, np.float32)
    scale = np.ascontiguousarray(scale, np.float32)
    m = {"l2": 0, "ip": 1, "cosine": 2}.get(metric, metric)
    return lib.vdbg_host_sq8_distance(kernels.encode(), m, _ptr(q), _ptr(c), _ptr(vmin),
                                      _ptr(scale), q.size, 1 if portable else 0)


def _sq8_train(self):
    vmin = np.empty(self.pd, np.float32)
    scale = np.empty(self.pd, np.float32)
    _check(lib.vdbg_sq8_train(self.h, _ptr(vmin), _ptr(scale)))
    return vmin, scale


Dataset.sq8_train = _sq8_train


class IvfPqIndex:
    """An IVF-PQ index resident in HBM (vdbg_ivfpq), from a VDBIVFP1 file."""

    def __init__(self, ds, h):
        self.ds, self.h = ds, h
        ds._children.add(self)

    @classmethod
    def load(cls, ds, blob):
        blob = bytes(blob)
        h = _vp()
        _check(lib.vdbg_ivfpq_load(ds.h, blob, len(blob), C.byref(h)))
        return cls(ds, h)

    @classmethod
    def build(cls, ds, nlist, m, seed=42, max_points=256, iters=25):
        """IvfPqIndex::build on the GPU (IndexOptions nlist, pq_m, seed,
        max_train_points_per_centroid; k-means iterations)."""
        h = _vp()
        _check(lib.vdbg_ivfpq_build(ds.h, nlist, m, seed, max_points, iters, C.byref(h)))
        return cls(ds, h)

    def close(self):
        if self.h:
            lib.vdbg_ivfpq_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def save(self):
        n = _sz()
        _check(lib.vdbg_ivfpq_save(self.h, None, 0, C.byref(n)))
        buf = C.create_string_buffer(n.value)
        _check(lib.vdbg_ivfpq_save(self.h, buf, n.value, C.byref(n)))
        return buf.raw[:n.value]

    def info(self):
        nl, m, pre = _sz(), _sz(), C.c_int()
        _check(lib.vdbg_ivfpq_info(self.h, C.byref(nl), C.byref(m), C.byref(pre)))
        return nl.value, m.value, bool(pre.value)

    def list_sizes(self):
        nl = self.info()[0]
        out = np.empty(nl, np.uint64)
        _check(lib.vdbg_ivfpq_list_sizes(self.h, _ptr(out)))
        return out

    def search(self, queries, k, nprobe, rerank=-1, allow=None):
        q = np.ascontiguousarray(queries, np.float32)
        nq = q.shape[0]
        ids = np.empty((nq, k), np.uint32)
        dists = np.empty((nq, k), np.float32)
        dc = np.empty(nq, np.uint64)
        if allow is not None:
            allow = np.ascontiguousarray(allow, np.uint64)
        _check(lib.vdbg_ivfpq_search_host(self.h, _ptr(q), nq, k, nprobe, rerank, _ptr(allow),
                                          _ptr(ids), _ptr(dists), _ptr(dc)))
        return ids, dists, dc

    def search_device(self, q_ptr, nq, k, nprobe, rerank, ids_ptr, dists_ptr, allow_ptr=None,
                      dc_ptr=None, stream=None):
        _check(lib.vdbg_ivfpq_search_device(self.h, q_ptr, nq, k, nprobe, rerank, allow_ptr,
                                            ids_ptr, dists_ptr, dc_ptr, stream))


class PqFlatIndex:
    """A PQ-flat index resident in HBM (vdbg_pqflat): PqFlatIndex built on the GPU or loaded
    from a VDBPQFL1 file."""

    def __init__(self, ds, h):
        self.ds, self.h = ds, h
        ds._children.add(self)

    @classmethod
    def build(cls, ds, m, seed=42, max_points=256, iters=25):
        h = _vp()
        _check(lib.vdbg_pqflat_build(ds.h, m, seed, max_points, iters, C.byref(h)))
        return cls(ds, h)

    @classmethod
    def load(cls, ds, blob):
        blob = bytes(blob)
        h = _vp()
        _check(lib.vdbg_pqflat_load(ds.h, blob, len(blob), C.byref(h)))
        return cls(ds, h)

    def close(self):
        if self.h:
            lib.vdbg_pqflat_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def save(self):
        n = _sz()
        _check(lib.vdbg_pqflat_save(self.h, None, 0, C.byref(n)))
        buf = C.create_string_buffer(n.value)
        _check(lib.vdbg_pqflat_save(self.h, buf, n.value, C.byref(n)))
        return buf.raw[:n.value]

    def codes(self):
        m = _sz()
        _check(lib.vdbg_pqflat_info(self.h, C.byref(m), None))
        out = np.empty((self.ds.n, m.value), np.uint8)
        _check(lib.vdbg_pqflat_codes(self.h, _ptr(out)))
        return out

    def search(self, queries, k, rerank=-1, allow=None):
        q = np.ascontiguousarray(queries, np.float32)
        nq = q.shape[0]
        ids = np.empty((nq, k), np.uint32)
        dists = np.empty((nq, k), np.float32)
        dc = np.empty(nq, np.uint64)
        if allow is not None:
            allow = np.ascontiguousarray(allow, np.uint64)
        _check(lib.vdbg_pqflat_search_host(self.h, _ptr(q), nq, k, rerank, _ptr(allow),
                                           _ptr(ids), _ptr(dists), _ptr(dc)))
        return ids, dists, dc

    def search_device(self, q_ptr, nq, k, rerank, ids_ptr, dists_ptr, allow_ptr=None,
                      dc_ptr=None, stream=None):
        _check(lib.vdbg_pqflat_search_device(self.h, q_ptr, nq, k, rerank, allow_ptr, ids_ptr,
                                             dists_ptr, dc_ptr, stream))


class Coalescer:
    """Concurrent one-query searches of one index gathered into device batches
    (vdbg_coalescer_*).  index: a Dataset (flat), Sq8Index (scan, or the HNSW walk with
    hnsw=True), IvfPqIndex or PqFlatIndex.  search() may be called from many threads at once
    (ctypes releases the GIL for the call); each call returns what the index's one-query
    search returns."""

    def __init__(self, index, max_batch=32, max_wait_us=50, hnsw=False):
        h = _vp()
        if isinstance(index, Dataset):
            fn, self.pd = lib.vdbg_coalescer_create_flat, index.pd
        elif isinstance(index, Sq8Index):
            fn = lib.vdbg_coalescer_create_sq8_hnsw if hnsw else lib.vdbg_coalescer_create_sq8
            self.pd = index.ds.pd
        elif isinstance(index, IvfPqIndex):
            fn, self.pd = lib.vdbg_coalescer_create_ivfpq, index.ds.pd
        elif isinstance(index, PqFlatIndex):
            fn, self.pd = lib.vdbg_coalescer_create_pqflat, index.ds.pd
        else:
            raise TypeError("unsupported index type")
        _check(fn(index.h, max_batch, max_wait_us, C.byref(h)))
        self.index, self.h = index, h

    def search(self, query, k, param=0, rerank=0, allow=None):
        """One query (pd floats): (ids uint32 [k], dists float32 [k], dist_comps)."""
        q = np.ascontiguousarray(query, np.float32).reshape(-1)
        assert q.size == self.pd
        ids = np.empty(k, np.uint32)
        d = np.empty(k, np.float32)
        dc = C.c_uint64()
        if allow is not None:
            assert allow.dtype == np.uint64 and allow.flags.c_contiguous
        _check(lib.vdbg_coalescer_search(self.h, _ptr(q), k, param, rerank, _ptr(allow),
                                         _ptr(ids), _ptr(d), C.byref(dc)))
        return ids, d, dc.value

    def stats(self):
        """(batches, queries) run so far."""
        b, q = C.c_uint64(), C.c_uint64()
        _check(lib.vdbg_coalescer_stats(self.h, C.byref(b), C.byref(q)))
        return b.value, q.value

    def close(self):
        if self.h:
            _check(lib.vdbg_coalescer_destroy(self.h))
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class SearchParams(C.Structure):
    """SearchParams (include/vdb/options.h:59-67), vdbg_search_params."""
    _fields_ = [("ef", _sz), ("nprobe", _sz), ("rerank", C.c_int), ("strategy", C.c_int),
                ("prefilter_threshold", _sz), ("post_filter_alpha", _sz)]

    def __init__(self, ef=64, nprobe=16, rerank=-1, strategy="auto", prefilter_threshold=10000,
                 post_filter_alpha=10):
        super().__init__(ef, nprobe, rerank, STRATEGIES[strategy], prefilter_threshold,
                         post_filter_alpha)


STRATEGIES = {"auto": 0, "prefilter": 1, "graph": 2, "post_filter": 3}
PLANS = ["index", "empty", "prefilter_exact", "filtered_index",
         "filtered_index+exact_fallback", "post_filter", "scan", "scan_filter", "host"]


class _Segment(C.Structure):
    _fields_ = [("rows", _vp), ("sq8", _vp), ("ivfpq", _vp), ("deleted_words", _vp),
                ("filter_words", _vp), ("pqflat", _vp), ("memory_part", C.c_int),
                ("host_dists", _vp), ("host_rows", _vp), ("host_ext", _vp),
                ("host_dist_comps", _vp)]


class HostHits:
    """The hits of a disk segment searched on the host (vdb's own SearchDiskSegment over an
    index this library does not hold, such as a float-row HNSW): per query [nq, k] distances
    and rows in ascending (dist, row) order (rows 0xFFFFFFFF after the last hit), each hit's
    external id, and optionally the distance computations per query."""

    def __init__(self, dists, rows, ext, dist_comps=None):
        self.dists = np.ascontiguousarray(dists, np.float32)
        self.rows = np.ascontiguousarray(rows, np.uint32)
        self.ext = np.ascontiguousarray(ext, np.uint64)
        self.dist_comps = None if dist_comps is None else np.ascontiguousarray(dist_comps, np.uint64)
        assert self.dists.shape == self.rows.shape == self.ext.shape


def collection_search(ctx, segments, dim, metric, queries, k, params=None):
    """CollectionImpl::SearchBatch over disk segments (vdbg_collection_search_host).
    segments: (dataset, index or None, deleted words or None, filter words or None[,
    memory part]) per segment, each dataset with its external ids set; a true fifth entry
    marks an in-memory part (the active or a frozen mutable segment), which vdb lists first;
    a HostHits in place of the tuple is a disk segment searched on the host.  Returns
    (external ids uint64 [nq, k], dists float32 [nq, k], distance computations per query,
    plan name per segment)."""
    params = params or SearchParams()
    q = np.ascontiguousarray(queries, np.float32)
    nq = q.shape[0]
    assert q.shape[1] == dim
    keep = []
    arr = (_Segment * max(len(segments), 1))()
    for i, seg in enumerate(segments):
        if isinstance(seg, HostHits):
            assert seg.dists.shape == (nq, k), "host hits are [nq, k]"
            keep.append(seg)
            arr[i] = _Segment(None, None, None, None, None, None, 0, seg.dists.ctypes.data,
                              seg.rows.ctypes.data, seg.ext.ctypes.data,
                              None if seg.dist_comps is None else seg.dist_comps.ctypes.data)
            continue
        ds, ix, deleted, filt = seg[:4]
        memory = bool(seg[4]) if len(seg) > 4 else False
        sq = ix.h if isinstance(ix, Sq8Index) else None
        iv = ix.h if isinstance(ix, IvfPqIndex) else None
        pf = ix.h if isinstance(ix, PqFlatIndex) else None
        dw = None if deleted is None else np.ascontiguousarray(deleted, np.uint64)
        fw = None if filt is None else np.ascontiguousarray(filt, np.uint64)
        keep += [dw, fw]
        arr[i] = _Segment(ds.h, sq, iv, None if dw is None else dw.ctypes.data,
                          None if fw is None else fw.ctypes.data, pf, 1 if memory else 0,
                          None, None, None, None)
    ids = np.empty((nq, k), np.uint64)
    d = np.empty((nq, k), np.float32)
    dc = np.empty(nq, np.uint64)
    plans = np.empty(max(len(segments), 1), np.int32)
    _check(lib.vdbg_collection_search_host(ctx.h, C.cast(arr, _vp), len(segments), dim,
                                           METRICS[metric], _ptr(q), nq, k, C.byref(params),
                                           _ptr(ids), _ptr(d), _ptr(dc), _ptr(plans)))
    return ids, d, dc, [PLANS[p] for p in plans[:len(segments)]]


def collection_search_device(ctx, segments, dim, metric, q_ptr, nq, k, out_ids_ptr,
                             out_dists_ptr, params=None, stream=None):
    """vdbg_collection_search_device: raw queries (nq x dim floats) and the outputs (uint64
    and float32 [nq, k]) in device memory; segments as for collection_search.  Returns
    (distance computations per query, plan name per segment)."""
    params = params or SearchParams()
    keep = []
    arr = (_Segment * max(len(segments), 1))()
    for i, seg in enumerate(segments):
        if isinstance(seg, HostHits):
            keep.append(seg)
            arr[i] = _Segment(None, None, None, None, None, None, 0, seg.dists.ctypes.data,
                              seg.rows.ctypes.data, seg.ext.ctypes.data,
                              None if seg.dist_comps is None else seg.dist_comps.ctypes.data)
            continue
        ds, ix, deleted, filt = seg[:4]
        memory = bool(seg[4]) if len(seg) > 4 else False
        sq = ix.h if isinstance(ix, Sq8Index) else None
        iv = ix.h if isinstance(ix, IvfPqIndex) else None
        pf = ix.h if isinstance(ix, PqFlatIndex) else None
        dw = None if deleted is None else np.ascontiguousarray(deleted, np.uint64)
        fw = None if filt is None else np.ascontiguousarray(filt, np.uint64)
        keep += [dw, fw]
        arr[i] = _Segment(ds.h, sq, iv, None if dw is None else dw.ctypes.data,
                          None if fw is None else fw.ctypes.data, pf, 1 if memory else 0,
                          None, None, None, None)
    dc = np.empty(max(nq, 1), np.uint64)
    plans = np.empty(max(len(segments), 1), np.int32)
    _check(lib.vdbg_collection_search_device(ctx.h, C.cast(arr, _vp), len(segments), dim,
                                             METRICS[metric], q_ptr, nq, k, C.byref(params),
                                             out_ids_ptr, out_dists_ptr, _ptr(dc), _ptr(plans),
                                             stream))
    return dc[:nq], [PLANS[p] for p in plans[:len(segments)]]


def crc32c(data, crc=0):
    """crc32c::Extend (src/util/crc32c.h:9-13)."""
    data = bytes(data)
    return int(lib.vdbg_crc32c_extend(crc, data, len(data)))


def blob_payload(data, magic):
    """DecodeBlob (src/storage/file_format.cc:21-33): the checked payload of a blob file."""
    data = bytes(data)
    off, n = _sz(), _sz()
    _check(lib.vdbg_blob_decode(data, len(data), magic.encode(), C.byref(off), C.byref(n)))
    return data[off.value:off.value + n.value]


def decode_deletes(data, rows):
    """A deletes-<n>.roar blob file as dense words (bit r set = row r deleted) and the
    number of deleted rows."""
    data = bytes(data)
    words = np.zeros((rows + 63) // 64, np.uint64)
    count = C.c_uint64()
    _check(lib.vdbg_deletes_decode(data, len(data), rows, _ptr(words) if rows else None,
                                   C.byref(count)))
    return words, int(count.value)


def kmeans(ctx, data, k, iters=25, seed=1234, max_points=256, kmeanspp=True, d=None):
    """KMeans over host rows (n x stride); returns (centroids k x d, inertia, reseeds)."""
    data = np.ascontiguousarray(data, np.float32)
    n, stride = data.shape
    d = stride if d is None else d
    cen = np.empty((k, d), np.float32)
    inertia = C.c_double()
    reseeds = _sz()
    _check(lib.vdbg_kmeans(ctx.h, _ptr(data), n, d, stride, k, iters, seed, max_points,
                           1 if kmeanspp else 0, _ptr(cen), C.byref(inertia), C.byref(reseeds)))
    return cen, inertia.value, reseeds.value


def assign_nearest(ctx, data, centroids, d=None):
    data = np.ascontiguousarray(data, np.float32)
    centroids = np.ascontiguousarray(centroids, np.float32)
    n, stride = data.shape
    d = stride if d is None else d
    assign = np.empty(n, np.uint32)
    dist = np.empty(n, np.float32)
    _check(lib.vdbg_assign_nearest(ctx.h, _ptr(data), n, d, stride, _ptr(centroids),
                                   centroids.shape[0], _ptr(assign), _ptr(dist)))
    return assign, dist


def prepare_queries(ctx, raw, pd, metric="l2"):
    """PrepareQuery for every row of raw (nq x dim): padded, checked, normalised for cosine."""
    raw = np.ascontiguousarray(raw, np.float32)
    nq, dim = raw.shape
    out = np.empty((nq, pd), np.float32)
    _check(lib.vdbg_prepare_queries_host(ctx.h, _ptr(raw), nq, dim, pd, METRICS[metric],
                                         _ptr(out)))
    return out


def merge_parts(ctx, part_dists, part_rows, ext_ids, part_offsets):
    """Cross-segment merge: part_* are (nparts, nq, k); returns (ext ids, dists), nq x k."""
    part_dists = np.ascontiguousarray(part_dists, np.float32)
    part_rows = np.ascontiguousarray(part_rows, np.uint32)
    ext_ids = np.ascontiguousarray(ext_ids, np.uint64)
    part_offsets = np.ascontiguousarray(part_offsets, np.uint64)
    nparts, nq, k = part_dists.shape
    out_ext = np.empty((nq, k), np.uint64)
    out_d = np.empty((nq, k), np.float32)
    _check(lib.vdbg_merge_parts_host(ctx.h, nq, nparts, k, _ptr(part_dists), _ptr(part_rows),
                                     _ptr(ext_ids), ext_ids.size, _ptr(part_offsets),
                                     _ptr(out_ext), _ptr(out_d)))
    return out_ext, out_d


def prepare_queries_device(ctx, raw_ptr, nq, dim, pd, metric, out_ptr, stream=None):
    _check(lib.vdbg_prepare_queries_device(ctx.h, raw_ptr, nq, dim, pd, METRICS[metric],
                                           out_ptr, stream))


def merge_parts_device(ctx, nq, nparts, k, dists_ptr, rows_ptr, ext_ptr, offsets_ptr,
                       out_ext_ptr, out_dists_ptr, stream=None):
    _check(lib.vdbg_merge_parts_device(ctx.h, nq, nparts, k, dists_ptr, rows_ptr, ext_ptr,
                                       offsets_ptr, out_ext_ptr, out_dists_ptr, stream))
