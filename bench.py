"""Benchmark: batch QPS of vdb's nearest-neighbour scans on one MI355X.

Workload (one "step" = one batch search over data resident in HBM):
  flat    exact L2 over 1M x 128 fp32 SIFT-like rows (integer values in [0, 255] from a
          1,000-centre mixture), 10,000 queries from the same mixture, k = 10.  This is the
          headline line (`value`).
  sq8     the same rows as SQ8 codes (trained on all rows), top-100 by SQ8 distance, fp32
          rerank to k = 10.
  ivfpq   IVF-PQ over the same rows, nlist 4,096 (k-means 20 iterations, seed 42), m = 16,
          nprobe 64, rerank 100 -> k = 10; built on the GPU.  Also swept over nprobe
          16/32/64/128 at rerank 0 and 100.
  flat_uniform  exact L2 over 100,000 x 128 rows uniform in [0, 1), 1,000 queries, k = 10
          (real-valued rows: the high-half fp16 GEMM with certificates).
  filtered  the collection read path: 5M unit rows of 384 dims (10,000-centre mixture, cosine)
          in 8 segments of 625,000, 2% of rows deleted, a filter passing 1%, 10% or 50% of
          rows; 4,096 raw queries go through PrepareQuery, the filtered exact scan of every
          segment and the cross-segment merge.
  hnsw_sq8  vdb's HNSW-SQ8 index (a VDBHSQ81 file built by vdb's own code over 320,000 of the
          rows): the graph walk on host threads and the beams reranked on the GPU, batched and
          one query per call, against the reference's HnswSq8Index::search.
  pqflat  the PQ flat scan (m = 16) over the 1M rows, against PqFlatIndex::search.
  append  appends of one and 100 rows to an appendable dataset, alone and beside searches.
  per_query  one-query calls from 16, 32 and 64 native threads (tests/cpp/per_query_load)
          through the coalescer, and direct one-query calls for comparison.
The flat path also records batch sizes 1, 64 and 1,024 and k = 100 at the full batch.
Queries, rows, codes and lists are resident before the timed region.  Each path's dominant
kernel is timed with HIP events on the stream it runs on; its roofline fraction uses the
algorithmic work (MFMA flops for the GEMM scans, code + id bytes for the IVF list scan).
Next to each, the reference's own CPU code (oracle/_ref, or the oracle's restatement where
that is not built) is timed on a bounded query sample on this host's cores, and the GPU
results on that sample are compared with it.
"""
import argparse
import json
import os
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "hnsw-vector-db_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))

METRIC = "batch QPS at k=10 (flat/SQ8/IVF-PQ, 1M×128); achieved HBM TB/s / MFMA %"
FP32_MFMA_PEAK_TFLOPS = 157.3
FP16_MFMA_PEAK_TFLOPS = 2500.0  # dense
INT8_MFMA_PEAK_TOPS = 5000.0    # dense
HBM_PEAK_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


PROFILES = {"flat": "flat_gemm8_sift_like_1m_x128_k10_b10000.md",
            "sq8": "sq8_gemm8_sift_like_1m_x128_d100_b10000.md",
            "ivfpq": "ivf_scan_sift_like_1m_nlist4096_m16_nprobe64.md"}


def profiled_traffic(path):
    """HBM bytes per launch of the path's dominant kernel, as measured by the rocprofv3
    FETCH_SIZE / WRITE_SIZE runs summarised under profiles/ (None when absent)."""
    f = os.path.join(ROOT, "profiles", PROFILES.get(path, ""))
    if not os.path.isfile(f):
        return None
    for line in open(f):
        if line.startswith("HBM bytes per launch (calibrated):"):
            try:
                return float(line.split(":")[1].split()[0])
            except ValueError:
                return None
    return None


def cpu_threads():
    """Host threads for the CPU baseline: every core this process may run on, capped by
    OMP_NUM_THREADS when the environment sets one (the host share of one GPU)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    cap = os.environ.get("OMP_NUM_THREADS", "")
    if cap.isdigit() and int(cap) > 0:
        n = min(n, int(cap))
    return max(1, n)


def cpu_model_name():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def host_rate(fn, nq, reps=3):
    """Queries per second of a call that takes host queries and returns host results (query
    upload, search, result download), the best of `reps` calls after one warm-up."""
    fn()
    best = float("inf")
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        best = min(best, time.perf_counter() - t0)
    return round(nq / best, 1), round(best * 1e3, 3)


def timed(ctx, torch, fn, steps, warmup, kernels):
    """Wall time of `steps` calls after `warmup`, with per-kernel profiling off (its events
    add host work to every launch), then, when kernel times are wanted, the same number of
    calls again with profiling on for the per-kernel event times (kernel totals over those
    calls, so per-step figures divide by `steps` as before).  Exact re-scans are counted call
    by call in that second pass (reading the count waits for the device, so the timed pass
    does not read it; the calls are deterministic)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    ctx.profile(False)
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ctx.profile(bool(kernels))
    ctx.profile_reset()
    fallbacks = 0
    for _ in range(steps):
        fn()
        fallbacks += ctx.last_fallbacks()
    torch.cuda.synchronize()
    prof = {k: ctx.profile_get(k) for k in kernels}
    ctx.profile(False)
    return elapsed, prof, fallbacks


def _words(allowed):
    """Dense row mask: bit r of word r / 64 set when row r is allowed."""
    n = allowed.size
    by = np.packbits(allowed, bitorder="little")
    w = np.zeros(((n + 63) // 64) * 8, np.uint8)
    w[:by.size] = by
    return w.view(np.uint64)


def run_filtered(args, ctx, torch, ref, threads, cpu_model):
    import vdbg
    from vdbg import datagen

    dim = pd = 384
    nseg, nq, k = 8, args.f_nq, args.k
    seg_n = args.f_rows // nseg
    N = seg_n * nseg
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream().cuda_stream
    want_cpu = not args.no_cpu and ref is not None
    log(f"filtered: generating {N}x{dim} unit rows in {nseg} segments on the device")
    t0 = time.perf_counter()
    dss, host_rows = [], []
    for p in range(nseg):
        rows = datagen.clustered_unit_t(torch, seg_n, dim, 5002, 5001, 10000, 1.0, dev,
                                        start_row=p * seg_n)
        dss.append(vdbg.Dataset.from_device(ctx, rows.data_ptr(), seg_n, dim, pd, "cosine"))
        if want_cpu:
            host_rows.append(rows.cpu().numpy())
        del rows
    raw = datagen.clustered_unit_t(torch, nq, dim, 5005, 5001, 10000, 1.0, dev, unit=False)
    raw_h = raw.cpu().numpy()
    torch.cuda.synchronize()
    # row attributes: deleted ~ Bernoulli(0.02), filter bucket ~ U{0..99}
    deleted = datagen.uniform01(5004, 0, N) < np.float32(0.02)
    bucket = datagen.rand_u64(5006, 0, N) % np.uint64(100)
    log(f"filtered: data ready in {time.perf_counter() - t0:.1f} s")
    for p in range(nseg):  # external ids of the one-call collection search
        dss[p].set_external_ids(np.arange(p * seg_n, (p + 1) * seg_n, dtype=np.uint64))
    ext_dev = torch.arange(N, dtype=torch.int64, device=dev)
    off_dev = torch.arange(0, N, seg_n, dtype=torch.int64, device=dev)[:nseg].contiguous()
    q_prep = torch.empty((nq, pd), dtype=torch.float32, device=dev)
    part_ids = torch.empty((nseg, nq, k), dtype=torch.int32, device=dev)
    part_d = torch.empty((nseg, nq, k), dtype=torch.float32, device=dev)
    out_ext = torch.empty((nq, k), dtype=torch.int64, device=dev)
    out_d = torch.empty((nq, k), dtype=torch.float32, device=dev)
    out = {"rows": N, "segments": nseg, "dim": dim, "queries": nq, "k": k,
           "deleted_frac": round(float(deleted.mean()), 5), "selectivity": {}}
    samples = {1: 4096, 10: 1024, 50: 256}
    for sel in (1, 10, 50):
        allowed = (bucket < np.uint64(sel)) & ~deleted
        words_h = [_words(allowed[p * seg_n:(p + 1) * seg_n]) for p in range(nseg)]
        masks = [torch.from_numpy(w.view(np.int64)).to(dev) for w in words_h]
        n_allowed = int(allowed.sum())

        # the batch as vdb's SearchBatch sees it, in one device call
        # (vdbg_collection_search_device): the raw queries and the results in HBM, each
        # segment's filter and delete words on the host (SegmentColumns::Evaluate and
        # DeleteBits), from which the planner takes its counts; the segments' filtered scans
        # run side by side on the call's lanes, then the merge
        filt_h = [_words(bucket[p * seg_n:(p + 1) * seg_n] < np.uint64(sel)) for p in range(nseg)]
        del_h = [_words(deleted[p * seg_n:(p + 1) * seg_n]) for p in range(nseg)]
        segs = [(dss[p], None, del_h[p], filt_h[p]) for p in range(nseg)]
        out_ext2 = torch.empty((nq, k), dtype=torch.int64, device=dev)
        out_d2 = torch.empty((nq, k), dtype=torch.float32, device=dev)

        def step():
            vdbg.collection_search_device(ctx, segs, dim, "cosine", raw.data_ptr(), nq, k,
                                          out_ext2.data_ptr(), out_d2.data_ptr(), stream=stream)

        names = ["prepare_queries", "compact", "query_prep", "sample_gemm", "kth", "flat_gemm",
                 "select", "exact_scan", "merge", "merge_parts"]
        el, prof, fb = timed(ctx, torch, step, args.steps, args.warmup, names)
        g_ms = prof["flat_gemm"][0] / args.steps
        flops = 2.0 * n_allowed * pd * nq
        r = {"allowed_rows": n_allowed, "qps": round(nq * args.steps / el, 1),
             "ms_per_step": round(el * 1e3 / args.steps, 3),
             "call": "vdbg_collection_search_device (plans from host words; the segments' "
                     "allowed rows scanned as one set up to 262,144 rows, else each segment "
                     "on 2 threaded lanes; merge)",
             "gemm_ms_per_step": round(g_ms, 3),
             "gemm_TFLOPs": round(flops / (g_ms * 1e-3) / 1e12, 2) if g_ms > 0 else None,
             "gemm_note": "GEMM time summed over the segments' launches, which overlap on the "
                          "lanes",
             "mfma_inputs": {8: "i8 two-part rows x two-part queries (4 int8 MFMA products each)",
                             16: "f16 high halves of rows and queries (1 MFMA product each)"}
                            .get(ctx.last_gemm_bits(), "f32"),
             "kernel_ms_per_step": {kk: round(v[0] / args.steps, 4) for kk, v in prof.items()},
             "exact_rescans": fb}
        log(f"filtered {sel}%: {r['qps']:.0f} q/s, {n_allowed} rows allowed")

        # the same batch composed from the single-segment calls: PrepareQuery, a filtered
        # scan per segment under device words (each counts its words on the device), merge
        def step_c():
            vdbg.prepare_queries_device(ctx, raw.data_ptr(), nq, dim, pd, "cosine",
                                        q_prep.data_ptr(), stream)
            for p in range(nseg):
                dss[p].flat_search_device(q_prep.data_ptr(), nq, k, part_ids[p].data_ptr(),
                                          part_d[p].data_ptr(), allow_ptr=masks[p].data_ptr(),
                                          stream=stream)
            vdbg.merge_parts_device(ctx, nq, nseg, k, part_d.data_ptr(), part_ids.data_ptr(),
                                    ext_dev.data_ptr(), off_dev.data_ptr(), out_ext.data_ptr(),
                                    out_d.data_ptr(), stream)

        el_c, _, fb_c = timed(ctx, torch, step_c, args.steps, 1, [])
        r["composed_device_path"] = {
            "qps": round(nq * args.steps / el_c, 1), "ms_per_step": round(el_c * 1e3 / args.steps, 3),
            "exact_rescans": fb_c,
            "equal_to_one_call": bool(
                np.array_equal(out_ext2.cpu().numpy(), out_ext.cpu().numpy()) and
                np.array_equal(out_d2.cpu().numpy().view(np.uint32),
                               out_d.cpu().numpy().view(np.uint32)))}
        log(f"filtered {sel}% composed: {r['composed_device_path']['qps']:.0f} q/s, equal "
            f"{r['composed_device_path']['equal_to_one_call']}")
        # the one-call C ABI with host queries in and host results out
        # (vdbg_collection_search_host): PCIe included
        ce, cd, _, plans = vdbg.collection_search(ctx, segs, dim, "cosine", raw_h, k)
        for _ in range(args.warmup):
            vdbg.collection_search(ctx, segs, dim, "cosine", raw_h, k)
        torch.cuda.synchronize()
        per_call = []
        t0 = time.perf_counter()
        for _ in range(args.steps):
            t1 = time.perf_counter()
            vdbg.collection_search(ctx, segs, dim, "cosine", raw_h, k)
            per_call.append(time.perf_counter() - t1)
        dt = time.perf_counter() - t0
        r["one_call_host"] = {
            "qps": round(nq * args.steps / dt, 1), "ms_per_step": round(dt * 1e3 / args.steps, 3),
            "median_ms_per_call": round(float(np.median(per_call)) * 1e3, 3),
            "plans": sorted(set(plans)),
            "equal_to_device_path": bool(
                np.array_equal(ce, out_ext2.cpu().numpy().view(np.uint64)) and
                np.array_equal(cd.view(np.uint32), out_d2.cpu().numpy().view(np.uint32)))}
        log(f"filtered {sel}% one call (host in/out): {r['one_call_host']['qps']:.0f} q/s, "
            f"equal {r['one_call_host']['equal_to_device_path']}")
        if want_cpu:
            s = min(samples[sel], nq)
            t0 = time.perf_counter()
            re_, rd_ = ref.filtered_collection_search(
                host_rows, dim, words_h, np.arange(N, dtype=np.uint64), raw_h[:s], k,
                threads=threads)
            dt = time.perf_counter() - t0
            ge = out_ext2[:s].cpu().numpy().view(np.uint64)
            gd = out_d2[:s].cpu().numpy()
            r["cpu_baseline"] = {
                "value": round(s / dt, 2), "unit": "queries/s", "cores": threads,
                "kind": "reference", "cpu_model": cpu_model,
                "sample": f"{s} of the {nq} queries: PrepareQuery, ExactOverBitmap over the "
                          f"allowed rows of each of the {nseg} segments (reference kernels and "
                          f"TopK), merge; {threads} threads, {dt:.1f} s"}
            r["parity_on_cpu_sample"] = bool(np.array_equal(ge, re_) and np.array_equal(
                gd.view(np.uint32), rd_.view(np.uint32)))
            log(f"filtered {sel}% cpu: {s / dt:.1f} q/s, parity {r['parity_on_cpu_sample']}")
        out["selectivity"][f"{sel}%"] = r
        del masks
    for d in dss:
        d.close()
    return out


def run_hnsw_sq8(args, ctx, torch, ref, base, queries, threads, cpu_model):
    """HnswSq8Index::search (hnsw_index.cc:82-100) on a segment of vdb's third compaction tier
    (320,000 of the SIFT-like rows, options.h:46-48: 20,000 x 4^2) with vdb's default graph
    (M 16, ef_construction 200, seed 42): the graph walk on the host threads, the beams'
    float rerank in one GPU launch.  vdb builds a segment's graph on the CPU and the backend
    reads the saved VDBHSQ81 file, so the file here is vdb's own build (HnswSq8Index::build on
    a thread pool, through the reference's code); without it the path is skipped."""
    import vdbg

    if ref is None:
        return {"skipped": "the VDBHSQ81 file is vdb's own CPU build (oracle/_ref not built or "
                           "--no-cpu)"}
    n, dim, k, ef, rr = 320_000, base.shape[1], args.k, 64, -1
    rows = np.ascontiguousarray(base[:n])
    t0 = time.perf_counter()
    blob = ref.hnsw_sq8_file(rows, dim, M=16, ef_construction=200, seed=42, threads=threads)
    build_s = time.perf_counter() - t0
    log(f"hnsw_sq8: vdb's graph over {n} rows built on {threads} threads in {build_s:.1f} s")
    ds = vdbg.Dataset(ctx, rows, dim)
    sq = vdbg.Sq8Index.load(ds, blob)
    nq = len(queries)
    dev = torch.device("cuda:0")
    q_dev = torch.from_numpy(np.ascontiguousarray(queries)).to(dev)
    ids = torch.empty((nq, k), dtype=torch.int32, device=dev)
    dd = torch.empty((nq, k), dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream().cuda_stream

    def step():
        sq.hnsw_search_device(q_dev.data_ptr(), nq, k, ef, rr, ids.data_ptr(), dd.data_ptr(),
                              stream=stream)

    steps = max(1, min(args.steps, 5))
    el, prof, _ = timed(ctx, torch, step, steps, 1, ["rerank"])
    gi = ids.cpu().numpy().view(np.uint32).copy()
    gd = dd.cpu().numpy().copy()
    rr_ms = prof["rerank"][0] / max(1, prof["rerank"][1])
    depth = ef  # rerank -1: depth max(ef, k) (hnsw_index.cc:88)
    r = {"qps": nq * steps / el, "ms_per_step": el * 1e3 / steps, "rows": n, "dim": dim,
         "k": k, "ef": ef, "rerank": rr, "M": 16, "ef_construction": 200,
         "graph_build_s": round(build_s, 2), "walk_threads": threads,
         "kernel": "k_rerank", "kernel_ms": rr_ms, "bound": "cache",
         "rerank_bytes_per_launch": nq * depth * dim,
         "achieved": nq * depth * dim / (rr_ms * 1e-3) / 1e9, "unit": "GB/s",
         "peak": HBM_PEAK_GBS,
         "note": "walk on the host threads (vdb's HnswGraph::search over the SQ8 codes, "
                 "restated), the beams of the whole batch reranked in one GPU launch; the "
                 "rows are integers, so the exact re-score reads each candidate's int8 copy "
                 "(dim bytes, counted here); candidates repeat across queries and the "
                 f"{n * dim / 1e6:.0f} MB int8 copy stays in the on-die caches, so 'achieved' "
                 "is bytes requested, not HBM traffic"}
    log(f"hnsw_sq8: {r['qps']:.0f} q/s batched (walk on {threads} threads), rerank "
        f"{rr_ms:.3f} ms per {nq} queries")
    # one query per call, as vdb's Index::search sends it (host query in, host result out)
    s1 = 400
    sq.hnsw_search(queries[:1], k, ef, rr)
    t0 = time.perf_counter()
    for i in range(s1):
        sq.hnsw_search(queries[i:i + 1], k, ef, rr)
    per_q = (time.perf_counter() - t0) / s1
    r["one_query_per_call"] = {"us_per_query": round(per_q * 1e6, 1),
                               "qps_one_thread": round(1.0 / per_q, 1)}
    s = min(nq, 4000)
    qs = np.ascontiguousarray(queries[:s])
    t0 = time.perf_counter()
    od, oi, _ = ref.hnsw_sq8_search(blob, rows, dim, qs, k, ef, rr, "l2", None, threads)
    dt = time.perf_counter() - t0
    t0 = time.perf_counter()
    ref.hnsw_sq8_search(blob, rows, dim, np.ascontiguousarray(queries[:s1]), k, ef, rr, "l2",
                        None, 1)
    dt1 = (time.perf_counter() - t0) / s1
    r["cpu_baseline"] = {
        "value": s / dt, "unit": "queries/s", "cores": threads, "kind": "reference",
        "cpu_model": cpu_model,
        "sample": f"{s} queries, HnswSq8Index::search (ef {ef}, rerank max(ef, k)) on the same "
                  f"file, {threads} threads, {dt:.1f} s",
        "one_thread_us_per_query": round(dt1 * 1e6, 1)}
    r["parity_on_cpu_sample"] = bool(np.array_equal(gi[:s], oi) and
                                     np.array_equal(gd[:s].view(np.uint32), od.view(np.uint32)))
    log(f"hnsw_sq8: one query per call {per_q * 1e6:.1f} us (reference, one thread: "
        f"{dt1 * 1e6:.1f} us); cpu {s / dt:.0f} q/s, parity {r['parity_on_cpu_sample']}")
    sq.close()
    ds.close()
    return r


def run_pqflat(args, ctx, torch, ref, ds, base, queries, threads, cpu_model):
    """PqFlatIndex (ivf_pq.cc:41-98) over the 1M SIFT-like rows, built on the GPU as vdb builds
    it (m 16, seed 42, 256 points per centroid, 25 k-means iterations): per query the ADC of
    every code, then the float rerank of the top max(10 k, 100) (RerankDepth, :16-19)."""
    import vdbg

    N, dim = base.shape
    k, m = args.k, 16
    t0 = time.perf_counter()
    pq = vdbg.PqFlatIndex.build(ds, m, seed=42, max_points=256, iters=25)
    build_s = time.perf_counter() - t0
    nq = min(len(queries), 2000)
    dev = torch.device("cuda:0")
    q_dev = torch.from_numpy(np.ascontiguousarray(queries[:nq])).to(dev)
    ids = torch.empty((nq, k), dtype=torch.int32, device=dev)
    dd = torch.empty((nq, k), dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream().cuda_stream

    def step():
        pq.search_device(q_dev.data_ptr(), nq, k, -1, ids.data_ptr(), dd.data_ptr(),
                         stream=stream)

    steps = max(1, min(args.steps, 5))
    el, prof, _ = timed(ctx, torch, step, steps, 1, ["pq_tables", "exact_scan", "merge",
                                                     "rerank"])
    gi = ids.cpu().numpy().view(np.uint32).copy()
    gd = dd.cpu().numpy().copy()
    sc_ms = prof["exact_scan"][0] / max(1, prof["exact_scan"][1])
    code_bytes = nq * N * m
    r = {"qps": nq * steps / el, "ms_per_step": el * 1e3 / steps, "batch": nq, "m": m,
         "build_s": round(build_s, 2), "kernel": "k_exact_scan over PQ codes (ADC, wave top-k per row split)",
         "kernel_ms": sc_ms, "bound": "hbm", "algorithmic_bytes_per_launch": code_bytes,
         "achieved": code_bytes / (sc_ms * 1e-3) / 1e9 if sc_ms > 0 else None, "unit": "GB/s",
         "peak": HBM_PEAK_GBS,
         "kernel_ms_per_step": {kk: v[0] / steps for kk, v in prof.items()},
         "note": "the 16 MB of codes stay in L2 / MALL across queries: 'achieved' counts the "
                 "codes each query reads (n m bytes), not HBM traffic"}
    log(f"pqflat: {r['qps']:.0f} q/s, scan {sc_ms:.3f} ms per {nq} queries")
    if ref is not None:
        blob = pq.save()
        s = 500
        qs = np.ascontiguousarray(queries[:s])
        t0 = time.perf_counter()
        od, oi, _ = ref.pqflat_search(blob, base, dim, qs, k, -1, "l2", None, threads)
        dt = time.perf_counter() - t0
        r["cpu_baseline"] = {
            "value": s / dt, "unit": "queries/s", "cores": threads, "kind": "reference",
            "cpu_model": cpu_model,
            "sample": f"{s} queries, PqFlatIndex::search (rerank max(10 k, 100)) on the same "
                      f"VDBPQFL1 file, {threads} threads, {dt:.1f} s"}
        r["parity_on_cpu_sample"] = bool(np.array_equal(gi[:s], oi) and
                                         np.array_equal(gd[:s].view(np.uint32), od.view(np.uint32)))
        log(f"pqflat cpu: {s / dt:.1f} q/s, parity {r['parity_on_cpu_sample']}")
    pq.close()
    return r


def run_per_query(args):
    """vdb's per-query path: pool workers each call Index::search with one query
    (collection_impl.cc:1120-1130).  tests/cpp/per_query_load drives T native threads of
    one-query calls on a 1M x 128 integer-row flat dataset of its own (k = 10), through the
    coalescer (vdbg_coalescer_search) and, for comparison, as direct one-query host calls;
    every answer of its first pass is checked against one batched call."""
    drv = os.path.join(ROOT, "tests", "cpp", "per_query_load")
    if not os.path.exists(drv):
        log("per_query: tests/cpp/per_query_load is not built")
        return None
    out = {}
    for name, extra in (("direct_16_threads", ["--direct", "--threads", "16"]),
                        ("coalesced_16_threads", ["--threads", "16", "--max-batch", "16"]),
                        ("coalesced_32_threads", ["--threads", "32", "--max-batch", "32"]),
                        ("coalesced_64_threads", ["--threads", "64", "--max-batch", "32"])):
        r = subprocess.run([drv, "--rows", str(args.n), "--dim", "128", "--k", str(args.k),
                            "--queries", "2048", "--seconds", "2", "--wait-us", "50", *extra],
                           capture_output=True, text=True, timeout=300)
        if r.returncode != 0:
            raise RuntimeError(f"per_query_load {name}: rc {r.returncode}: {r.stderr[-500:]}")
        rep = json.loads(r.stdout.strip().splitlines()[-1])
        out[name] = {"qps": rep["qps"], "mean_batch": rep["mean_batch"],
                     "differ_from_batch": rep["differ_from_batch"]}
        log(f"per_query {name}: {rep['qps']:.0f} q/s, mean batch {rep['mean_batch']:.1f}")
    out["note"] = ("one-query flat calls (1M x 128 integer rows, k = 10) from native threads; "
                   "differ_from_batch counts queries whose answer differs from the same "
                   "query's row of one batched call (2,048 checked)")
    return out


def run_append(args, ctx, torch, base):
    """MutableSegment::Append (mutable_segment.cc:24-44) on an appendable dataset: single rows
    (vdb appends one row per upsert) and 100-row calls, alone and while another context
    searches on another thread (batches of 64 queries over 100,000 rows)."""
    import threading

    import vdbg

    dim = base.shape[1]

    def appends(rows_per_call, calls):
        ap = vdbg.Dataset.appendable(ctx, dim, "l2", capacity=1 << 20)
        ext = np.arange(rows_per_call * calls, dtype=np.uint64)
        t0 = time.perf_counter()
        for c in range(calls):
            a = c * rows_per_call
            ap.append(base[a:a + rows_per_call], ext[a:a + rows_per_call])
        dt = time.perf_counter() - t0
        ap.close()
        return {"calls": calls, "rows_per_call": rows_per_call,
                "us_per_call": round(dt / calls * 1e6, 1),
                "rows_per_s": round(rows_per_call * calls / dt, 1)}

    r = {"alone": {"one_row": appends(1, 2000), "hundred_rows": appends(100, 300)}}
    ctx2 = vdbg.Context(0)
    ds2 = vdbg.Dataset(ctx2, np.ascontiguousarray(base[:100_000]), dim)
    q = np.ascontiguousarray(base[200_000:200_064])
    stop = threading.Event()
    done = [0]

    def searcher():
        while not stop.is_set():
            ds2.flat_search(q, 10)
            done[0] += 1

    th = threading.Thread(target=searcher)
    th.start()
    time.sleep(0.2)
    try:
        t0 = time.perf_counter()
        n0 = done[0]
        one = appends(1, 2000)
        hundred = appends(100, 300)
        dt = time.perf_counter() - t0
        r["with_search_on_another_context"] = {
            "one_row": one, "hundred_rows": hundred,
            "searches_per_s": round((done[0] - n0) / dt, 1)}
    finally:
        stop.set()
        th.join()
    t0 = time.perf_counter()
    for _ in range(200):
        ds2.flat_search(q, 10)
    r["searches_per_s_alone"] = round(200 / (time.perf_counter() - t0), 1)
    ds2.close()
    ctx2.close()
    log(f"append: one row {r['alone']['one_row']['us_per_call']} us, 100 rows "
        f"{r['alone']['hundred_rows']['us_per_call']} us per call; beside a search: "
        f"{r['with_search_on_another_context']['one_row']['us_per_call']} / "
        f"{r['with_search_on_another_context']['hundred_rows']['us_per_call']} us, searches "
        f"{r['with_search_on_another_context']['searches_per_s']} /s (alone "
        f"{r['searches_per_s_alone']} /s)")
    return r


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--n", type=int, default=1_000_000)
    ap.add_argument("--nq", type=int, default=10_000)
    ap.add_argument("--k", type=int, default=10)
    ap.add_argument("--paths", default="flat,flat_uniform,sq8,ivfpq,filtered,hnsw_sq8,pqflat,"
                                        "append,per_query")
    ap.add_argument("--nprobe", type=int, default=64)
    ap.add_argument("--cpu-sample", type=int, default=6400,
                    help="queries in the flat CPU-baseline sample (SQ8 uses half, IVF-PQ all)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--sweeps", type=int, default=1,
                    help="also time flat batch sizes / k=100 and the IVF-PQ nprobe sweep")
    ap.add_argument("--f-rows", type=int, default=5_000_000, help="filtered: total rows")
    ap.add_argument("--f-nq", type=int, default=4096, help="filtered: queries")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run a plain device-to-device copy of MIB MiB (3 times); used "
                         "to calibrate rocprofv3 FETCH_SIZE / WRITE_SIZE")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported (one process "
              "drives one MI355X; a run over several GPUs is not part of this build)",
              file=sys.stderr)
        sys.exit(2)

    import torch

    if args.copy_probe:
        n = args.copy_probe * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_mib": args.copy_probe, "launches": 3}))
        return

    import vdbg
    from vdbg import datagen

    paths = set(args.paths.split(","))
    dim, k, nq, N = 128, args.k, args.nq, args.n
    threads, cpu_model = cpu_threads(), cpu_model_name()
    log(f"cpu baseline: {threads} threads on {cpu_model}")
    log(f"generating sift-like base {N}x{dim} and {nq} queries")
    base = datagen.sift_like(N, dim, 2002)
    queries = datagen.sift_like(nq, dim, 2003)

    ref = oracle = None
    if not args.no_cpu:
        from oracle_lib import load_oracle, load_reference
        ref = load_reference()
        oracle = load_oracle()

    ctx = vdbg.Context(0)
    ds = vdbg.Dataset(ctx, base, dim)
    dev = torch.device("cuda:0")
    q_dev = torch.from_numpy(queries).to(dev)
    ids_dev = torch.empty((nq, k), dtype=torch.int32, device=dev)
    d_dev = torch.empty((nq, k), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream().cuda_stream

    def gpu_out():
        return ids_dev.cpu().numpy().view(np.uint32).copy(), d_dev.cpu().numpy().copy()

    def parity(gi, gd, oi, od):
        s = len(oi)
        return bool(np.array_equal(gi[:s], oi) and
                    np.array_equal(gd[:s].view(np.uint32), od.view(np.uint32)))

    results = {}

    # ------------------------------------------------------------ flat
    if "flat" in paths:
        def step():
            ds.flat_search_device(q_dev.data_ptr(), nq, k, ids_dev.data_ptr(), d_dev.data_ptr(),
                                  stream=stream)

        el, prof, fb = timed(ctx, torch, step, args.steps, args.warmup,
                             ["query_prep", "sample_gemm", "kth", "flat_gemm", "select",
                              "exact_scan", "merge"])
        gi, gd = gpu_out()
        g_ms = prof["flat_gemm"][0] / max(1, prof["flat_gemm"][1])
        tflops = 2.0 * nq * N * dim / (g_ms * 1e-3) / 1e12
        # integer-valued rows and queries (SIFT-like, values 0..120) rank on the int8 GEMM
        # (rows and queries shifted into int8, exact int32 sums), priced at the int8 MFMA
        # peak; the exact fp16-input GEMM and the fp32 GEMM run the same workload below
        bits = ctx.last_gemm_bits()
        kern = {8: "k_gemm8<128,L2,2 query blocks,threshold>",
                16: "k_gemm16<128,L2,2 query blocks,threshold>"}.get(bits, "k_gemm<128,L2,rows,filter>")
        r = {"qps": nq * args.steps / el, "ms_per_step": el * 1e3 / args.steps,
             "kernel": kern, "kernel_ms": g_ms, "achieved": tflops,
             "unit": "TOP/s" if bits == 8 else "TFLOP/s",
             "peak": {8: INT8_MFMA_PEAK_TOPS, 16: FP16_MFMA_PEAK_TFLOPS}.get(bits, FP32_MFMA_PEAK_TFLOPS),
             "bound": "mfma",
             "mfma_inputs": {8: "i8 (rows and queries shifted by one constant; exact int32 sums)",
                             16: "f16 (exact: integer values, sums < 2^24)"}.get(bits, "f32"),
             "kernel_ms_per_step": {kk: v[0] / args.steps for kk, v in prof.items()},
             "exact_rescans": fb}
        log(f"flat: {r['qps']:.0f} q/s, GEMM {g_ms:.2f} ms = {tflops:.1f} T(FL)OP/s ({bits}-bit inputs)")
        if bits == 8:
            # the same workload on the exact fp16-input GEMM (identical results)
            ctx.set_int8_gemm(False)
            el16, prof16, _ = timed(ctx, torch, step, args.steps, 1, ["flat_gemm"])
            ctx.set_int8_gemm(True)
            g16 = prof16["flat_gemm"][0] / max(1, prof16["flat_gemm"][1])
            t16 = 2.0 * nq * N * dim / (g16 * 1e-3) / 1e12
            r["fp16_gemm"] = {"qps": round(nq * args.steps / el16, 1),
                              "kernel": "k_gemm16<128,L2,2 query blocks,threshold>",
                              "kernel_ms": round(g16, 4), "achieved_TFLOPs": round(t16, 2),
                              "peak_TFLOPs": FP16_MFMA_PEAK_TFLOPS,
                              "frac": round(t16 / FP16_MFMA_PEAK_TFLOPS, 4)}
            log(f"flat (fp16 GEMM): {nq * args.steps / el16:.0f} q/s, GEMM {g16:.2f} ms = "
                f"{t16:.1f} TFLOP/s")
        if bits in (8, 16):
            # the same workload ranked on the fp32 GEMM (identical results), against the fp32
            # MFMA peak
            ctx.set_fp16_gemm(False)
            el32, prof32, _ = timed(ctx, torch, step, args.steps, 1, ["flat_gemm"])
            ctx.set_fp16_gemm(True)
            g32 = prof32["flat_gemm"][0] / max(1, prof32["flat_gemm"][1])
            t32 = 2.0 * nq * N * dim / (g32 * 1e-3) / 1e12
            r["fp32_gemm"] = {"qps": round(nq * args.steps / el32, 1), "kernel": "k_gemm<128,L2,rows,filter>",
                              "kernel_ms": round(g32, 4), "achieved_TFLOPs": round(t32, 2),
                              "peak_TFLOPs": FP32_MFMA_PEAK_TFLOPS,
                              "frac": round(t32 / FP32_MFMA_PEAK_TFLOPS, 4)}
            log(f"flat (fp32 GEMM): {nq * args.steps / el32:.0f} q/s, GEMM {g32:.2f} ms = "
                f"{t32:.1f} TFLOP/s")
        if not args.no_cpu:
            s = min(args.cpu_sample, nq)
            qs = np.ascontiguousarray(queries[:s])
            od = np.empty((s, k), np.float32)
            oi = np.empty((s, k), np.uint32)
            t0 = time.perf_counter()
            if ref is not None:
                ref.lib.ref_flat_index_batch(0, base, N, dim, dim, qs, s, k, od, oi, threads)
                kind, kern = "reference", ref.lib.ref_best_kernels().decode()
            else:
                od, oi = oracle.flat_search(base, qs, k, threads=threads)
                kind, kern = "port", "avx512-order restatement"
            dt = time.perf_counter() - t0
            r["cpu_baseline"] = {
                "value": s / dt, "unit": "queries/s", "cores": threads, "kind": kind,
                "cpu_model": cpu_model,
                "sample": f"{s} of the {nq} queries, FlatIndex::search per query over all {N} "
                          f"rows ({kern} kernels), queries over {threads} threads, {dt:.1f} s"}
            r["parity_on_cpu_sample"] = parity(gi, gd, oi, od)
            log(f"flat cpu: {s / dt:.1f} q/s ({kind}), parity {r['parity_on_cpu_sample']}")
            if ref is not None:
                # one thread (the per-thread rate vdb's own figures quote) and the blocked
                # FlatSearchBatch (flat_index.cc:41-68), vdb's best CPU batch form
                s1 = min(s, 160)
                t0 = time.perf_counter()
                ref.lib.ref_flat_index_batch(0, base, N, dim, dim, qs, s1, k, od, oi, 1)
                dt1 = time.perf_counter() - t0
                r["cpu_baseline"]["one_thread"] = {
                    "value": s1 / dt1, "sample": f"{s1} queries, FlatIndex::search, 1 thread, "
                                                 f"{dt1:.1f} s"}
                t0 = time.perf_counter()
                ref.lib.ref_flat_search_blocked(b"", 0, base, N, dim, dim, qs, s, k, od, oi,
                                                threads)
                dtb = time.perf_counter() - t0
                r["cpu_baseline"]["flat_search_batch"] = {
                    "value": s / dtb, "parity": parity(gi, gd, oi, od),
                    "sample": f"{s} queries, FlatSearchBatch (64-query x 512-row blocks), "
                              f"{threads} threads, {dtb:.1f} s"}
                log(f"flat cpu: 1 thread {s1 / dt1:.1f} q/s, FlatSearchBatch {s / dtb:.1f} q/s")
        # host queries in, host results out (vdbg_flat_search_host): PCIe included
        qps_h, ms_h = host_rate(lambda: ds.flat_search(queries, k), nq)
        r["host_in_out"] = {"qps": qps_h, "ms_per_batch": ms_h,
                            "note": "vdbg_flat_search_host: query upload + search + result "
                                    "download, best of 3"}
        log(f"flat host in/out: {qps_h:.0f} q/s")
        if args.sweeps:
            sweep = {}
            for b, kb in ((1, k), (64, k), (1024, k), (nq, 100)):
                ib = torch.empty((b, kb), dtype=torch.int32, device=dev)
                db = torch.empty((b, kb), dtype=torch.float32, device=dev)

                def step_b():
                    ds.flat_search_device(q_dev.data_ptr(), b, kb, ib.data_ptr(), db.data_ptr(),
                                          stream=stream)

                reps = max(args.steps, 20) if b < 1024 else args.steps
                elb, _, fbb = timed(ctx, torch, step_b, reps, 2, [])
                sweep[f"batch{b}_k{kb}"] = {"qps": round(b * reps / elb, 1),
                                            "ms_per_batch": round(elb * 1e3 / reps, 4),
                                            "exact_rescans": fbb}
                log(f"flat batch {b} k {kb}: {b * reps / elb:.0f} q/s")
            r["sweep"] = sweep
        results["flat"] = r

    # ------------------------------------------------------------ flat, real-valued rows
    if "flat_uniform" in paths:
        # 100,000 x 128 rows uniform in [0, 1), 1,000 queries from the same distribution, k = 10:
        # float rows rank on the high fp16 halves of rows and queries (one MFMA product per
        # product, under a widened bound) and every answer is re-scored in the reference's
        # AVX-512 order
        nu, nqu = 100_000, 1000
        ubase = datagen.uniform_rows(nu, dim, 1001)
        uq = datagen.uniform_rows(nqu, dim, 1002)
        uds = vdbg.Dataset(ctx, ubase, dim)
        uq_dev = torch.from_numpy(uq).to(dev)
        ui = torch.empty((nqu, k), dtype=torch.int32, device=dev)
        ud = torch.empty((nqu, k), dtype=torch.float32, device=dev)
        torch.cuda.synchronize()

        def step_u():
            uds.flat_search_device(uq_dev.data_ptr(), nqu, k, ui.data_ptr(), ud.data_ptr(),
                                   stream=stream)

        reps = max(args.steps, 20)
        el, prof, fb = timed(ctx, torch, step_u, reps, args.warmup,
                             ["query_prep", "sample_gemm", "kth", "flat_gemm", "select",
                              "exact_scan", "merge"])
        g_ms = prof["flat_gemm"][0] / max(1, prof["flat_gemm"][1])
        bits = ctx.last_gemm_bits()
        peak = {8: INT8_MFMA_PEAK_TOPS, 16: FP16_MFMA_PEAK_TFLOPS}.get(bits, FP32_MFMA_PEAK_TFLOPS)
        ach = 2.0 * nqu * nu * dim / (g_ms * 1e-3) / 1e12
        r = {"qps": nqu * reps / el, "ms_per_step": el * 1e3 / reps, "rows": nu, "queries": nqu,
             "kernel_ms": g_ms, "achieved": ach, "peak": peak,
             "unit": "TOP/s" if bits == 8 else "TFLOP/s", "frac": ach / peak,
             "mfma_inputs": {8: "i8 two-part rows x two-part queries",
                             16: "f16 high halves of rows and queries"}.get(bits, "f32"),
             "kernel_ms_per_step": {kk: v[0] / reps for kk, v in prof.items()},
             "exact_rescans": fb}
        ugi = ui.cpu().numpy().view(np.uint32).copy()
        ugd = ud.cpu().numpy().copy()
        if ref is not None:
            s_ = nqu
            qs = np.ascontiguousarray(uq[:s_])
            od = np.empty((s_, k), np.float32)
            oi = np.empty((s_, k), np.uint32)
            t0 = time.perf_counter()
            ref.lib.ref_flat_index_batch(0, ubase, nu, dim, dim, qs, s_, k, od, oi, threads)
            dt = time.perf_counter() - t0
            r["cpu_baseline"] = {"value": s_ / dt, "unit": "queries/s", "cores": threads,
                                 "kind": "reference", "cpu_model": cpu_model,
                                 "sample": f"{s_} queries, FlatIndex::search, {threads} threads, "
                                           f"{dt:.2f} s"}
            r["parity_on_cpu_sample"] = parity(ugi, ugd, oi, od)
        log(f"flat uniform 100k: {r['qps']:.0f} q/s, GEMM {g_ms:.3f} ms ({bits}-bit), "
            f"parity {r.get('parity_on_cpu_sample')}")
        uds.close()
        results["flat_uniform"] = r

    # ------------------------------------------------------------ SQ8
    if "sq8" in paths:
        depth = 100
        sq = vdbg.Sq8Index(ds)

        def step():
            sq.search_device(q_dev.data_ptr(), nq, k, depth, ids_dev.data_ptr(),
                             d_dev.data_ptr(), stream=stream)

        el, prof, fb = timed(ctx, torch, step, args.steps, args.warmup,
                             ["query_prep", "sample_gemm", "kth", "sq8_gemm", "select",
                              "rerank", "exact_scan", "merge"])
        gi, gd = gpu_out()
        g_ms = prof["sq8_gemm"][0] / max(1, prof["sq8_gemm"][1])
        tflops = 2.0 * nq * N * dim / (g_ms * 1e-3) / 1e12
        # the codes rank on int8 MFMA against the query operand rounded to integers in two
        # int8 parts (two MFMA products per code x query product), or, with the int8 GEMM
        # switched off, on fp16 MFMA against two fp16 parts; achieved counts the algorithmic
        # work (2 N d per query), priced at the peak of the MFMA type that ran
        bits = ctx.last_gemm_bits()
        kern = {8: "k_gemm8<128,L2,SQ8 two-part operand,threshold>",
                16: "k_gemm16<128,L2,split codes>"}.get(bits, "k_gemm<128,L2,codes,filter>")
        r = {"qps": nq * args.steps / el, "ms_per_step": el * 1e3 / args.steps,
             "kernel": kern, "kernel_ms": g_ms, "achieved": tflops,
             "unit": "TOP/s" if bits == 8 else "TFLOP/s",
             "peak": {8: INT8_MFMA_PEAK_TOPS, 16: FP16_MFMA_PEAK_TFLOPS}.get(bits, FP32_MFMA_PEAK_TFLOPS),
             "bound": "mfma",
             "mfma_inputs": {8: "i8 codes - 128 x query operand as two int8 parts (exact int32 sums)",
                             16: "f16 codes x two-part f16 query operand"}.get(bits, "f32"),
             "kernel_ms_per_step": {kk: v[0] / args.steps for kk, v in prof.items()},
             "exact_rescans": fb, "depth": depth}
        if bits == 8:
            ctx.set_int8_gemm(False)
            el16, prof16, _ = timed(ctx, torch, step, args.steps, 1, ["sq8_gemm"])
            ctx.set_int8_gemm(True)
            g16 = prof16["sq8_gemm"][0] / max(1, prof16["sq8_gemm"][1])
            r["fp16_gemm"] = {"qps": round(nq * args.steps / el16, 1),
                              "kernel": "k_gemm16<128,L2,split codes>", "kernel_ms": round(g16, 4),
                              "achieved_TFLOPs": round(2.0 * nq * N * dim / (g16 * 1e-3) / 1e12, 2),
                              "peak_TFLOPs": FP16_MFMA_PEAK_TFLOPS}
            log(f"sq8 (fp16 GEMM): {nq * args.steps / el16:.0f} q/s, GEMM {g16:.2f} ms")
        log(f"sq8: {r['qps']:.0f} q/s, GEMM {g_ms:.2f} ms = {tflops:.1f} TFLOP/s")
        if not args.no_cpu:
            s = min(args.cpu_sample // 2, nq)
            qs = np.ascontiguousarray(queries[:s])
            codes = sq.codes()
            od = np.empty((s, k), np.float32)
            oi = np.empty((s, k), np.uint32)
            t0 = time.perf_counter()
            if ref is not None:
                ref.lib.ref_sq8_search_batch(b"", 0, base, codes, N, dim, dim, sq.vmin, sq.scale,
                                             qs, s, k, depth, od, oi, threads)
                kind = "reference"
            else:
                od, oi = oracle.sq8_search(base, codes, sq.vmin, sq.scale, qs, k, depth,
                                           threads=threads)
                kind = "port"
            dt = time.perf_counter() - t0
            r["cpu_baseline"] = {
                "value": s / dt, "unit": "queries/s", "cores": threads, "kind": kind,
                "cpu_model": cpu_model,
                "sample": f"{s} queries: SQ8 scan of all {N} codes into top-{depth} + fp32 "
                          f"Rerank, {threads} threads, {dt:.1f} s"}
            r["parity_on_cpu_sample"] = parity(gi, gd, oi, od)
            log(f"sq8 cpu: {s / dt:.1f} q/s ({kind}), parity {r['parity_on_cpu_sample']}")
        qps_h, ms_h = host_rate(lambda: sq.search(queries, k, depth), nq)
        r["host_in_out"] = {"qps": qps_h, "ms_per_batch": ms_h,
                            "note": "vdbg_sq8_search_host: PCIe included, best of 3"}
        log(f"sq8 host in/out: {qps_h:.0f} q/s")
        sq.close()
        results["sq8"] = r

    # ------------------------------------------------------------ IVF-PQ
    if "ivfpq" in paths:
        nlist, m, rerank, nprobe = 4096, 16, 100, args.nprobe
        t0 = time.perf_counter()
        ix = vdbg.IvfPqIndex.build(ds, nlist=nlist, m=m, seed=42, max_points=256, iters=20)
        build_s = time.perf_counter() - t0
        log(f"ivfpq: built nlist={nlist} m={m} in {build_s:.1f} s")
        dc_dev = torch.empty(nq, dtype=torch.int64, device=dev)
        # codes scanned per query (rerank 0: dist_comps = nlist + codes scanned)
        ix.search_device(q_dev.data_ptr(), nq, k, nprobe, 0, ids_dev.data_ptr(),
                         d_dev.data_ptr(), dc_ptr=dc_dev.data_ptr(), stream=stream)
        torch.cuda.synchronize()
        scanned = int(dc_dev.cpu().numpy().sum()) - nq * nlist

        def step():
            ix.search_device(q_dev.data_ptr(), nq, k, nprobe, rerank, ids_dev.data_ptr(),
                             d_dev.data_ptr(), stream=stream)

        el, prof, _ = timed(ctx, torch, step, args.steps, args.warmup,
                            ["query_prep", "sample_gemm", "kth", "flat_gemm", "select",
                             "exact_scan", "merge", "ivf_qtab", "ivf_scan", "rerank"])
        gi, gd = gpu_out()
        s_ms = prof["ivf_scan"][0] / max(1, prof["ivf_scan"][1])
        # algorithmic bytes of the list scan: the codes and ids of every scanned row (m + 4
        # bytes each).  The row-sum scan reads each row's code and its 4-byte term-2 sum (ids
        # only for the rows it scores exactly); the per-list term-2 tables the reference reads
        # (m x 256 floats per probed list, ivf_pq.cc:197-217) are not streamed.
        alg_bytes = scanned * (m + 4)
        gbs = alg_bytes / (s_ms * 1e-3) / 1e9
        r = {"qps": nq * args.steps / el, "ms_per_step": el * 1e3 / args.steps,
             "kernel": "k_ivf_scan_rs", "kernel_ms": s_ms, "achieved": gbs, "unit": "GB/s",
             "peak": HBM_PEAK_GBS, "bound": "hbm",
             "algorithmic_bytes": "codes + ids of the scanned rows",
             "algorithmic_bytes_per_launch": alg_bytes,
             "stream_bytes_per_launch": scanned * (m + 4),
             "stream_note": "codes + per-row term-2 sums (m + 4 bytes per scanned row)",
             "codes_scanned_per_query": scanned / nq,
             "kernel_ms_per_step": {kk: v[0] / args.steps for kk, v in prof.items()},
             "nlist": nlist, "m": m, "nprobe": nprobe, "rerank": rerank,
             "kmeans_iters": 20, "build_s": build_s}
        log(f"ivfpq: {r['qps']:.0f} q/s, scan {s_ms:.3f} ms = {gbs:.0f} GB/s")
        # the per-list table scan (one table fl(term2 + qtab) per probed list) beside it
        ctx.set_ivf_row_sums(False)
        try:
            el_t, prof_t, _ = timed(ctx, torch, step, args.steps, 1, ["ivf_qtab", "ivf_scan"])
            gi_t, gd_t = gpu_out()
        finally:
            ctx.set_ivf_row_sums(True)
        t_ms = prof_t["ivf_scan"][0] / max(1, prof_t["ivf_scan"][1])
        r["table_scan"] = {
            "qps": nq * args.steps / el_t, "kernel": "k_ivf_scan_fast", "kernel_ms": t_ms,
            "achieved": alg_bytes / (t_ms * 1e-3) / 1e9,
            "term2_bytes_per_launch": nq * nprobe * m * 256 * 4,
            "same_results": bool(np.array_equal(gi_t, gi) and
                                 np.array_equal(gd_t.view(np.uint32), gd.view(np.uint32)))}
        log(f"ivfpq table scan: scan {t_ms:.3f} ms, same {r['table_scan']['same_results']}")
        if not args.no_cpu and ref is not None:
            blob = ix.save()
            s = nq
            qs = np.ascontiguousarray(queries[:s])
            od = np.empty((s, k), np.float32)
            oi = np.empty((s, k), np.uint32)
            t0 = time.perf_counter()
            rc = ref.lib.ref_ivfpq_search_batch(0, blob, len(blob), base, N, dim, dim, qs, s, k,
                                                nprobe, rerank, None, od, oi, None, threads)
            dt = time.perf_counter() - t0
            if rc == 0:
                r["cpu_baseline"] = {
                    "value": s / dt, "unit": "queries/s", "cores": threads, "kind": "reference",
                    "cpu_model": cpu_model,
                    "sample": f"all {s} queries, IvfPqIndex::search (nprobe {nprobe}, rerank "
                              f"{rerank}) on the same index file, {threads} threads, {dt:.1f} s"}
                r["parity_on_cpu_sample"] = parity(gi, gd, oi, od)
                log(f"ivfpq cpu: {s / dt:.1f} q/s, parity {r['parity_on_cpu_sample']}")
        qps_h, ms_h = host_rate(lambda: ix.search(queries, k, nprobe, rerank), nq)
        r["host_in_out"] = {"qps": qps_h, "ms_per_batch": ms_h,
                            "note": "vdbg_ivfpq_search_host: PCIe included, best of 3"}
        log(f"ivfpq host in/out: {qps_h:.0f} q/s")
        if args.sweeps:
            sweep = {}
            for npb in (16, 32, 64, 128):
                ix.search_device(q_dev.data_ptr(), nq, k, npb, 0, ids_dev.data_ptr(),
                                 d_dev.data_ptr(), dc_ptr=dc_dev.data_ptr(), stream=stream)
                torch.cuda.synchronize()
                sc = int(dc_dev.cpu().numpy().sum()) - nq * nlist
                for rr in (0, 100):
                    def step_s():
                        ix.search_device(q_dev.data_ptr(), nq, k, npb, rr, ids_dev.data_ptr(),
                                         d_dev.data_ptr(), stream=stream)

                    els, prs, _ = timed(ctx, torch, step_s, args.steps, 1, ["ivf_scan"])
                    sms = prs["ivf_scan"][0] / max(1, prs["ivf_scan"][1])
                    sweep[f"nprobe{npb}_rerank{rr}"] = {
                        "qps": round(nq * args.steps / els, 1),
                        "scan_ms": round(sms, 4),
                        "scan_GBps": round(sc * (m + 4) / (sms * 1e-3) / 1e9, 1),
                        "codes_scanned_per_query": round(sc / nq, 1)}
                    log(f"ivfpq nprobe {npb} rerank {rr}: {nq * args.steps / els:.0f} q/s")
            r["sweep"] = sweep
        ix.close()
        results["ivfpq"] = r

    # ------------------------------------------------------------ filtered collection
    if "filtered" in paths:
        results["filtered"] = run_filtered(args, ctx, torch, ref, threads, cpu_model)

    # ------------------------------------------------------------ the next rows
    if "hnsw_sq8" in paths:
        results["hnsw_sq8"] = run_hnsw_sq8(args, ctx, torch, ref, base, queries, threads,
                                           cpu_model)
    if "pqflat" in paths:
        results["pqflat"] = run_pqflat(args, ctx, torch, ref, ds, base, queries, threads,
                                       cpu_model)
    if "append" in paths:
        results["append"] = run_append(args, ctx, torch, base)
    if "per_query" in paths:
        pq = run_per_query(args)
        if pq is not None:
            results["per_query"] = pq

    if N == 1_000_000 and nq == 10_000 and k == 10:
        for name in ("flat", "sq8", "ivfpq"):
            if name in results and (name != "ivfpq" or args.nprobe == 64):
                results[name]["traffic"] = profiled_traffic(name)
    paths_out = {name: {kk: (round(v, 4) if isinstance(v, float) else v)
                        for kk, v in r.items()} for name, r in results.items()}
    if "flat" not in results:  # the headline is the flat path's; report the others alone
        print(json.dumps({"metric": METRIC, "value": None, "unit": "queries/s",
                          "note": "headline needs the flat path (--paths flat,...)",
                          "paths": paths_out}), flush=True)
        return
    head = results["flat"]
    out = {
        "metric": METRIC,
        "value": round(head["qps"], 1),
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8 ranking GEMM (exact), f32 distances" if head.get("unit") == "TOP/s" else "f32",
        "data": "synthetic (seeded SIFT-like mixture, resident in HBM)",
        "config": {"workload": f"flat_l2_sift_like_{N}x{dim}_k{k}_batch{nq}", "n": N,
                   "dim": dim, "k": k, "batch": nq, "metric": "l2"},
        "roofline": {"bound": head["bound"], "achieved": round(head["achieved"], 2),
                     "peak": head["peak"], "unit": head["unit"],
                     "frac": round(head["achieved"] / head["peak"], 4),
                     "traffic": head.get("traffic"), "traffic_unit": "bytes per launch",
                     "kernel": head["kernel"], "kernel_ms": round(head["kernel_ms"], 3),
                     "mfma_inputs": head.get("mfma_inputs")},
        "cpu_baseline": head.get("cpu_baseline"),
        "parity_on_cpu_sample": head.get("parity_on_cpu_sample"),
        "paths": paths_out,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
