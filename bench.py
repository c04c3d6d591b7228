"""Benchmark: batch QPS of vdb's flat exact search on one MI355X.

Workload (one "step" = one batch search over resident data): flat exact L2 over 1M x 128
fp32 SIFT-like rows (integer values in [0, 255] from a 1,000-centre mixture), a batch of
10,000 queries from the same mixture, k = 10.  Rows, norms and queries are resident in HBM
before the timed region; the step is the full search (sample pre-pass, MFMA GEMM + filter,
selection, exact re-scoring and any exact re-scan).

Printed: one JSON line with the metric, the MFMA roofline of the dominant kernel (GEMM time
from HIP events on the stream it runs on) and the reference's CPU FlatIndex timed on a
bounded query sample on this host's cores.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "hnsw-vector-db_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))

METRIC = "batch QPS at k=10 (flat/SQ8/IVF-PQ, 1M×128); achieved HBM TB/s / MFMA %"
FP32_MFMA_PEAK_TFLOPS = 157.3


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_baseline(base, queries, k, sample_q, threads):
    """The reference's FlatIndex (oracle/_ref) or, where it is not built, the oracle's
    restatement, over `sample_q` queries fanned over `threads` host threads."""
    from oracle_lib import load_oracle, load_reference

    qs = np.ascontiguousarray(queries[:sample_q])
    ref = load_reference()
    od = np.empty((sample_q, k), np.float32)
    oi = np.empty((sample_q, k), np.uint32)
    if ref is not None:
        kind = "reference"
        t0 = time.perf_counter()
        ref.lib.ref_flat_index_batch(0, base, base.shape[0], base.shape[1], base.shape[1], qs,
                                     sample_q, k, od, oi, threads)
        dt = time.perf_counter() - t0
        kernels = ref.lib.ref_best_kernels().decode()
    else:
        kind = "port"
        o = load_oracle()
        t0 = time.perf_counter()
        od, oi = o.flat_search(base, qs, k, threads=threads)
        dt = time.perf_counter() - t0
        kernels = "avx512-order emulation"
    return {"value": sample_q / dt, "unit": "queries/s", "cores": threads, "kind": kind,
            "sample": f"{sample_q} of the batch's queries, FlatIndex::search per query over "
                      f"all {base.shape[0]} rows, {kernels} kernels, {dt:.1f} s"}, oi, od


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--n", type=int, default=1_000_000)
    ap.add_argument("--nq", type=int, default=10_000)
    ap.add_argument("--k", type=int, default=10)
    ap.add_argument("--cpu-sample", type=int, default=6400)
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run a plain device-to-device copy of MIB MiB (3 times); used "
                         "to calibrate rocprofv3 FETCH_SIZE / WRITE_SIZE")
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported (every box "
              "in this setup has one MI355X; the sharded design is described in DESIGN.md)",
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

    dim = 128
    k = args.k
    log(f"generating sift-like base {args.n}x{dim} and {args.nq} queries")
    base = datagen.sift_like(args.n, dim, 2002)
    queries = datagen.sift_like(args.nq, dim, 2003)

    ctx = vdbg.Context(0)
    ds = vdbg.Dataset(ctx, base, dim)
    dev = torch.device("cuda:0")
    q_dev = torch.from_numpy(queries).to(dev)
    ids_dev = torch.empty((args.nq, k), dtype=torch.int32, device=dev)
    d_dev = torch.empty((args.nq, k), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream().cuda_stream

    def step():
        ds.flat_search_device(q_dev.data_ptr(), args.nq, k, ids_dev.data_ptr(),
                              d_dev.data_ptr(), stream=stream)

    for i in range(args.warmup):
        step()
        log(f"warmup step {i + 1}/{args.warmup} done")
    torch.cuda.synchronize()
    ctx.profile(True)
    ctx.profile_reset()
    fallbacks = 0
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step()
        fallbacks += ctx.last_fallbacks()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    log(f"timed {args.steps} steps in {elapsed:.3f} s")
    gemm_ms, gemm_n = ctx.profile_get("flat_gemm")
    kernel_ms = {name: ctx.profile_get(name)[0] / max(1, args.steps)
                 for name in ("query_prep", "sample_gemm", "kth", "flat_gemm", "select", "exact_scan",
                              "merge")}
    ctx.profile(False)

    ms_per_step = elapsed * 1000.0 / args.steps
    qps = args.nq * args.steps / elapsed
    flops = 2.0 * args.nq * args.n * dim
    gemm_avg_ms = gemm_ms / max(1, gemm_n)
    achieved = flops / (gemm_avg_ms * 1e-3) / 1e12

    ids = ids_dev.cpu().numpy().view(np.uint32)
    dists = d_dev.cpu().numpy()

    cpu = None
    parity = None
    if not args.no_cpu:
        threads = min(16, os.cpu_count() or 1)
        cpu, oi, od = cpu_baseline(base, queries, k, args.cpu_sample, threads)
        parity = bool(np.array_equal(ids[:args.cpu_sample], oi) and
                      np.array_equal(dists[:args.cpu_sample].view(np.uint32), od.view(np.uint32)))
        log(f"cpu baseline: {cpu['value']:.1f} q/s ({cpu['kind']}), parity on sample: {parity}")

    out = {
        "metric": METRIC,
        "value": round(qps, 1),
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded SIFT-like mixture, resident in HBM)",
        "config": {"workload": f"flat_l2_sift_like_{args.n}x{dim}_k{k}_batch{args.nq}",
                   "n": args.n, "dim": dim, "k": k, "batch": args.nq, "metric": "l2"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2),
                     "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / FP32_MFMA_PEAK_TFLOPS, 4), "traffic": None,
                     "kernel": "k_flat_gemm<128,L2>", "kernel_ms": round(gemm_avg_ms, 3)},
        "cpu_baseline": cpu,
        "kernel_ms_per_step": {k_: round(v, 3) for k_, v in kernel_ms.items()},
        "exact_rescans": fallbacks,
        "parity_on_cpu_sample": parity,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
