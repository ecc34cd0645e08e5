"""Batch search throughput on one MI355X.

Default workload (the configuration the headline metric is quoted on):
IVF-PQ over 1,000,000 x 128 f32 vectors with non-negative integer components
drawn from a 1024-component Gaussian mixture (per-dim std 20, clipped to
[0, 255]); nlist = 1024 k-means lists, M = 16 subvectors x 8 dims, 256
codewords each; nprobe = 16; 10,000 queries from the same mixture; k = 10;
Euclidean.

A step is one batch_search of all queries with the queries, the index and the
outputs resident in HBM.  For IVF-PQ that is coarse selection + the fused
LUT/ADC/top-k scan; the index is built on the GPU first (seeded).

The roofline object covers the dominant kernel.  IVF-PQ: the algorithmic code
bytes (sum over queries of the sizes of its probed lists, times M bytes)
divided by the scan kernel's mean duration, measured with HIP events on the
stream it runs on.

Other workloads (--workload), each measured the same way with its own
roofline:
  bf_10k        brute force 10,000 x 128 U[0,1), 100 queries, k 10, L2^2
  bf_1m_cosine  brute force 1,000,000 x 128 normalised Gaussian, 10,000
  bf_1m_dot     queries, k 100 (cosine / dot product); flops 2*Q*N*D
  ivf_1m_l2     IVF (full vectors) 1,000,000 x 96 Gaussian mixture, nlist
  ivf_1m_l1     4096, nprobe 32, 10,000 queries, k 100 (Euclidean /
                Manhattan); bytes: the probed lists' rows as the scan reads
                them (half precision when screening, plus the K'
                candidates' f32 rows; else f32)
  ivfpq_10m     IVF-PQ 10,000,000 x 96 Gaussian mixture, nlist 4096,
                M 32 x 3, nprobe 64, 10,000 queries, k 100

cpu_baseline: the oracle (a C++ restatement of the reference's CPU path with
its AVX2 kernels) on a bounded query sample, on the host cores of the same
machine.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "forge-db_amd"))

HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3  # MI355X dense fp32 matrix peak
FP16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 matrix peak

WORKLOADS = {
    "ivfpq_1m": dict(kind="ivfpq", data="ivfpq_int", n=1_000_000, nq=10_000, nlist=1024, M=16,
                     nprobe=16, k=10, metric=0, tag="1Mx128",
                     metric_name="batch QPS at k=10, IVF-PQ 1M×128 nprobe=16; ADC-scan HBM GB/s",
                     desc="IVF-PQ 1Mx128 integer Gaussian mixture (1024 comps, std 20), nlist 1024, "
                          "M 16x8, nprobe 16, Q 10000, k 10, Euclidean"),
    "ivfpq_10m": dict(kind="ivfpq", data="ivfpq_large", n=10_000_000, nq=10_000, nlist=4096, M=32,
                      nprobe=64, k=100, metric=0, tag="10Mx96",
                      metric_name="batch QPS at k=100, IVF-PQ 10M×96 M=32x3 nprobe=64",
                      desc="IVF-PQ 10Mx96 Gaussian mixture (4096 comps), nlist 4096, M 32x3, "
                           "nprobe 64, Q 10000, k 100, Euclidean"),
    "bf_10k": dict(kind="bf", data="bf_small", n=10_000, nq=100, k=10, metric=1,
                   metric_name="batch QPS at k=10, brute force 10k×128 L2²",
                   desc="BruteForce 10kx128 U[0,1), Q 100, k 10, EuclideanSquared"),
    "bf_1m_cosine": dict(kind="bf", data="bf_norm", n=1_000_000, nq=10_000, k=100, metric=2,
                         metric_name="batch QPS at k=100, brute force 1M×128 cosine",
                         desc="BruteForce 1Mx128 normalised Gaussian, Q 10000, k 100, Cosine"),
    "bf_1m_dot": dict(kind="bf", data="bf_norm", n=1_000_000, nq=10_000, k=100, metric=3,
                      metric_name="batch QPS at k=100, brute force 1M×128 dot product",
                      desc="BruteForce 1Mx128 normalised Gaussian, Q 10000, k 100, DotProduct"),
    "ivf_1m_l2": dict(kind="ivf", data="ivf_flat", n=1_000_000, nq=10_000, nlist=4096, nprobe=32,
                      k=100, metric=0,
                      metric_name="batch QPS at k=100, IVF-flat 1M×96 nprobe=32 Euclidean",
                      desc="IVF 1Mx96 Gaussian mixture (4096 comps), nlist 4096, nprobe 32, "
                           "Q 10000, k 100, Euclidean"),
    "ivf_1m_l1": dict(kind="ivf", data="ivf_flat", n=1_000_000, nq=10_000, nlist=4096, nprobe=32,
                      k=100, metric=4,
                      metric_name="batch QPS at k=100, IVF-flat 1M×96 nprobe=32 Manhattan",
                      desc="IVF 1Mx96 Gaussian mixture (4096 comps), nlist 4096, nprobe 32, "
                           "Q 10000, k 100, Manhattan"),
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def read_traffic(name):
    """HBM bytes per launch of the dominant kernel from a committed
    rocprofv3 --pmc summary (profiles/<name>), if present."""
    p = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(p):
        return None
    for line in open(p):
        if line.startswith("hbm_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


class Runner:
    """Device buffers, the timed loop and kernel timing shared by workloads."""

    def __init__(self, args, queries, k):
        import torch
        self.torch = torch
        self.args = args
        self.dev = torch.device("cuda:0")
        self.stream = torch.cuda.Stream(device=self.dev)
        self.sptr = self.stream.cuda_stream
        self.nq = queries.shape[0]
        self.k = k
        self.q_d = torch.from_numpy(queries).to(self.dev)
        self.ids_d = torch.empty((self.nq, k), dtype=torch.int64, device=self.dev)
        self.dist_d = torch.empty((self.nq, k), dtype=torch.float32, device=self.dev)
        self.cnt_d = torch.empty(self.nq, dtype=torch.int32, device=self.dev)
        torch.cuda.synchronize()

    def ptrs(self):
        return (self.q_d.data_ptr(), self.nq, self.k, self.ids_d.data_ptr(),
                self.dist_d.data_ptr(), self.cnt_d.data_ptr(), self.sptr)

    def timed_loop(self, step, sync):
        torch = self.torch
        for _ in range(self.args.warmup):
            step()
        sync()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(self.args.steps):
            step()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        sync()
        return (t1 - t0) * 1e3 / self.args.steps

    def ids(self):
        import numpy as np
        return self.ids_d.cpu().numpy().view(np.uint64)


def agreement(a, b, k):
    import numpy as np
    return float(np.mean([len(set(a[q].tolist()) & set(b[q].tolist())) / k for q in range(len(a))]))


def host_threads():
    """The threads the CPU baseline uses: every core this process may run on
    (Rayon's default pool is one thread per available core)."""
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return os.cpu_count() or 1


def cpu_leg(run, nq, args, gpu_ids, k, threads, how):
    """The cpu_baseline object.  run(m) searches the first m queries on the
    host and returns (ids, dists, counts).  After a warm-up on a few queries,
    the per-query time picks a sample size (all queries when three runs fit
    in --cpu-seconds, else a prefix); the figure is the median of three runs
    over that sample.  The sample's ids are compared with the GPU's."""
    warm = min(nq, 64)
    t = time.perf_counter()
    run(warm)
    per_q = (time.perf_counter() - t) / warm
    sample = int(min(nq, max(warm, args.cpu_seconds / 3 / max(per_q, 1e-9))))
    secs, first = [], None
    for _ in range(3):
        t = time.perf_counter()
        out = run(sample)
        secs.append(time.perf_counter() - t)
        first = first if first is not None else out
    med = float(np.median(secs))
    agree = agreement(gpu_ids[:sample], first[0], k)
    what = f"all {nq} queries" if sample == nq else f"first {sample} of the {nq} queries"
    log(f"[bench] CPU baseline {sample / med:,.1f} QPS on {threads} threads (median of 3 runs over {what}: "
        f"{', '.join(f'{x:.2f}' for x in secs)} s); id agreement {agree:.6f}")
    return {"value": round(sample / med, 1), "unit": "queries/s", "cores": threads, "kind": "port",
            "sample": f"{what}, {how}; median of 3 runs after a warm-up",
            "run_seconds": [round(x, 4) for x in secs], "nproc": os.cpu_count(),
            "cpu_model": cpu_model(), "gpu_id_agreement": round(agree, 6)}


def w_name(w):
    """The WORKLOADS key of a workload."""
    return next(name for name, v in WORKLOADS.items() if v is w)


def thresh_kernel_name(dim):
    """The threshold screening kernel (stage B) an IVF-PQ shape runs:
    <k-chunks, ring stages, waves per SIMD, groups of 32 pairs per wave,
    waves per workgroup>."""
    kc = (dim + 15) // 16
    waves = 3 if kc <= 6 else (4 if kc <= 8 else (3 if kc <= 12 else 2))
    return f"pq16_thresh_kernel<{kc}, 3, {waves}, {2 if kc <= 6 else 1}, 4>"


def latency_leg(index, oracle, queries, k, reps):
    """Single-query search latency (the call the server makes per query,
    grpc.rs:294-310 -> ivf_pq.rs:590-677): the GPU's fdb_ivfpq_search with the
    query and results in host memory (upload, kernels, download), and the
    oracle's search on one thread; medians over `reps` queries after a
    warm-up."""
    n = min(reps, len(queries))
    for q in queries[:20]:
        index.search(q, k)
    g = []
    for q in queries[:n]:
        t = time.perf_counter()
        index.search(q, k)
        g.append(time.perf_counter() - t)
    out = {"queries": n, "k": k, "gpu_search_us_median": round(float(np.median(g)) * 1e6, 1),
           "gpu_search_us_p99": round(float(np.percentile(g, 99)) * 1e6, 1),
           "gpu_includes": "host-to-device query copy, coarse + scan kernels, device-to-host results"}
    if oracle is not None:
        for q in queries[:5]:
            oracle.search(q, k)
        c = []
        for q in queries[:n]:
            t = time.perf_counter()
            oracle.search(q, k)
            c.append(time.perf_counter() - t)
        out["cpu_search_us_median_1thread"] = round(float(np.median(c)) * 1e6, 1)
        out["cpu_kind"] = "port (the oracle's search: groups-of-4 ADC, one thread)"
    log(f"[bench] single-query search: GPU {out['gpu_search_us_median']:.1f} us median "
        f"(p99 {out['gpu_search_us_p99']:.1f})" +
        (f", CPU one thread {out['cpu_search_us_median_1thread']:.1f} us" if oracle is not None else ""))
    return out


def bench_ivfpq(args, w, base, queries, compare=True):
    """compare: also time the table scan and the fast LUT mode on the same
    batch, and the single-query latency."""
    from forgedb import LUT_EXACT, LUT_FAST, IVFPQIndex

    nlist, M, nprobe, k = w["nlist"], w["M"], w["nprobe"], w["k"]
    tag = w["tag"]
    t = time.time()
    index = IVFPQIndex.build(base, nlist, M, seed=args.seed)
    log(f"[bench] GPU build (k-means {nlist}, PQ {M}x256, encode) in {time.time() - t:.1f}s")
    index.set_nprobe(nprobe)
    index.set_coarse_mode({"auto": 0, "exact": 1, "screen": 2}[args.coarse])
    mode = {"auto": 0, "exact": 1, "screen": 2}[args.ivfpq_mode]
    index.set_search_mode(mode)
    r = Runner(args, queries, k)
    nq = r.nq

    def step():
        index.batch_search_device(*r.ptrs())

    def sync():
        index.sync(r.sptr)

    # the first batch after the build also builds the screening's decoded
    # half-precision copy of the lists (timed once, outside the steps)
    r.torch.cuda.synchronize()
    t0 = time.perf_counter()
    step()
    sync()
    first_ms = (time.perf_counter() - t0) * 1e3
    ms_per_step = r.timed_loop(step, sync)
    log(f"[bench] {args.steps} steps: {ms_per_step:.3f} ms/step, {nq / ms_per_step * 1e3:,.0f} QPS")

    screen_ms = []  # the threshold screening kernel, per timed batch

    def kernel_times():
        coarse, scan = [], []
        for _ in range(args.timing_reps):
            c, s = index.batch_search_device(*r.ptrs(), timed=True)
            coarse.append(c)
            scan.append(s)
            screen_ms.append(index.last_screen_kernel_ms())
        return float(np.mean(coarse)), float(np.mean(scan))

    coarse_ms, scan_ms = kernel_times()
    screen_kernel_ms = float(np.mean(screen_ms))
    exact_ids = r.ids().copy()
    path = index.last_search_path()
    fallbacks, cands = index.last_screen_stats(r.sptr)
    extra = {}
    if path == 2:
        log(f"[bench] path 2 (fp16 screening): {fallbacks} of {nq} queries rescanned exactly, "
            f"{cands / nq:,.0f} candidates rescored per query")
        # decoded codes (2 bytes per dimension, rounded up to 16 dimensions)
        # and their fp32 norms, beside the index's own codes (M bytes a code)
        d16 = (base.shape[1] + 15) // 16 * 16
        copy_bytes = (2 * d16 + 4) * base.shape[0]
        extra["screen_copy"] = {"bytes": copy_bytes, "index_code_bytes": M * base.shape[0],
                                "first_batch_ms": round(first_ms, 3),
                                "note": "built by the first screened batch after the lists change"}
        log(f"[bench] screening copy: {copy_bytes / 1e6:,.0f} MB of decoded codes and norms "
            f"({M * base.shape[0] / 1e6:,.0f} MB of codes in the index); first batch {first_ms:.2f} ms")
    if path == 2 and compare:
        # the table scan on the same batch, for comparison
        index.set_search_mode(1)
        table_ms = r.timed_loop(step, sync)
        _, table_scan_ms = kernel_times()
        table_same = agreement(r.ids(), exact_ids, k)
        index.set_search_mode(mode)
        step()
        sync()
        log(f"[bench] table scan: {table_ms:.3f} ms/step, {nq / table_ms * 1e3:,.0f} QPS, scan "
            f"{table_scan_ms:.3f} ms; id agreement with the screened path {table_same:.6f}")
        traffic = read_traffic(f"ivfpq_scan_{tag}_traffic.txt")
        extra["table_scan"] = {"value": round(nq / table_ms * 1e3, 1), "ms_per_step": round(table_ms, 4),
                               "scan_ms": round(table_scan_ms, 4), "id_agreement": round(table_same, 6),
                               "hbm_bytes_per_launch": traffic,
                               "hbm_gbs": round(traffic / (table_scan_ms / 1e3) / 1e9, 1) if traffic else None}

    lists, _ = index.probe(queries, nprobe)
    sizes = np.diff(index.list_offsets().astype(np.int64))
    scanned = int(sizes[lists].sum())
    code_bytes = scanned * M
    logical = code_bytes / (scan_ms / 1e3) / 1e9
    log(f"[bench] coarse {coarse_ms:.3f} ms, scan {scan_ms:.3f} ms; {scanned / nq:,.0f} codes per query; "
        f"{code_bytes / 1e9:.3f} GB of codes counted once per probing query -> {logical:,.0f} GB/s (logical, "
        f"not HBM traffic)")
    dim = base.shape[1]
    dsub = dim // M
    if path == 2:
        # the threshold screening kernel: 2 * D16 flops per (query, probed code)
        d16 = (dim + 15) // 16 * 16
        flops = 2 * d16 * scanned
        tflops = flops / (screen_kernel_ms / 1e3) / 1e12
        stage = flops / (scan_ms / 1e3) / 1e12
        traffic = read_traffic(f"ivfpq_screen_{tag}_traffic.txt")
        hbm = traffic / (screen_kernel_ms / 1e3) / 1e9 if traffic else None
        log(f"[bench] threshold screen {screen_kernel_ms:.3f} ms for {scanned / nq:,.0f} codes per query x "
            f"{d16} dims: {flops / 1e12:.3f} TFLOP -> {tflops:,.1f} TFLOP/s ({stage:,.1f} over the whole "
            f"scan stage)" + (f"; HBM {hbm:,.0f} GB/s from the committed counters" if hbm else ""))
        roof = {"bound": "mfma", "achieved": round(tflops, 1), "peak": FP16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(tflops / FP16_PEAK_TFLOPS, 4), "traffic": traffic,
                "kernel": thresh_kernel_name(dim), "kernel_ms": round(screen_kernel_ms, 4),
                "algorithmic_flops": flops, "hbm_gbs": round(hbm, 1) if hbm else None,
                "hbm_frac": round(hbm / HBM_PEAK_GBS, 4) if hbm else None,
                "scan_stage_ms": round(scan_ms, 4), "scan_stage_tflops": round(stage, 1),
                "adc_logical_code_bytes_per_s": round(logical * 1e9, 1),
                "coarse_ms": round(coarse_ms, 4), "fallbacks": fallbacks,
                "candidates_per_query": round(cands / nq, 1)}
    else:
        traffic = read_traffic(f"ivfpq_scan_{tag}_traffic.txt")
        roof = {"bound": "hbm", "achieved": round(logical, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(logical / HBM_PEAK_GBS, 4), "traffic": traffic,
                "kernel": f"ivfpq_scan_kernel<{M},{dsub},...>", "kernel_ms": round(scan_ms, 4),
                "algorithmic_bytes": code_bytes,
                "hbm_gbs": round(traffic / (scan_ms / 1e3) / 1e9, 1) if traffic else None,
                "coarse_ms": round(coarse_ms, 4)}

    if compare:
        # the opt-in fast LUT mode, timed the same way (distances within ~1e-6)
        index.set_lut_mode(LUT_FAST)
        fast_ms = r.timed_loop(step, sync)
        _, fast_scan_ms = kernel_times()
        fast_agree = agreement(r.ids(), exact_ids, k)
        index.set_lut_mode(LUT_EXACT)
        step()
        sync()
        log(f"[bench] fast LUT mode: {fast_ms:.3f} ms/step, {nq / fast_ms * 1e3:,.0f} QPS, scan "
            f"{fast_scan_ms:.3f} ms; id agreement with exact mode {fast_agree:.6f}")
        extra["fast_lut"] = {"value": round(nq / fast_ms * 1e3, 1), "ms_per_step": round(fast_ms, 4),
                             "scan_ms": round(fast_scan_ms, 4), "id_agreement_with_exact": round(fast_agree, 6)}

    cpu, oracle = None, None
    if not args.no_cpu:
        import refcpu  # CPU baseline leg only
        art = index.export()
        oracle = refcpu.IvfPq.create(art["centroids"], art["codebooks"], art["list_offsets"],
                                     art["ids"], art["codes"])
        oracle.set_nprobe(nprobe)
        threads = host_threads()
        cpu = cpu_leg(
            lambda m: oracle.batch_search(queries[:m], k, parallel=True, nthreads=threads),
            nq, args, exact_ids, k, threads, "batch_search_parallel (chunks of 4)")
    if compare:
        extra["latency"] = latency_leg(index, oracle, queries, k, args.latency_queries)
    cfg = {"n": base.shape[0], "nq": nq, "nlist": nlist, "M": M, "nprobe": nprobe, "k": k}
    return ms_per_step, roof, cpu, cfg, extra


def bench_bf(args, w, base, queries):
    import numpy as np
    from forgedb import BruteForceIndex, DistanceMetric

    k, metric = w["k"], DistanceMetric(w["metric"])
    t = time.time()
    index = BruteForceIndex.from_arrays(base, None, metric)
    index.set_search_mode({"auto": 0, "exact": 1, "screen": 2, "screen_f32": 3}[args.bf_mode])
    r = Runner(args, queries, k)
    nq = r.nq

    def step():
        index.batch_search_device(*r.ptrs())

    step()  # uploads the rows
    r.torch.cuda.synchronize()
    log(f"[bench] brute-force index resident in {time.time() - t:.1f}s")
    ms_per_step = r.timed_loop(step, lambda: None)
    log(f"[bench] {args.steps} steps: {ms_per_step:.3f} ms/step, {nq / ms_per_step * 1e3:,.0f} QPS")
    kms = float(np.mean([index.batch_search_device(*r.ptrs(), timed=True)
                         for _ in range(args.timing_reps)]))
    path = index.last_search_path()
    fallbacks = index.last_fallbacks()
    flops = 2.0 * nq * base.shape[0] * base.shape[1]
    achieved = flops / (kms / 1e3) / 1e12
    # the product each path runs on: exact-order fp32 VALU, fp32 or fp16 matrix cores
    peak, kernel = {0: (FP32_PEAK_TFLOPS, "flat_topk_kernel + merge_parts_kernel"),
                    1: (FP32_PEAK_TFLOPS, "mfma_screen_kernel (fp32) + rescore_kernel"),
                    2: (FP16_PEAK_TFLOPS, "screen16_kernel (fp16) + select16_kernel + rescore_kernel")}[path]
    log(f"[bench] search kernels {kms:.3f} ms -> {achieved:.1f} TFLOP/s (2*Q*N*D); path {path}, "
        f"{fallbacks} of {nq} queries rescanned exactly")
    traffic = read_traffic("bf_screen16_1Mx128_dot_traffic.txt") if (path == 2 and w is WORKLOADS["bf_1m_dot"]) \
        else None
    roof = {"bound": "mfma", "achieved": round(achieved, 2), "peak": peak,
            "unit": "TFLOP/s", "frac": round(achieved / peak, 4), "traffic": traffic,
            "kernel": kernel, "kernel_ms": round(kms, 4), "algorithmic_flops": flops,
            "fallbacks": fallbacks}
    gpu_ids = r.ids().copy()
    cpu = None
    if not args.no_cpu:
        import refcpu  # CPU baseline leg only
        threads = host_threads()
        ids = np.arange(base.shape[0], dtype=np.uint64)
        cpu = cpu_leg(
            lambda m: refcpu.bf_batch_search(base, ids, int(metric), queries[:m], k, threads),
            nq, args, gpu_ids, k, threads, "batch_search (queries in parallel)")
    cfg = {"n": base.shape[0], "nq": nq, "k": k, "metric": metric.name}
    return ms_per_step, roof, cpu, cfg, {}


def bench_ivf(args, w, base, queries):
    import numpy as np
    from forgedb import DistanceMetric, IVFIndex

    nlist, nprobe, k, metric = w["nlist"], w["nprobe"], w["k"], DistanceMetric(w["metric"])
    t = time.time()
    index = IVFIndex.build(base, nlist, metric, seed=args.seed)
    log(f"[bench] GPU build (k-means {nlist}, 100 iterations max) in {time.time() - t:.1f}s")
    index.set_nprobe(nprobe)
    index.set_coarse_mode({"auto": 0, "exact": 1, "screen": 2}[args.coarse])
    index.set_search_mode({"auto": 0, "exact": 1}[args.ivf_mode])
    r = Runner(args, queries, k)
    nq = r.nq

    def step():
        index.batch_search_device(*r.ptrs())

    ms_per_step = r.timed_loop(step, lambda: index.sync(r.sptr))
    log(f"[bench] {args.steps} steps: {ms_per_step:.3f} ms/step, {nq / ms_per_step * 1e3:,.0f} QPS")
    times, screen_ms = [], []
    for _ in range(args.timing_reps):
        times.append(index.batch_search_device(*r.ptrs(), timed=True))
        screen_ms.append(index.last_screen_kernel_ms())
    coarse_ms = float(np.mean([c for c, _ in times]))
    scan_ms = float(np.mean([s for _, s in times]))
    path = index.last_search_path()
    fallbacks = index.last_fallbacks()
    lists = index.probe(queries, nprobe)
    sizes = np.diff(index.export()["list_offsets"].astype(np.int64))
    scanned = int(sizes[lists].sum())
    dim = base.shape[1]
    fp32_bytes = scanned * dim * 4
    if path == 3:
        # list screening on the matrix cores: stage B's products, 2 x D16
        # flops per (query, probed row), against the fp16 matrix peak
        kernel_ms = float(np.mean(screen_ms))
        kc = (dim + 15) // 16
        flops = 2 * 16 * kc * scanned
        tflops = flops / (kernel_ms / 1e3) / 1e12
        tag = {"ivf_1m_l2": "1Mx96_l2"}.get(w_name(w))
        traffic = read_traffic(f"ivf_lists_{tag}_traffic.txt") if tag else None
        log(f"[bench] coarse {coarse_ms:.3f} ms, scan {scan_ms:.3f} ms; {scanned / nq:,.0f} rows per query; "
            f"path 3 (list screening; {fallbacks} of {nq} queries rescanned exactly); threshold kernel "
            f"{kernel_ms:.3f} ms: {flops / 1e9:.1f} GFLOP -> {tflops:,.1f} TFLOP/s"
            + (f"; {traffic / 1e9:.2f} GB past L2 from the committed counters" if traffic else ""))
        roof = {"bound": "mfma", "achieved": round(tflops, 1), "peak": FP16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(tflops / FP16_PEAK_TFLOPS, 4), "traffic": traffic,
                "kernel": thresh_kernel_name(dim), "kernel_ms": round(kernel_ms, 4), "algorithmic_flops": flops,
                "hbm_gbs": round(traffic / (kernel_ms / 1e3) / 1e9, 1) if traffic else None,
                "scan_stage_ms": round(scan_ms, 4), "f32_row_bytes": fp32_bytes, "coarse_ms": round(coarse_ms, 4),
                "fallbacks": fallbacks}
    elif path == 2:
        # half-precision rows of the probed lists + the K' candidates' rows
        kp = 64 if k + 16 <= 64 else 128
        row_bytes = scanned * ((dim + 1) // 2) * 4 + nq * kp * dim * 4
        kernel = "ivf16_screen_kernel + rescore_kernel"
    else:
        row_bytes = fp32_bytes
        kernel = "ivf_flat_scan_kernel"
    if path != 3:
        achieved = row_bytes / (scan_ms / 1e3) / 1e9
        log(f"[bench] coarse {coarse_ms:.3f} ms, scan {scan_ms:.3f} ms; {scanned / nq:,.0f} rows per "
            f"query; path {path} ({fallbacks} of {nq} queries rescanned exactly); {row_bytes / 1e9:.2f} GB "
            f"read -> {achieved:,.0f} GB/s ({fp32_bytes / 1e9:.2f} GB of f32 rows in the probed lists)")
        traffic = read_traffic("ivf16_screen_1Mx96_l2_traffic.txt") \
            if (path == 2 and w is WORKLOADS["ivf_1m_l2"]) else None
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                "kernel": kernel, "kernel_ms": round(scan_ms, 4),
                "algorithmic_bytes": row_bytes, "f32_row_bytes": fp32_bytes, "coarse_ms": round(coarse_ms, 4),
                "fallbacks": fallbacks}
    gpu_ids = r.ids().copy()
    cpu = None
    if not args.no_cpu:
        import refcpu  # CPU baseline leg only
        art = index.export()
        threads = host_threads()
        cpu = cpu_leg(
            lambda m: refcpu.ivf_batch_search(art["centroids"], art["list_offsets"], art["ids"],
                                              art["rows"], int(metric), nprobe, queries[:m], k,
                                              threads),
            nq, args, gpu_ids, k, threads, "batch_search (queries in parallel)")
    cfg = {"n": base.shape[0], "nq": nq, "nlist": nlist, "nprobe": nprobe, "k": k,
           "metric": metric.name}
    return ms_per_step, roof, cpu, cfg, {}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=10,
                    help="untimed steps first (the GPU clock settles over the first ~10)")
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--workload", default="ivfpq_1m", choices=sorted(WORKLOADS))
    ap.add_argument("--n", type=int, default=None, help="override the base size")
    ap.add_argument("--nq", type=int, default=None, help="override the query count")
    ap.add_argument("--timing-reps", type=int, default=10)
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="target wall time of the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--ivf-mode", default="auto", choices=["auto", "exact"],
                    help="IVF scan strategy (IVFIndex.set_search_mode)")
    ap.add_argument("--bf-mode", default="auto", choices=["auto", "exact", "screen", "screen_f32"],
                    help="brute-force search strategy (BruteForceIndex.set_search_mode)")
    ap.add_argument("--ivfpq-mode", default="auto", choices=["auto", "exact", "screen"],
                    help="IVF-PQ scan: auto (fp16 screening for large batches), table scan, or screening")
    ap.add_argument("--coarse", default="auto", choices=["auto", "exact", "screen"],
                    help="coarse selection strategy of the IVF indexes (same probes)")
    ap.add_argument("--latency-queries", type=int, default=200,
                    help="queries timed one at a time for the single-query search latency")
    ap.add_argument("--no-c5", action="store_true",
                    help="skip the 10M x 96 IVF-PQ object of the default run")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run one plain 1 GiB device-to-device copy (a known-size "
                         "reference for the FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              f"(asked for --gpus {args.gpus}).", file=sys.stderr)
        sys.exit(2)
    sys.path.insert(0, os.path.join(ROOT, "oracle"))

    import torch

    from forgedb import datagen

    w = WORKLOADS[args.workload]
    t = time.time()
    base, queries = datagen.workload(w["data"], n=args.n or w["n"], nq=args.nq or w["nq"])
    log(f"[bench] {args.workload}: generated {base.shape} base, {queries.shape} queries in "
        f"{time.time() - t:.1f}s")
    if args.calibrate_copy:
        src = torch.empty(1 << 28, dtype=torch.float32, device="cuda:0")  # 1 GiB
        dst = torch.empty_like(src)
        src.fill_(1.0)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        log("[bench] calibration copy: 1 GiB device to device")

    fn = {"ivfpq": bench_ivfpq, "bf": bench_bf, "ivf": bench_ivf}[w["kind"]]
    ms_per_step, roof, cpu, cfg, extra = fn(args, w, base, queries)
    nq = queries.shape[0]
    if args.workload == "ivfpq_1m" and not args.no_c5 and args.n is None and args.nq is None:
        # the 10M x 96 configuration, whose codes exceed the 256 MB MALL,
        # timed the same way in the same run (the headline value stays C3's)
        del base
        import gc
        gc.collect()
        w5 = WORKLOADS["ivfpq_10m"]
        t = time.time()
        b5, q5 = datagen.workload(w5["data"], n=w5["n"], nq=w5["nq"])
        log(f"[bench] ivfpq_10m: generated {b5.shape} base, {q5.shape} queries in {time.time() - t:.1f}s")
        ms5, roof5, cpu5, cfg5, extra5 = bench_ivfpq(args, w5, b5, q5, compare=False)
        extra["ivfpq_10m"] = {"metric": w5["metric_name"], "value": round(q5.shape[0] / ms5 * 1e3, 1),
                              "unit": "queries/s", "ms_per_step": round(ms5, 4), "steps": args.steps,
                              "warmup": args.warmup, "config": dict({"workload": w5["desc"]}, **cfg5),
                              "roofline": roof5, "cpu_baseline": cpu5}
        if "screen_copy" in extra5:
            extra["ivfpq_10m"]["screen_copy"] = extra5["screen_copy"]
    line = {
        "metric": w["metric_name"],
        "value": round(nq / ms_per_step * 1e3, 1),
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": dict({"workload": w["desc"]}, **cfg),
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    line.update(extra)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
