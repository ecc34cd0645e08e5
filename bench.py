"""Batch IVF-PQ search throughput on one MI355X.

Workload (the configuration the headline metric is quoted on): IVF-PQ over
1,000,000 x 128 f32 vectors with non-negative integer components drawn from a
1024-component Gaussian mixture (per-dim std 20, clipped to [0, 255]);
nlist = 1024 k-means lists, M = 16 subvectors x 8 dims, 256 codewords each;
nprobe = 16; 10,000 queries from the same mixture; k = 10; Euclidean.

A step is one batch_search of all 10,000 queries with the queries, the index
and the outputs resident in HBM: coarse selection + fused LUT/ADC/top-k scan.
The index is built on the GPU first (IVFPQIndex::build, seeded).

The roofline object covers the dominant kernel (the fused scan).  Its
achieved figure is the algorithmic code bytes (sum over queries of the sizes
of its 16 probed lists, times M = 16 bytes) divided by the scan kernel's mean
duration measured with HIP events on the stream it runs on.

cpu_baseline: the oracle (a C++ restatement of the reference's
batch_search_parallel with its AVX2 kernels) on a bounded query sample, on
the host cores of the same machine.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "forge-db_amd"))

METRIC = "batch QPS at k=10, IVF-PQ 1M×128 nprobe=16; ADC-scan HBM GB/s"
HBM_PEAK_GBS = 8000.0


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


def read_traffic():
    """HBM bytes per scan launch from the committed rocprofv3 --pmc summary, if any."""
    p = os.path.join(ROOT, "profiles", "ivfpq_scan_1Mx128_traffic.txt")
    if not os.path.exists(p):
        return None
    for line in open(p):
        if line.startswith("hbm_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--n", type=int, default=1_000_000)
    ap.add_argument("--nq", type=int, default=10_000)
    ap.add_argument("--timing-reps", type=int, default=10)
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="target wall time of the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run one plain 1 GiB device-to-device copy (a known-size "
                         "reference for the FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              f"(asked for --gpus {args.gpus}).", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from forgedb import LUT_EXACT, LUT_FAST, IVFPQIndex, datagen

    nlist, M, nprobe, k = 1024, 16, 16, 10
    t = time.time()
    base, queries = datagen.workload("ivfpq_int", n=args.n, nq=args.nq)
    log(f"[bench] generated {base.shape} base, {queries.shape} queries in {time.time() - t:.1f}s")
    t = time.time()
    index = IVFPQIndex.build(base, nlist, M, seed=args.seed)
    log(f"[bench] GPU build (k-means {nlist}, PQ {M}x256, encode) in {time.time() - t:.1f}s")
    index.set_nprobe(nprobe)

    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream(device=dev)
    nq = queries.shape[0]
    q_d = torch.from_numpy(queries).to(dev)
    ids_d = torch.empty((nq, k), dtype=torch.int64, device=dev)
    dist_d = torch.empty((nq, k), dtype=torch.float32, device=dev)
    cnt_d = torch.empty(nq, dtype=torch.int32, device=dev)
    torch.cuda.synchronize()
    sptr = stream.cuda_stream
    if args.calibrate_copy:
        src = torch.empty(1 << 28, dtype=torch.float32, device=dev)  # 1 GiB
        dst = torch.empty_like(src)
        src.fill_(1.0)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        log("[bench] calibration copy: 1 GiB device to device")

    def step():
        index.batch_search_device(q_d.data_ptr(), nq, k, ids_d.data_ptr(), dist_d.data_ptr(),
                                  cnt_d.data_ptr(), sptr)

    for _ in range(args.warmup):
        step()
    index.sync(sptr)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    index.sync(sptr)
    ms_per_step = (t1 - t0) * 1e3 / args.steps
    qps = nq / (ms_per_step / 1e3)
    log(f"[bench] {args.steps} steps: {ms_per_step:.3f} ms/step, {qps:,.0f} QPS")

    def kernel_times():
        coarse, scan = [], []
        for _ in range(args.timing_reps):
            c, s = index.batch_search_device(q_d.data_ptr(), nq, k, ids_d.data_ptr(),
                                             dist_d.data_ptr(), cnt_d.data_ptr(), sptr, timed=True)
            coarse.append(c)
            scan.append(s)
        return float(np.mean(coarse)), float(np.mean(scan))

    coarse_ms, scan_ms = kernel_times()
    exact_ids = ids_d.cpu().numpy().view(np.uint64).copy()

    # the opt-in fast LUT mode, timed the same way (distances within ~1e-6)
    index.set_lut_mode(LUT_FAST)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    fast_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    _, fast_scan_ms = kernel_times()
    fast_ids = ids_d.cpu().numpy().view(np.uint64)
    fast_agree = float(np.mean([len(set(fast_ids[q].tolist()) & set(exact_ids[q].tolist())) / k
                                for q in range(nq)]))
    index.set_lut_mode(LUT_EXACT)
    index.batch_search_device(q_d.data_ptr(), nq, k, ids_d.data_ptr(), dist_d.data_ptr(),
                              cnt_d.data_ptr(), sptr)
    index.sync(sptr)
    log(f"[bench] fast LUT mode: {fast_ms:.3f} ms/step, {nq / fast_ms * 1e3:,.0f} QPS, scan "
        f"{fast_scan_ms:.3f} ms; id agreement with exact mode {fast_agree:.6f}")

    lists, _ = index.probe(queries, nprobe)
    sizes = np.diff(index.list_offsets().astype(np.int64))
    scanned = int(sizes[lists].sum())
    code_bytes = scanned * M
    achieved = code_bytes / (scan_ms / 1e3) / 1e9
    log(f"[bench] coarse {coarse_ms:.3f} ms, scan {scan_ms:.3f} ms; {scanned / nq:,.0f} codes "
        f"per query; {code_bytes / 1e9:.3f} GB of codes -> {achieved:,.0f} GB/s")

    cpu = None
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import refcpu  # CPU baseline leg only
        art = index.export()
        oracle = refcpu.IvfPq.create(art["centroids"], art["codebooks"], art["list_offsets"],
                                     art["ids"], art["codes"])
        oracle.set_nprobe(nprobe)
        threads = min(16, os.cpu_count() or 1)
        probe_n = min(nq, 200)
        t = time.perf_counter()
        oracle.batch_search(queries[:probe_n], k, parallel=True, nthreads=threads)
        per_q = (time.perf_counter() - t) / probe_n
        sample = int(min(nq, max(probe_n, args.cpu_seconds / max(per_q, 1e-9))))
        t = time.perf_counter()
        oi, od, oc = oracle.batch_search(queries[:sample], k, parallel=True, nthreads=threads)
        cpu_s = time.perf_counter() - t
        cpu_qps = sample / cpu_s
        gi = ids_d[:sample].cpu().numpy().view(np.uint64)
        agree = float(np.mean([len(set(gi[q].tolist()) & set(oi[q].tolist())) / k
                               for q in range(sample)]))
        cpu = {"value": round(cpu_qps, 1), "unit": "queries/s", "cores": threads, "kind": "port",
               "sample": f"first {sample} of the {nq} queries, batch_search_parallel "
                         f"(chunks of 4), {cpu_s:.1f} s on {cpu_model()}",
               "gpu_id_agreement": round(agree, 6)}
        log(f"[bench] CPU baseline {cpu_qps:,.0f} QPS on {threads} threads "
            f"({sample} queries in {cpu_s:.1f}s); id agreement {agree:.6f}")

    line = {
        "metric": METRIC,
        "value": round(qps, 1),
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
        "config": {"workload": "IVF-PQ 1Mx128 integer Gaussian mixture (1024 comps, std 20), "
                               "nlist 1024, M 16x8, nprobe 16, Q 10000, k 10, Euclidean",
                   "n": args.n, "nq": nq, "nlist": nlist, "M": M, "nprobe": nprobe, "k": k},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": read_traffic(),
                     "kernel": "ivfpq_scan_kernel<16,8,1,0>", "kernel_ms": round(scan_ms, 4),
                     "algorithmic_bytes": code_bytes, "coarse_ms": round(coarse_ms, 4)},
        "fast_lut": {"value": round(nq / fast_ms * 1e3, 1), "ms_per_step": round(fast_ms, 4),
                     "scan_ms": round(fast_scan_ms, 4),
                     "achieved_gbs": round(code_bytes / (fast_scan_ms / 1e3) / 1e9, 1),
                     "id_agreement_with_exact": round(fast_agree, 6)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
