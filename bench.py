"""Benchmark of the exact brute-force k-NN hot path on one MI355X.

Workload (default): N=1,000,000 base vectors, D=1024, Q=100 queries, K=10,
on the clustered L2-normalised distribution (64 N(0, I) centres, sigma 0.3,
seed 12345).  The dataset is resident in HBM as fp16 tiles + fp32 norms (and
fp32 rows for the exact re-rank); queries and outputs are device buffers.
One step = one exact 10-NN search of the 100-query batch.

Prints ONE JSON line: whole-job throughput (queries/s), the roofline of the
dominant kernel (bf_scan, HBM-bound) from HIP events recorded on its stream,
recall@10 against an independent exact ground truth, and the reference's CPU
search path timed on this host on a bounded sample.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, published
REF_M3MAX_QPS = 1012.0  # reference README.md:23 (M3 Max, different data)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def load_package():
    from __graft_entry__ import load_package as lp
    return lp()


def exact_ground_truth(base: np.ndarray, qs: np.ndarray, k: int, extra: int = 64):
    """Exact k-NN on the host, independent of the GPU path: fp32 GEMM
    candidates (k + extra per query, over row chunks and query blocks), each
    re-scored in fp64 and ordered by (distance, id).  Returns k + 1 ids and
    fp64 distances per query."""
    n = base.shape[0]
    norms = np.einsum("ij,ij->i", base, base)
    keep_n = min(k + extra, n)
    gt_i = np.empty((qs.shape[0], k + 1), np.int64)
    gt_d = np.empty((qs.shape[0], k + 1), np.float64)
    qblock, chunk = 1000, 250_000
    for q0 in range(0, qs.shape[0], qblock):
        qb = qs[q0:q0 + qblock]
        best_d = np.full((qb.shape[0], 0), np.inf, np.float32)
        best_i = np.zeros((qb.shape[0], 0), np.int64)
        for s in range(0, n, chunk):
            e = min(n, s + chunk)
            approx = norms[None, s:e] - 2.0 * (qb @ base[s:e].T)
            m = min(keep_n, e - s)
            part = np.argpartition(approx, m - 1, axis=1)[:, :m]
            best_d = np.concatenate([best_d, np.take_along_axis(approx, part, 1)], 1)
            best_i = np.concatenate([best_i, part + s], 1)
            keep = np.argpartition(best_d, min(keep_n, best_d.shape[1]) - 1, axis=1)[:, :keep_n]
            best_d = np.take_along_axis(best_d, keep, 1)
            best_i = np.take_along_axis(best_i, keep, 1)
        for r in range(qb.shape[0]):
            c = best_i[r]
            dd = ((base[c].astype(np.float64) - qb[r].astype(np.float64)) ** 2).sum(1)
            o = np.lexsort((c, dd))[:k + 1]
            gt_i[q0 + r, :len(o)], gt_d[q0 + r, :len(o)] = c[o], dd[o]
    return gt_i, gt_d


def recall_at_k(nbr: np.ndarray, gt_i: np.ndarray, k: int) -> float:
    hits = sum(len(set(nbr[i, :k].tolist()) & set(gt_i[i, :k].tolist())) for i in range(nbr.shape[0]))
    return hits / float(nbr.shape[0] * k)


def cpu_baseline(base: np.ndarray, qs: np.ndarray, k: int, sample_q: int):
    """The reference's CPU search (src/cagra.cpp:211-252) on `sample_q` queries."""
    import oracle

    sub = np.ascontiguousarray(qs[:sample_q])
    if oracle.have_reference():
        kind = "reference"
        fn = lambda: oracle.ref_bf_search(base, sub, k)
    else:
        kind = "port"
        fn = lambda: oracle.bf_exact(base, sub, k, threads=1)
    t0 = time.perf_counter()
    fn()
    dt = time.perf_counter() - t0
    return {
        "value": sample_q / dt,
        "unit": "queries/s",
        "cores": 1,
        "kind": kind,
        "sample": f"{sample_q} of the {qs.shape[0]} queries against all {base.shape[0]} rows "
                  f"(D={base.shape[1]}, K={k}), single thread; host has {os.cpu_count()} cores",
    }


def read_traffic(name: str):
    """HBM bytes per launch from a committed rocprofv3 PMC summary, if any."""
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def calibrate_mfma() -> int:
    """The matrix-core rate this device sustains on a plain fp16 GEMM from
    the vendor library (torch.matmul -> hipBLASLt), fp32 accumulate, at the
    brute-force scan's inner dimension (M = 10,240 queries, N = 65,536 rows,
    K = 1,024) and at a square 8,192 shape.  A reference point next to the
    fused scan's fraction of the nominal 2.5 PFLOP/s (clocks drop under
    sustained matrix load)."""
    import torch

    out = {}
    for name, (m, n_, k) in {"scan_shape": (10240, 65536, 1024), "square_8192": (8192, 8192, 8192)}.items():
        a = torch.randn(m, k, device="cuda:0", dtype=torch.float16)
        b = torch.randn(n_, k, device="cuda:0", dtype=torch.float16).t().contiguous()
        for _ in range(3):
            torch.matmul(a, b)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 20
        start.record()
        for _ in range(reps):
            torch.matmul(a, b)
        end.record()
        torch.cuda.synchronize()
        tflops = 2.0 * m * n_ * k * reps / (start.elapsed_time(end) * 1e-3) / 1e12
        out[name] = {"m": m, "n": n_, "k": k, "tflops": tflops, "frac_of_nominal": tflops / MFMA_F16_PEAK_TFLOPS}
        del a, b
    print(json.dumps({"calibrate_mfma_fp16_gemm": out}), flush=True)

    # The library's own matrix-core loop (cvs_calibrate_mfma): the large-batch
    # scan's 4 x 4 register block of 32 x 32 x 16 MFMAs, one workgroup of 4
    # waves per compute unit, no memory traffic; operands held in registers
    # or re-read from LDS every k-step as the scan reads them.  The operand
    # values change the rate (power): random normals, the scan's own value
    # distribution (benchmark rows centred and scaled by a power of two so
    # that the largest magnitude lies in [128, 256), as the index stores
    # them), and zeros.
    cvs = load_package()
    ctx = cvs.Context(0)
    rows = torch.from_numpy(cvs.synth_clustered(12345, cvs.STREAM_BASE, 8192, 1024)).to("cuda:0")
    rows = rows - rows.mean(0)
    rows = rows * float(2.0 ** (8 - int(np.frexp(np.float32(rows.abs().max().item()))[1])))
    data = {"randn": torch.randn(8192, 1024, device="cuda:0", dtype=torch.float16),
            "scan_values": rows.to(torch.float16).contiguous(),
            "zeros": torch.zeros(8192, 1024, device="cuda:0", dtype=torch.float16)}
    loop = {}
    for name, t in data.items():
        for from_lds in (False, True):
            tf = ctx.calibrate_mfma(t.data_ptr(), t.numel() * 2, ctx.device_info()["compute_units"], 65536,
                                    from_lds=from_lds, reps=5)
            loop[f"{name}_{'lds' if from_lds else 'registers'}"] = {
                "tflops": tf, "frac_of_nominal": tf / MFMA_F16_PEAK_TFLOPS}
    ctx.close()
    print(json.dumps({"calibrate_mfma_loop": loop}), flush=True)
    return 0


def calibrate_copy(mib: int) -> int:
    """Copies `mib` MiB device-to-device with torch's copy_, which the HIP
    runtime serves with its blit kernel `__amd_rocclr_copyBuffer` (reads mib
    MiB, writes mib MiB per launch).  rocprofv3's FETCH_SIZE and
    WRITE_SIZE of that kernel, divided by mib MiB, give the factor by which
    the counters over- or under-report bytes on this device."""
    import torch

    n = mib * (1 << 20) // 4
    src = torch.rand(n, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    # Achievable streaming-read rate: a full reduction over the same buffer
    # (reads mib MiB, writes one float), timed with events on its stream.
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(3):
        src.sum()
    start.record()
    reps = 20
    for _ in range(reps):
        src.sum()
    end.record()
    torch.cuda.synchronize()
    read_gbs = n * 4 * reps / (start.elapsed_time(end) * 1e-3) / 1e9
    start.record()
    for _ in range(reps):
        dst.copy_(src)
    end.record()
    torch.cuda.synchronize()
    copy_gbs = 2 * n * 4 * reps / (start.elapsed_time(end) * 1e-3) / 1e9
    # The library's own streaming read (cvs_calibrate_stream_read): each
    # workgroup reads one contiguous share with non-temporal 16-byte loads,
    # as the brute-force scan reads its row range.
    # And its random whole-row gathers (cvs_calibrate_gather_read), the graph
    # search's access shape: 16-lane teams reading 256-byte segments of rows
    # picked at random over 100,000 rows, the graph-search configuration's
    # fp32 rows (4 KiB, a 410 MB set) and fp16 copy (2 KiB, 205 MB).
    cvs = load_package()
    with cvs.Context(0) as ctx:
        stream = {str(g): ctx.calibrate_stream_read(n * 4, g) for g in (256, 512, 1024, 2048, 4096, 8192)}
        gather = {f"{rb}B_rows": ctx.calibrate_gather_read(rb, 100_000, 1024, 64, reps=10) for rb in (4096, 2048)}
    print(json.dumps({"calibrate_copy_bytes": n * 4, "launches": 5, "read_gbs": read_gbs,
                      "copy_gbs_read_plus_write": copy_gbs, "stream_read_gbs_by_workgroups": stream,
                      "gather_read_gbs_100k_rows": gather}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--n", type=int, default=1_000_000)
    ap.add_argument("--d", type=int, default=1024)
    ap.add_argument("--q", type=int, default=100)
    ap.add_argument("--k", type=int, default=10)
    ap.add_argument("--seed", type=int, default=12345)
    ap.add_argument("--cpu-sample", type=int, default=10, help="queries timed on the CPU baseline")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-recall", action="store_true")
    ap.add_argument("--no-extras", action="store_true",
                    help="headline line only (no N=10K, Q=10,000 and graph-search legs)")
    ap.add_argument("--settle-ms", type=float, default=200.0,
                    help="wall time the search runs before the warmup steps, while the device's clocks settle")
    ap.add_argument("--calibrate-mfma", action="store_true",
                    help="time a plain fp16 GEMM from the vendor library (matrix-core reference point)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB a few times (PMC byte-counter calibration)")
    ap.add_argument("--workload", choices=["bf", "bf-large", "cagra-search", "cagra-build"], default="bf",
                    help="bf: the headline brute-force line (default); bf-large: brute force at N=1M "
                         "D=1024 Q=10,000 K=100; cagra-search: graph search at N=100K D=1024 Q=10,000 "
                         "degree 64; cagra-build: graph build at N=1M D=1024")
    ap.add_argument("--itopk", type=int, default=64)
    ap.add_argument("--degree", type=int, default=64)
    ap.add_argument("--exact-lists", action="store_true",
                    help="cagra-build: also prune exact k-NN lists of every row (brute force, the row itself "
                         "excluded) at the build's intermediate degree and compare the two graphs")
    args = ap.parse_args()

    if args.calibrate_copy:
        return calibrate_copy(args.calibrate_copy)
    if args.calibrate_mfma:
        return calibrate_mfma()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); "
              "how the search would shard over several GPUs is described in the design notes, "
              "but only the one-GPU path is built.", file=sys.stderr)
        return 2
    if args.workload == "cagra-search":
        return run_cagra_search(args)
    if args.workload == "bf-large":
        return run_bf_large(args)
    if args.workload == "cagra-build":
        return run_cagra_build(args)
    return run_bf(args)


def blas_topk(base: np.ndarray, qs: np.ndarray, k: int, chunk: int = 131_072):
    """The reference README's "AMX cblas" brute force (README.md:29) on this
    host: fp32 sgemm of the queries against row chunks (the vendor BLAS that
    numpy links, on all its threads), d = |q|^2 - 2 q.x + |x|^2, per-query
    top-k by (d, id).  Returns the ids (q x k)."""
    n = base.shape[0]
    qn = np.einsum("ij,ij->i", qs, qs)
    best_d = np.full((qs.shape[0], 0), np.inf, np.float32)
    best_i = np.zeros((qs.shape[0], 0), np.int64)
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        blk = base[s:e]
        d = qn[:, None] - 2.0 * (qs @ blk.T) + np.einsum("ij,ij->i", blk, blk)[None, :]
        m = min(k, e - s)
        part = np.argpartition(d, m - 1, axis=1)[:, :m]
        best_d = np.concatenate([best_d, np.take_along_axis(d, part, 1)], 1)
        best_i = np.concatenate([best_i, part + s], 1)
    o = np.lexsort((best_i, best_d), axis=1)[:, :k]
    return np.take_along_axis(best_i, o, 1)


def blas_threads() -> int:
    try:
        from threadpoolctl import threadpool_info
        return int(max(i.get("num_threads", 1) for i in threadpool_info() if i.get("user_api") == "blas"))
    except Exception:
        return 0


def timed_steps(ctx, fn, steps: int, families):
    """Runs `fn` `steps` times between two device synchronisations with the
    context's kernel timing off: the seconds returned.  Then the same
    `steps` again with the timing on (each launch carries start / end
    dispatch timestamps, which add ~6 us per launch to the step but not to
    the kernels): the mean ms per span of each family.  Returns (seconds,
    {family: mean ms per span})."""
    ctx.set_timing(False)
    ctx.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    ctx.synchronize()
    dt = time.perf_counter() - t0
    ctx.set_timing(True)
    for _ in range(steps):
        fn()
    ctx.synchronize()
    kt = {}
    for name in families:
        tot, cnt = ctx.kernel_time(name)
        kt[name] = tot / max(cnt, 1)
    ctx.set_timing(False)
    return dt, kt


def run_bf(args) -> int:
    rank = int(os.environ.get("RANK", "0"))
    cvs = load_package()
    n, d, q, k = args.n, args.d, args.q, args.k
    log(f"generating clustered data N={n} D={d} Q={q}")
    t = time.perf_counter()
    base = cvs.synth_clustered(args.seed, cvs.STREAM_BASE, n, d)
    qs = cvs.synth_clustered(args.seed, cvs.STREAM_QUERIES, q, d)
    log(f"data ready in {time.perf_counter() - t:.1f}s")
    gt_i = gt_d = None
    if not args.no_recall:
        # Host ground truth first, so that the GPU passes below run back to back.
        log("computing exact ground truth on the host")
        gt_i, gt_d = exact_ground_truth(base, qs, k)

    ctx = cvs.Context(0)
    info = ctx.device_info()
    log(f"device {info['name']} CUs={info['compute_units']}")
    t = time.perf_counter()
    ds = ctx.dataset(base)
    log(f"dataset uploaded + tiled in {time.perf_counter() - t:.2f}s")
    dq = cvs.DeviceArray.from_host(ctx, qs)
    dn = cvs.DeviceArray(ctx, (q, k), np.uint32)
    dd = cvs.DeviceArray(ctx, (q, k), np.float32)
    step = lambda: ds.bf_search_async(dq, k, dn, dd)
    families = ("bf_prep", "bf_sample", "bf_scan", "bf_merge")

    # Settle: on a GPU that has been idle, the first ~40 ms of this workload
    # run the HBM-bound scan up to 1.5x slower while the device's clocks
    # settle (kernel trace of the driver's command in profiles/).  The search
    # runs for --settle-ms of wall time before the warmup steps, with timing
    # on, which also fills the event pools the timed region reuses.
    settle_steps = 0
    ctx.set_timing(True)
    t_end = time.perf_counter() + args.settle_ms * 1e-3
    while time.perf_counter() < t_end:
        for _ in range(8):
            step()
        ctx.synchronize()
        settle_steps += 8
    for name in families:
        ctx.kernel_time(name)
    for _ in range(args.warmup):
        step()
    ctx.synchronize()
    for name in families:
        ctx.kernel_time(name)
    ctx.set_timing(False)
    log(f"settle ({settle_steps} steps) and warmup done")

    # Timed region: exactly K searches, device synchronised on both sides,
    # no timestamps; then each kernel's duration from its own dispatch
    # timestamps over K more searches (the timestamps lengthen a step by
    # ~24 us of the four dispatches' bookkeeping, not the kernels).
    ctx.bf_escalations(reset=True)
    elapsed, kavg = timed_steps(ctx, step, args.steps, families)
    escalated, rescanned = ctx.bf_escalations(reset=True)
    ms_per_step = 1e3 * elapsed / args.steps
    qps = q * args.steps / elapsed
    log(f"timed {args.steps} steps: {ms_per_step:.4f} ms/step, {qps:.0f} QPS")
    log("kernel avg ms: " + ", ".join(f"{kn}={v:.4f}" for kn, v in kavg.items()))
    scan_ms = kavg["bf_scan"]
    alg_bytes = n * d * 2 + n * 4 + q * d * 2 + q * k * 8
    achieved = alg_bytes / (scan_ms * 1e-3) / 1e9

    nbr = dn.to_host()
    dist = dd.to_host()
    result = {
        "metric": "brute-force QPS + recall@10 at N=1M D=1024 K=10 Q=100; % of HBM roofline",
        "value": qps,
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {
            "workload": f"exact brute-force k-NN, N={n} D={d} Q={q} K={k}, clustered L2-normalised "
                        "(64 centres, sigma 0.3), fp16 dataset tiles + fp32 norms, fp32 accumulate, "
                        "fp32 exact re-rank",
            "n": n, "d": d, "q": q, "k": k, "seed": args.seed,
            "device": info["name"], "compute_units": info["compute_units"],
        },
        "roofline": {
            "kernel": "bf_scan",
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": read_traffic("bf_scan_n1M_d1024_q100_k10_traffic.txt"),
            "algorithmic_bytes_per_launch": alg_bytes,
            "avg_launch_ms": scan_ms,
            "launch_timing": "dispatch timestamps (HIP events on the context stream) over a second pass "
                             f"of {args.steps} searches right after the timed region",
            "step_frac": alg_bytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS,
        },
        "kernel_avg_ms": kavg,
        # Queries (over both passes of timed_steps) whose fp16 candidate
        # selection was not certified exact and were re-ranked over more
        # rows: from the candidate lists, or over every row.
        "uncertified_queries": {"escalated": escalated, "rescanned_all_rows": rescanned,
                                "of": 2 * args.steps * q},
        "settle": {"ms": args.settle_ms, "steps": settle_steps},
        "reference_published_qps_m3max": REF_M3MAX_QPS,
    }
    if gt_i is not None:
        result["recall_at_10"] = recall_at_k(nbr, gt_i, k)
        rel = np.abs(dist.astype(np.float64) - gt_d[:, :k]) / np.maximum(gt_d[:, :k], 1e-30)
        result["max_rel_dist_err"] = float(rel.max())
    if not args.no_extras:
        result["c3_large_batch"] = leg_c3(cvs, ctx, ds, base, args)
    ds.close()
    if not args.no_extras:
        result["c4_graph_search"] = leg_c4(cvs, ctx, args)
        result["c1_small"] = leg_c1(cvs, ctx, args)
        result["c5_graph_build"] = leg_c5(cvs, ctx, base, args)
        result["bf_beyond_fused_limits"] = leg_wide(cvs, ctx, args)
    if rank == 0 and not args.no_cpu_baseline:
        log(f"timing the reference CPU path on {args.cpu_sample} queries")
        result["cpu_baseline"] = cpu_baseline(base, qs, k, args.cpu_sample)
        log("timing the all-core BLAS brute force")
        t0 = time.perf_counter()
        bi = blas_topk(base, qs, k)
        bdt = time.perf_counter() - t0
        result["cpu_blas_all_cores"] = {
            "value": q / bdt, "unit": "queries/s", "threads": blas_threads(), "host_cores": os.cpu_count(),
            "recall_at_10": recall_at_k(bi, gt_i, k) if gt_i is not None else None,
            "sample": f"all {q} queries against all {n} rows: fp32 sgemm (OpenBLAS via numpy) + top-k, "
                      "the reference README's cblas brute force (README.md:29)"}
    ctx.close()
    if rank == 0:
        print(json.dumps(result), flush=True)
    return 0


def leg_wide(cvs, ctx, args) -> dict:
    """N=1M D=1536 Q=100 K=10: the same search beyond the fused scan's
    dimension limit (1024), served by the keys-matrix path (sampled
    per-query threshold, list-only keys kernel, certified exact re-rank);
    the reference's CPU loop (src/cagra.cpp:211-252) has no such limit.
    Timed like the headline line: settle, warmup, exactly --steps searches
    between device synchronisations, then the kernels' dispatch timestamps
    over as many more."""
    n, d, q, k = 1_000_000, 1536, 100, 10
    t = time.perf_counter()
    base = cvs.synth_clustered(args.seed, cvs.STREAM_BASE, n, d)
    qs = cvs.synth_clustered(args.seed, cvs.STREAM_QUERIES, q, d)
    gt_i = None if args.no_recall else exact_ground_truth(base, qs, k)[0]
    ds = ctx.dataset(base)
    del base
    dq = cvs.DeviceArray.from_host(ctx, qs)
    dn = cvs.DeviceArray(ctx, (q, k), np.uint32)
    dd = cvs.DeviceArray(ctx, (q, k), np.float32)
    step = lambda: ds.bf_search_async(dq, k, dn, dd)
    families = ("bf_prep", "bf_sample", "bf_scan", "bf_merge")
    ctx.set_timing(True)
    t_end = time.perf_counter() + args.settle_ms * 1e-3
    while time.perf_counter() < t_end:
        for _ in range(8):
            step()
        ctx.synchronize()
    for _ in range(args.warmup):
        step()
    ctx.synchronize()
    for name in families:
        ctx.kernel_time(name)
    steps = min(args.steps, 100)
    ctx.bf_escalations(reset=True)
    elapsed, kavg = timed_steps(ctx, step, steps, families)
    escalated, rescanned = ctx.bf_escalations(reset=True)
    nbr = dn.to_host()
    ds.close()
    ms = 1e3 * elapsed / steps
    # Algorithmic bytes of the keys kernel: the fp16 tiles (1536 columns, no
    # padding at this width), the norms, the fp16 queries and the results.
    alg_bytes = n * d * 2 + n * 4 + q * d * 2 + q * k * 8
    achieved = alg_bytes / (kavg["bf_scan"] * 1e-3) / 1e9
    out = {"workload": f"exact brute-force k-NN, N={n} D={d} Q={q} K={k} (keys-matrix path: d > 1024)",
           "steps": steps, "ms_per_search": ms, "qps": q * steps / elapsed, "kernel_avg_ms": kavg,
           "keys_kernel_roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                    "frac": achieved / HBM_PEAK_GBS, "algorithmic_bytes_per_launch": alg_bytes,
                                    "traffic": read_traffic("bf_wide_n1M_d1536_q100_k10_traffic.txt")},
           "step_frac": alg_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
           "uncertified_queries": {"escalated": escalated, "rescanned_all_rows": rescanned, "of": 2 * steps * q},
           "recall_at_10": recall_at_k(nbr, gt_i, k) if gt_i is not None else None,
           "leg_seconds": time.perf_counter() - t}
    log(f"beyond the fused limits (D={d}): {ms:.4f} ms per search, keys kernel {achieved / HBM_PEAK_GBS:.3f} of HBM")
    return out


def leg_c1(cvs, ctx, args) -> dict:
    """N=10,000 D=1024 Q=100 K=10: the reference's CPU search loop
    (src/cagra.cpp:211-252, compiled from the reference sources) on one
    thread, and the GPU path on the same inputs."""
    import oracle

    n, d, q, k = 10_000, 1024, 100, 10
    base = cvs.synth_clustered(args.seed, cvs.STREAM_BASE, n, d)
    qs = cvs.synth_clustered(args.seed, cvs.STREAM_QUERIES, q, d)
    gt_i, _ = exact_ground_truth(base, qs, k)
    if oracle.have_reference():
        kind, fn = "reference", (lambda: oracle.ref_bf_search(base, qs, k))
    else:
        kind, fn = "port", (lambda: oracle.bf_exact(base, qs, k, threads=1))
    t0 = time.perf_counter()
    cpu_nbr, _ = fn()
    cpu_dt = time.perf_counter() - t0
    ds = ctx.dataset(base)
    dq = cvs.DeviceArray.from_host(ctx, qs)
    dn = cvs.DeviceArray(ctx, (q, k), np.uint32)
    dd = cvs.DeviceArray(ctx, (q, k), np.float32)
    stepf = lambda: ds.bf_search_async(dq, k, dn, dd)
    for _ in range(20):
        stepf()
    dt, kt = timed_steps(ctx, stepf, 200, ("bf_scan",))
    gpu_nbr = dn.to_host()
    ds.close()
    out = {"workload": f"N={n} D={d} Q={q} K={k}",
           "cpu_reference": {"value": q / cpu_dt, "unit": "queries/s", "cores": 1, "host_cores": os.cpu_count(),
                             "kind": kind, "recall_at_10": recall_at_k(cpu_nbr, gt_i, k)},
           "gpu": {"qps": q * 200 / dt, "ms_per_batch": 1e3 * dt / 200, "scan_ms": kt["bf_scan"],
                   "recall_at_10": recall_at_k(gpu_nbr, gt_i, k)}}
    log("C1: " + json.dumps(out))
    return out


def leg_c5(cvs, ctx, base, args) -> dict:
    """Graph build on the same N=1M D=1024 rows, intermediate degree 128 ->
    degree 64 (the default build): seconds per phase, the local join's
    algorithmic rate (member rows gathered x fp16 row bytes / join kernel
    time) against the HBM peak, and recall@10 at itopk 64 of the built graph
    on 100 queries against an fp64 ground truth."""
    n, d = base.shape
    k, degree, itopk = 10, 64, 64
    qs = cvs.synth_clustered(args.seed, cvs.STREAM_QUERIES, 100, d)
    drows = cvs.DeviceArray.from_host(ctx, base)
    g = cvs.DeviceArray(ctx, (n, degree), np.uint32)
    ctx.synchronize()
    t = time.perf_counter()
    _, bst = ctx.cagra_build(drows, intermediate_degree=2 * degree, graph_degree=degree, out=g)
    wall = time.perf_counter() - t
    idx = ctx.cagra_index(drows, g, cvs.cagra_nav_nodes(n))
    nbr, _ = idx.search(qs, k, itopk_size=itopk)
    idx.close()
    g.free()
    drows.free()
    gt_i, _ = exact_ground_truth(base, qs, k)
    join_gbs = bst["join_bytes"] / (bst["join_ms"] * 1e-3) / 1e9 if bst["join_ms"] else None
    out = {"workload": f"CAGRA build N={n} D={d}, intermediate degree {2 * degree} -> {degree}",
           "seconds": wall, "seconds_seed": bst["seconds_seed"], "seconds_descent": bst["seconds_descent"],
           "seconds_prune": bst["seconds_prune"], "iterations": bst["iterations"], "join_ms": bst["join_ms"],
           "join_gbs_algorithmic": join_gbs,
           "join_hbm_frac_algorithmic": join_gbs / HBM_PEAK_GBS if join_gbs else None,
           "recall_at_10_itopk64": recall_at_k(nbr, gt_i, k), "recall_queries": len(qs)}
    if not args.no_cpu_baseline:
        # The reference's build algorithm on the host cores, restated (its
        # 1M run took 2714 s, partly on its GPU), on a bounded sample: the
        # first 10,000 rows, which the reference builds by exact seeding plus
        # nn-descent.  The GPU builds of the same rows beside it.
        import oracle

        sub = np.ascontiguousarray(base[:10_000])
        threads = max(1, min(os.cpu_count() or 1, 16))
        t0 = time.perf_counter()
        oracle.cagra_build_reference(sub, degree, threads=threads)
        cdt = time.perf_counter() - t0
        ctx.synchronize()
        t0 = time.perf_counter()
        ctx.cagra_build(sub, intermediate_degree=2 * degree, graph_degree=degree)
        own = time.perf_counter() - t0
        t0 = time.perf_counter()
        ctx.cagra_build_reference(sub, degree)
        refg = time.perf_counter() - t0
        out["cpu_baseline"] = {
            "value": cdt, "unit": "seconds per 10,000-row build", "cores": threads, "kind": "port",
            "sample": f"the reference's graph build restated (src/metal_context.mm:289-914), first 10,000 of the "
                      f"{n} rows, D={d}, degree {degree}, OpenMP over rows",
            "gpu_same_rows_seconds": {"this_build": own, "reference_algorithm": refg}}
    return out


def leg_c3(cvs, ctx, ds, base, args) -> dict:
    """N=1M D=1024 Q=10,000 K=100 on the dataset already resident: ms per
    1k queries, the scan's fraction of the fp16 dense MFMA peak, recall@100
    of 100 sampled queries against an fp64 ground truth."""
    n, d = base.shape
    q, k = 10_000, 100
    qs = cvs.synth_clustered(args.seed, cvs.STREAM_QUERIES, q, d)
    dq = cvs.DeviceArray.from_host(ctx, qs)
    dn = cvs.DeviceArray(ctx, (q, k), np.uint32)
    dd = cvs.DeviceArray(ctx, (q, k), np.float32)
    stepf = lambda: ds.bf_search_async(dq, k, dn, dd)
    for _ in range(2):
        stepf()
    ctx.bf_escalations(reset=True)
    dt, kt = timed_steps(ctx, stepf, 3, ("bf_prep", "bf_sample", "bf_scan", "bf_merge"))
    escalated, rescanned = ctx.bf_escalations(reset=True)
    dt /= 3
    nbr = dn.to_host()
    sample = np.random.default_rng(0).choice(q, 100, replace=False)
    gt_i, _ = exact_ground_truth(base, qs[sample], k)
    flops = 2.0 * q * n * d
    out = {"workload": f"N={n} D={d} Q={q} K={k}", "ms_per_batch": 1e3 * dt, "ms_per_1k_queries": 1e6 * dt / q,
           "qps": q / dt, "kernel_avg_ms": kt,
           "scan_tflops": flops / (kt["bf_scan"] * 1e-3) / 1e12,
           "scan_mfma_frac": flops / (kt["bf_scan"] * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS,
           "step_mfma_frac": flops / dt / 1e12 / MFMA_F16_PEAK_TFLOPS,
           "recall_at_100_sampled": recall_at_k(nbr[sample], gt_i, k), "recall_queries": len(sample),
           "uncertified_queries": {"escalated": escalated, "rescanned_all_rows": rescanned, "of": 6 * q}}
    if not args.no_cpu_baseline:
        sub = qs[:200]
        t0 = time.perf_counter()
        blas_topk(base, sub, k)
        bdt = time.perf_counter() - t0
        out["cpu_blas_all_cores"] = {"ms_per_1k_queries": 1e6 * bdt / len(sub), "threads": blas_threads(),
                                     "sample": f"{len(sub)} queries, per-1k time extrapolated"}
    dq.free()
    dn.free()
    dd.free()
    log("C3: " + json.dumps(out))
    return out


def leg_c4(cvs, ctx, args) -> dict:
    """Graph search at N=100,000 D=1024 fp32 on a degree-64 graph built by
    the reference's algorithm (on the GPU), navigation nodes as the
    reference picks them, itopk 64, K=10, Q=10,000, fp32 traversal (the
    reference's precision) at widths 1 and 4: QPS, recall@10 against an fp64
    ground truth, HBM bytes read per the committed counter profile, Q=1
    latency; and the restated reference search on the same graph."""
    import oracle

    n, d, q, k, itopk, degree = 100_000, 1024, 10_000, 10, 64, 64
    base = cvs.synth_clustered(args.seed, cvs.STREAM_BASE, n, d)
    qs = cvs.synth_clustered(args.seed, cvs.STREAM_QUERIES, q, d)
    t = time.perf_counter()
    graph, rst = ctx.cagra_build_reference(base, degree)
    build_s = time.perf_counter() - t
    nav = cvs.cagra_nav_nodes(n)
    idx = ctx.cagra_index(base, graph, nav, traversal_bits=32)
    gt_i, _ = exact_ground_truth(base, qs, k)
    dq = cvs.DeviceArray.from_host(ctx, qs)
    dn = cvs.DeviceArray(ctx, (q, k), np.uint32)
    dd = cvs.DeviceArray(ctx, (q, k), np.float32)
    st = cvs.DeviceArray(ctx, (q, 2), np.uint32)
    cap = 8192
    rec = cvs.DeviceArray(ctx, (q, cap), np.uint32)
    widths = []
    for width in (1, 4):
        stepf = lambda: idx.search_async(dq, k, dn, dd, itopk_size=itopk, search_width=width)
        for _ in range(2):
            stepf()
        dt, kt = timed_steps(ctx, stepf, 5, ("cagra_search",))
        dt /= 5
        nbr = dn.to_host()
        if width == 1:
            nbr_w1 = nbr
        # The same search once more, recording every query's evaluated rows,
        # then those row gathers replayed alone: the time the search's data
        # movement takes without the search (the roofline's denominator).
        idx.search_record_async(dq, k, dn, dd, st, rec, itopk_size=itopk, search_width=width)
        stats = st.to_host().astype(np.int64)
        replay_ms = idx.replay_gathers(rec, st, 32, reps=5)
        alg = float((stats[:, 0] * d * 4 + stats[:, 1] * width * degree * 4 + d * 4).sum())
        gathered = float(np.minimum(stats[:, 0], cap).sum() * d * 4)
        traffic = read_traffic(f"cagra_search_n100k_d1024_q10000_itopk64_fp32_w{width}_traffic.txt")
        kms = kt["cagra_search"]
        ent = {"search_width": width, "qps": q / dt, "ms_per_batch": 1e3 * dt, "kernel_ms": kms,
               "recall_at_10": recall_at_k(nbr, gt_i, k),
               "mean_distance_evaluations": float(stats[:, 0].mean()),
               "max_distance_evaluations": int(stats[:, 0].max()),
               "roofline": {"bound": "row gathers", "unit": "GB/s",
                            "achieved": gathered / (kms * 1e-3) / 1e9,
                            "peak": gathered / (replay_ms * 1e-3) / 1e9,
                            "frac": replay_ms / kms,
                            "peak_is": "the same rows gathered alone, same row shape, no search work "
                                       "(cvs_cagra_replay_gathers), measured in this run",
                            "gathered_bytes_per_batch": gathered, "replay_ms": replay_ms},
               "algorithmic_bytes_per_batch": alg,
               "algorithmic_rate_over_hbm_peak": alg / (kms * 1e-3) / 1e9 / HBM_PEAK_GBS}
        if traffic:
            # L2 -> memory-side fetches (FETCH_SIZE); on this device they
            # include Infinity Cache hits, which no exposed counter separates.
            ent["memory_side_bytes_per_batch"] = traffic
            ent["memory_side_rate_over_hbm_peak"] = traffic / (kms * 1e-3) / 1e9 / HBM_PEAK_GBS
        widths.append(ent)
    rec.free()
    # Q=1: 100 single-query calls, launch to results on the device.
    dn1 = cvs.DeviceArray(ctx, (1, k), np.uint32)
    dd1 = cvs.DeviceArray(ctx, (1, k), np.float32)
    lat = []
    for i in range(100):
        dq1 = cvs.DeviceArray.from_host(ctx, qs[i:i + 1])
        ctx.synchronize()
        t1 = time.perf_counter()
        idx.search_async(dq1, k, dn1, dd1, itopk_size=itopk)
        ctx.synchronize()
        lat.append(time.perf_counter() - t1)
        dq1.free()
    lat.sort()
    # The restated reference search (nearest nav node entry, beam of itopk)
    # on the same graph, all host cores, sampled queries.
    sample = 500
    threads = os.cpu_count() or 1
    t0 = time.perf_counter()
    ref_nbr, _ = oracle.cagra_reference_search(base, graph, nav, qs[:sample], k, itopk_size=itopk, threads=threads)
    cpu_dt = time.perf_counter() - t0
    idx.close()
    for a in (dq, dn, dd, st, dn1, dd1):
        a.free()
    out = {"workload": f"N={n} D={d} Q={q} K={k} itopk={itopk} degree={degree}, fp32 traversal",
           "graph_build_s": build_s, "graph_build": rst, "widths": widths,
           "q1_latency_ms_p50": 1e3 * lat[50], "q1_latency_ms_p99": 1e3 * lat[98],
           "reference_search_same_graph": {"recall_at_10": recall_at_k(ref_nbr, gt_i[:sample], k),
                                           "gpu_width1_recall_same_queries": recall_at_k(nbr_w1[:sample], gt_i[:sample], k),
                                           "queries": sample},
           "cpu_baseline": {"value": sample / cpu_dt, "unit": "queries/s", "cores": threads, "kind": "port",
                            "sample": f"restated reference beam search, {sample} queries, OpenMP over queries"}}
    log("C4: " + json.dumps(out))
    return out


MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16, published


def run_bf_large(args) -> int:
    """Brute force in the large-batch regime: N=1,000,000 D=1024, Q=10,000,
    K=100 in one call (device-resident queries and outputs).  Reports ms per
    batch and per 1k queries, MFMA utilisation of the scan (2*Q*N*D flops /
    scan time / fp16 dense peak), recall@100 on 200 sampled queries, and the
    reference CPU path on a few queries."""
    cvs = load_package()
    n = args.n
    d, q, k = args.d, 10_000 if args.q == 100 else args.q, 100 if args.k == 10 else args.k
    log(f"generating clustered data N={n} D={d} Q={q}")
    base = cvs.synth_clustered(args.seed, cvs.STREAM_BASE, n, d)
    qs = cvs.synth_clustered(args.seed, cvs.STREAM_QUERIES, q, d)
    ctx = cvs.Context(0)
    ds = ctx.dataset(base)
    dq = cvs.DeviceArray.from_host(ctx, qs)
    dn = cvs.DeviceArray(ctx, (q, k), np.uint32)
    dd = cvs.DeviceArray(ctx, (q, k), np.float32)
    for _ in range(2):
        ds.bf_search_async(dq, k, dn, dd)
    ctx.synchronize()
    steps = max(2, args.steps // 50)
    ctx.bf_escalations(reset=True)
    t0 = time.perf_counter()
    for _ in range(steps):
        ds.bf_search_async(dq, k, dn, dd)
    ctx.synchronize()
    dt = (time.perf_counter() - t0) / steps
    ctx.set_timing(True)
    for _ in range(steps):
        ds.bf_search_async(dq, k, dn, dd)
    ctx.synchronize()
    kt = {name: ctx.kernel_time(name) for name in ("bf_prep", "bf_sample", "bf_scan", "bf_merge")}
    ctx.set_timing(False)
    escalated, rescanned = ctx.bf_escalations(reset=True)
    kavg = {kn: v[0] / max(v[1], 1) for kn, v in kt.items()}
    flops = 2.0 * q * n * d
    nbr = dn.to_host()
    sample = np.random.default_rng(0).choice(q, 200, replace=False)
    gt_i, _ = exact_ground_truth(base, qs[sample], k)
    rec = recall_at_k(nbr[sample], gt_i, k)
    out = {
        "metric": "brute-force ms per 1k queries at N=1M D=1024 K=100 Q=10,000; MFMA utilisation",
        "value": dt * 1e3 * 1000 / q, "unit": "ms per 1k queries", "n_gpus": 1, "higher_is_better": False,
        "ms_per_batch": dt * 1e3, "qps": q / dt, "dtype": "f16", "data": "synthetic",
        "config": {"workload": f"exact brute-force k-NN, N={n} D={d} Q={q} K={k}, clustered L2-normalised",
                   "seed": args.seed},
        "kernel_avg_ms": kavg,
        "roofline": {"kernel": "bf_scan", "bound": "mfma", "achieved": flops / (kavg["bf_scan"] * 1e-3) / 1e12,
                     "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": flops / (kavg["bf_scan"] * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS,
                     "step_frac": flops / dt / 1e12 / MFMA_F16_PEAK_TFLOPS},
        "recall_at_100_sampled": rec,
        "uncertified_queries": {"escalated": escalated, "rescanned_all_rows": rescanned, "of": 2 * steps * q},
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(base, qs, k, 4)
    print(json.dumps(out), flush=True)
    return 0


def run_cagra_search(args) -> int:
    """Graph search, N=100,000 D=1024 fp32, degree-64 graph built on the GPU,
    itopk 64, search_width 1 and 4, K=10: QPS at Q=10,000 (device-resident
    queries and outputs), Q=1 latency, recall@10 against exact k-NN, and the
    restated reference search (nav-node entry, beam of itopk) on the same
    graph and the host's cores for the recall floor and the CPU baseline."""
    import oracle

    cvs = load_package()
    n = 100_000 if args.n == 1_000_000 else args.n
    d, k, q = args.d, 10, 10_000 if args.q == 100 else args.q
    log(f"generating clustered data N={n} D={d} Q={q}")
    base = cvs.synth_clustered(args.seed, cvs.STREAM_BASE, n, d)
    qs = cvs.synth_clustered(args.seed, cvs.STREAM_QUERIES, q, d)
    ctx = cvs.Context(0)
    # The configuration's graph: degree 64 built by the reference's algorithm
    # (IVF k-means seeding, bucketing, 2-hop nn-descent), here on the GPU.
    t = time.perf_counter()
    graph, rst = ctx.cagra_build_reference(base, args.degree)
    log(f"reference-algorithm graph built in {time.perf_counter() - t:.2f}s: {json.dumps(rst)}")
    t = time.perf_counter()
    own_graph, bst = ctx.cagra_build(base, intermediate_degree=2 * args.degree, graph_degree=args.degree)
    log(f"own graph built in {time.perf_counter() - t:.2f}s ({bst['iterations']} nn-descent iterations)")
    nav = cvs.cagra_nav_nodes(n)
    idx = ctx.cagra_index(base, graph, nav)
    gt = exact_ground_truth(base, qs, k)[0]
    own_idx = ctx.cagra_index(base, own_graph, nav, traversal_bits=16)
    own_nbr, _ = own_idx.search(qs, k, itopk_size=args.itopk)
    own_idx.close()
    dq = cvs.DeviceArray.from_host(ctx, qs)
    dn = cvs.DeviceArray(ctx, (q, k), np.uint32)
    dd = cvs.DeviceArray(ctx, (q, k), np.float32)
    st = cvs.DeviceArray(ctx, (q, 2), np.uint32)
    results = []
    for bits, width in ((16, 1), (16, 4), (32, 1), (32, 4)):
        idx.set_traversal(bits)
        for _ in range(2):
            idx.search_async(dq, k, dn, dd, itopk_size=args.itopk, search_width=width)
        ctx.synchronize()
        steps = max(1, args.steps // 50)
        t0 = time.perf_counter()
        for _ in range(steps):
            idx.search_async(dq, k, dn, dd, itopk_size=args.itopk, search_width=width)
        ctx.synchronize()
        dt = (time.perf_counter() - t0) / steps
        ctx.set_timing(True)
        idx.search_async(dq, k, dn, dd, itopk_size=args.itopk, search_width=width, stats=st)
        kms, _ = ctx.kernel_time("cagra_search")
        ctx.set_timing(False)
        nbr = dn.to_host()
        # The evaluated rows recorded, then their gathers replayed alone.
        rec = cvs.DeviceArray(ctx, (q, 8192), np.uint32)
        idx.search_record_async(dq, k, dn, dd, st, rec, itopk_size=args.itopk, search_width=width)
        replay_ms = idx.replay_gathers(rec, st, bits, reps=5)
        rec.free()
        stats = st.to_host().astype(np.int64)
        gathered = float(np.minimum(stats[:, 0], 8192).sum() * d * (bits // 8))
        if width == 1 and bits == 16:
            nbr_w1 = nbr.copy()
        # algorithmic bytes per query: distance evaluations x D x (2 for the
        # fp16 traversal copy, 4 for fp32 rows) + with fp16 traversal the
        # fp32 re-rank of the itopk list (itopk x D*4) + expanded nodes x
        # degree*4 (graph rows) + D*4 (the query)
        expanded = stats[:, 1] * width
        rerank = args.itopk * d * 4 if bits == 16 else 0
        alg_bytes = float((stats[:, 0] * d * (bits // 8) + rerank + expanded * args.degree * 4 + d * 4).sum())
        # Q=1 latency: 100 distinct queries, one call each (launch to results
        # on the device, synchronised), then the kernel alone (HIP events)
        dn1 = cvs.DeviceArray(ctx, (1, k), np.uint32)
        dd1 = cvs.DeviceArray(ctx, (1, k), np.float32)
        single = [cvs.DeviceArray.from_host(ctx, qs[i:i + 1]) for i in range(100)]
        lat, hits = [], 0
        for i, dq1 in enumerate(single):
            ctx.synchronize()
            t1 = time.perf_counter()
            idx.search_async(dq1, k, dn1, dd1, itopk_size=args.itopk, search_width=width)
            ctx.synchronize()
            lat.append(time.perf_counter() - t1)
            hits += len(set(dn1.to_host()[0].tolist()) & set(gt[i].tolist()))
        ctx.set_timing(True)
        for dq1 in single:
            idx.search_async(dq1, k, dn1, dd1, itopk_size=args.itopk, search_width=width)
        ctx.synchronize()
        k1ms, k1n = ctx.kernel_time("cagra_search")
        ctx.set_timing(False)
        lat.sort()
        res = {
            "traversal_bits": bits, "search_width": width, "qps": q / dt, "ms_per_batch": dt * 1e3, "kernel_ms": kms,
            "recall_at_10": recall_at_k(nbr, gt, k), "q1_latency_ms_p50": 1e3 * lat[50],
            "q1_latency_ms_p99": 1e3 * lat[98], "q1_kernel_ms": k1ms / max(k1n, 1), "q1_recall_at_10": hits / 1000,
            "mean_distance_evaluations": float(stats[:, 0].mean()), "mean_iterations": float(stats[:, 1].mean()),
            "algorithmic_bytes_per_batch": alg_bytes, "algorithmic_gbs": alg_bytes / (kms * 1e-3) / 1e9,
            "algorithmic_rate_over_hbm_peak": alg_bytes / (kms * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "roofline": {"bound": "row gathers", "unit": "GB/s", "achieved": gathered / (kms * 1e-3) / 1e9,
                         "peak": gathered / (replay_ms * 1e-3) / 1e9, "frac": replay_ms / kms,
                         "peak_is": "the same rows gathered alone (cvs_cagra_replay_gathers)",
                         "replay_ms": replay_ms},
        }
        # L2 -> memory-side fetches from the committed counter profile of this
        # kernel; they include Infinity Cache hits (no exposed counter
        # separates them from HBM reads).
        traffic = read_traffic(f"cagra_search_n100k_d1024_q10000_itopk64_fp{bits}_w{width}_traffic.txt")
        if traffic:
            res["memory_side_bytes_per_batch"] = traffic
            res["memory_side_gbs"] = traffic / (kms * 1e-3) / 1e9
        log(json.dumps(res))
        results.append(res)
    # Q=1 latency of multi-team search (teams x per-team list, fp16 traversal)
    idx.set_traversal(16)
    teams_lat = []
    for teams, per_team in ((8, 32), (16, 32), (8, 64)):
        lat, hits = [], 0
        for i, dq1 in enumerate(single):
            ctx.synchronize()
            t1 = time.perf_counter()
            idx.search_teams_async(dq1, k, dn1, dd1, teams, itopk_size=per_team)
            ctx.synchronize()
            lat.append(time.perf_counter() - t1)
            hits += len(set(dn1.to_host()[0].tolist()) & set(gt[i].tolist()))
        ctx.set_timing(True)
        for dq1 in single:
            idx.search_teams_async(dq1, k, dn1, dd1, teams, itopk_size=per_team)
        ctx.synchronize()
        tms, tn = ctx.kernel_time("cagra_search")
        ctx.set_timing(False)
        lat.sort()
        teams_lat.append({"teams": teams, "itopk_per_team": per_team, "q1_latency_ms_p50": 1e3 * lat[50],
                          "q1_latency_ms_p99": 1e3 * lat[98], "q1_kernel_ms": tms / max(tn, 1),
                          "q1_recall_at_10": hits / 1000})
        log(json.dumps(teams_lat[-1]))
    # restated reference search on the same graph, all host cores, sampled queries
    sample = min(q, args.cpu_sample * 50)
    threads = os.cpu_count() or 1
    t0 = time.perf_counter()
    ref_nbr, _ = oracle.cagra_reference_search(base, graph, nav, qs[:sample], k, itopk_size=args.itopk,
                                               threads=threads)
    cpu_dt = time.perf_counter() - t0
    ref_recall = recall_at_k(ref_nbr, gt[:sample], k)
    gpu_recall_sample = recall_at_k(nbr_w1[:sample], gt[:sample], k)
    out = {
        "metric": "CAGRA search QPS at recall@10, N=100K D=1024 degree 64 itopk 64 K=10 Q=10,000",
        "value": results[0]["qps"], "unit": "queries/s", "n_gpus": 1, "higher_is_better": True,
        "dtype": "f16 traversal, f32 re-rank", "data": "synthetic",
        "config": {"workload": f"CAGRA graph search, N={n} D={d} Q={q} K={k} itopk={args.itopk} "
                               f"degree={args.degree}, graph built by the reference's algorithm (on the GPU)",
                   "seed": args.seed},
        "widths": results,
        "reference_algorithm_build": rst,
        "own_build_graph": {"build": bst, "recall_at_10_fp16_width1": recall_at_k(own_nbr, gt, k)},
        "q1_teams": teams_lat,
        "reference_search_same_graph": {"recall_at_10": ref_recall, "queries": sample,
                                        "gpu_recall_at_10_same_queries": gpu_recall_sample},
        "cpu_baseline": {"value": sample / cpu_dt, "unit": "queries/s", "cores": threads, "kind": "port",
                         "sample": f"restated reference beam search, {sample} queries, itopk {args.itopk}, "
                                   f"OpenMP over queries"},
    }
    print(json.dumps(out), flush=True)
    return 0


def exact_list_graph(cvs, ctx, drows, inter, nav, idx, qs, gt, k: int, kd: int, args) -> dict:
    """The build's last phase (detour pruning, cvs_cagra_optimize) applied
    to the exact kd nearest neighbours of every row instead of the
    nn-descent lists: exact lists of width kd + 1 from the brute-force path
    with the rows as queries (the row itself is dropped by the pruning), in
    batches of 65,536 rows.  Reports the seconds of both steps, how many of
    the exact kd neighbours the nn-descent lists hold (first 2,000 rows),
    and recall@10 at itopk 64 to 512 of graphs made from either kind of
    list: detour-pruned with 0 to degree / 2 reverse edges, the plain k-NN
    graph, and the nn-descent lists of length `degree` (the shape of the
    reference's graph)."""
    n = drows.shape[0]
    ds = ctx.dataset(drows)
    knn = cvs.DeviceArray(ctx, (n, kd + 1), np.uint32)
    kdist = cvs.DeviceArray(ctx, (n, kd + 1), np.float32)
    ctx.bf_escalations(reset=True)
    ctx.synchronize()
    t = time.perf_counter()
    step = 65_536
    for lo in range(0, n, step):
        hi = min(n, lo + step)
        ds.bf_search_async(drows.rows(lo, hi), kd + 1, knn.rows(lo, hi), kdist.rows(lo, hi))
        ctx.synchronize()
        log(f"exact lists: rows {hi} of {n}, {time.perf_counter() - t:.1f} s")
    t_lists = time.perf_counter() - t
    escalated, rescanned = ctx.bf_escalations(reset=True)
    kdist.free()
    ds.close()
    g_ex = cvs.DeviceArray(ctx, (n, args.degree), np.uint32)
    t = time.perf_counter()
    ctx.cagra_optimize(knn, args.degree, out=g_ex)
    t_prune = time.perf_counter() - t
    g_ex_half = ctx.cagra_optimize(knn, args.degree, reverse_edges=args.degree // 2)
    m = min(n, 2000)
    ex = knn.to_host()
    nd = inter.rows(0, m).to_host()
    knn.free()
    held = []
    for u in range(m):
        row = ex[u][ex[u] != u][:kd]
        held.append(len(np.intersect1d(row, nd[u])) / len(row))
    # the plain exact k-NN graph: each row's `degree` nearest other rows, no
    # pruning and no reverse edges
    g = args.degree
    is_self = ex == np.arange(n, dtype=np.uint32)[:, None]
    plain = np.take_along_axis(ex, np.argsort(is_self, axis=1, kind="stable")[:, :g], 1)
    del ex, is_self
    nd_all = inter.to_host()
    # the graph the reference's build makes (src/cagra.cpp:47-60): nn-descent
    # lists of length `degree`, used as they are
    inter64 = cvs.DeviceArray(ctx, (n, g), np.uint32)
    ctx.cagra_build(drows, intermediate_degree=g, graph_degree=g, intermediate_out=inter64)
    nd64 = inter64.to_host()
    inter64.free()
    graphs = {"nn-descent 128 -> detour (this build)": None}
    for r in (4, 8, 16, g // 2):
        graphs[f"nn-descent 128 -> detour, {r} reverse"] = ctx.cagra_optimize(nd_all, g, reverse_edges=r)
    graphs["nn-descent 128 -> first 64"] = np.ascontiguousarray(nd_all[:, :g])
    graphs["nn-descent 64 (the reference's graph shape)"] = nd64
    graphs["exact 128 -> detour"] = g_ex
    graphs[f"exact 128 -> detour, {g // 2} reverse"] = g_ex_half
    graphs["exact knn 64"] = plain
    del nd_all
    rec = {}
    for name, gr in graphs.items():
        ix = idx if gr is None else ctx.cagra_index(drows, gr, nav)
        row = {}
        for it in (args.itopk, 2 * args.itopk, 4 * args.itopk, 512):
            for w in (1, 4):
                r, _ = ix.search(qs, k, itopk_size=it, search_width=w)
                row[f"itopk {it} width {w}"] = recall_at_k(r, gt, k)
        rec[name] = row
        if gr is not None:
            ix.close()
        log(f"graph variant {name}: {json.dumps(row)}")
    g_ex.free()
    res = {"seconds_exact_lists": t_lists, "seconds_prune": t_prune,
           "exact_list_queries_escalated": escalated, "exact_list_queries_rescanned": rescanned,
           "nn_descent_list_recall_of_exact": float(np.mean(held)), "list_recall_rows": m,
           "recall_at_10": rec, "queries": len(qs)}
    log("exact lists: " + json.dumps(res))
    return res


def run_cagra_build(args) -> int:
    """Graph build, N=1,000,000 D=1024 fp32, intermediate degree 128 ->
    degree 64: seconds per phase, local-join GB/s (rows gathered x fp16 row
    bytes / join kernel time), downstream recall@10 at itopk 64 on 1,000
    queries against exact k-NN."""
    cvs = load_package()
    n, d, k = args.n, args.d, 10
    q = 1000
    log(f"generating clustered data N={n} D={d}")
    base = cvs.synth_clustered(args.seed, cvs.STREAM_BASE, n, d)
    qs = cvs.synth_clustered(args.seed, cvs.STREAM_QUERIES, q, d)
    ctx = cvs.Context(0)
    drows = cvs.DeviceArray.from_host(ctx, base)
    g = cvs.DeviceArray(ctx, (n, args.degree), np.uint32)
    kd = 2 * args.degree
    inter = cvs.DeviceArray(ctx, (n, kd), np.uint32) if args.exact_lists else None
    log("building")
    t = time.perf_counter()
    _, bst = ctx.cagra_build(drows, intermediate_degree=kd, graph_degree=args.degree, out=g, intermediate_out=inter)
    wall = time.perf_counter() - t
    log(json.dumps(bst))
    nav = cvs.cagra_nav_nodes(n)
    idx = ctx.cagra_index(drows, g, nav)
    gt = exact_ground_truth(base, qs, k)[0]
    nbr, _ = idx.search(qs, k, itopk_size=args.itopk)
    # exact length of every edge of the built graph (the reference's
    # recompute_graph_distances): algorithmic bytes per node = degree
    # neighbour rows + the node's row (D*4 each) + graph row and output
    # (degree*4 each)
    ed = cvs.DeviceArray(ctx, (n, args.degree), np.float32)
    idx.edge_distances(out=ed)
    ctx.synchronize()
    ctx.set_timing(True)
    for _ in range(3):
        idx.edge_distances(out=ed)
    ctx.synchronize()
    ems, ecnt = ctx.kernel_time("cagra_edge_distances")
    ctx.set_timing(False)
    ems /= max(ecnt, 1)
    e_bytes = n * ((args.degree + 1) * d * 4 + 2 * args.degree * 4)
    out = {
        "metric": "CAGRA build seconds, N=1M D=1024 degree 128 -> 64; local-join HBM GB/s; recall@10 at itopk 64",
        "value": wall, "unit": "s", "n_gpus": 1, "higher_is_better": False, "dtype": "f16 (build distances)",
        "data": "synthetic",
        "config": {"workload": f"CAGRA graph build N={n} D={d}, random bucketing + nn-descent + pruning",
                   "seed": args.seed},
        "build": bst,
        "join_gbs": bst["join_bytes"] / (bst["join_ms"] * 1e-3) / 1e9 if bst["join_ms"] else None,
        "recall_at_10_itopk": {"itopk": args.itopk, "recall": recall_at_k(nbr, gt, k), "queries": q},
        "edge_distances": {"kernel_ms": ems, "algorithmic_bytes": e_bytes,
                           "achieved_gbs": e_bytes / (ems * 1e-3) / 1e9 if ems else None,
                           "hbm_frac": e_bytes / (ems * 1e-3) / 1e9 / HBM_PEAK_GBS if ems else None},
    }
    # The same build with the final intermediate lists re-ranked by exact
    # fp32 distances before pruning (cvs_cagra_build_ex): time and recall
    # against the fp16-ranked build above.
    if not args.no_recall:
        log("building with the fp32 re-score before pruning")
        g2 = cvs.DeviceArray(ctx, (n, args.degree), np.uint32)
        t = time.perf_counter()
        _, bst2 = ctx.cagra_build(drows, intermediate_degree=2 * args.degree, graph_degree=args.degree, out=g2,
                                  rescore_fp32=True)
        wall2 = time.perf_counter() - t
        idx2 = ctx.cagra_index(drows, g2, nav)
        rec2 = {}
        for it in (args.itopk, 512):
            r_on, _ = idx.search(qs, k, itopk_size=it)
            r_rs, _ = idx2.search(qs, k, itopk_size=it)
            rec2[f"itopk {it}"] = {"fp16_ranked": recall_at_k(r_on, gt, k), "fp32_rescored": recall_at_k(r_rs, gt, k)}
        idx2.close()
        g2.free()
        out["rescore_fp32"] = {"seconds": wall2, "seconds_rescore": bst2["seconds_rescore"],
                               "iterations": bst2["iterations"], "recall_at_10": rec2, "queries": q}
        log(json.dumps(out["rescore_fp32"]))
    if args.exact_lists:
        out["exact_lists"] = exact_list_graph(cvs, ctx, drows, inter, nav, idx, qs, gt, k, kd, args)
        inter.free()
    # The reference's own build algorithm at this size, on the GPU, for
    # comparison (above 200,000 rows: IVF k-means, product-quantised
    # per-cluster seeding re-scored exactly, one bucketing round, no
    # nn-descent; src/metal_context.mm:289-914, src/cagra.cpp:59).  The
    # reference's own run of it at N=1M took 2714 s for recall 0.72 at itopk
    # 512 (docs/multi-cta-ivf-pq-lessons.md:5).
    if n > 200_000 and d == 1024 and not args.no_recall:
        log("building with the reference's algorithm")
        t = time.perf_counter()
        rgraph, rst = ctx.cagra_build_reference(base, args.degree)
        rwall = time.perf_counter() - t
        log(json.dumps(rst))
        ridx = ctx.cagra_index(drows, rgraph, nav)
        rec = {}
        for it in (args.itopk, 512):
            rn, _ = ridx.search(qs, k, itopk_size=it)
            on, _ = idx.search(qs, k, itopk_size=it)
            rec[f"itopk {it}"] = {"reference_algorithm_graph": recall_at_k(rn, gt, k), "this_build": recall_at_k(on, gt, k)}
        out["reference_algorithm"] = {"seconds": rwall, "stats": rst, "recall_at_10": rec, "queries": q}
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
