"""Benchmark of the exact Lloyd pass on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload outliers_d32]

A step is one Lloyd iteration over the whole workload (assignment, compensated per-cluster accumulation,
float64 centre update and stopping test), run by the engine's GPU-resident loop with the data already in HBM.
The default workload is 10M x 32 float32, k=64, with 1% outliers (synthetic, seeded). The JSON line carries the
per-pass time, the dominant kernel's achieved HBM bandwidth measured with HIP events on the engine's stream,
and the CPU baseline (this repository's restatement of the reference's multithreaded C++ pass, kmeans.mm,
timed on the host's cores over a row sample and scaled to the full workload).
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "mlx-kmeans_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "ms per Lloyd pass + achieved % of HBM/MFMA roofline, 10M×32 fp32 k=64"
HBM_PEAK_GBS = 8000.0          # MI355X published HBM3E bandwidth
FP32_PEAK_TFLOPS = 157.3       # MI355X published fp32 (matrix) peak
BF16_PEAK_TFLOPS = 2500.0      # MI355X published dense bf16 MFMA peak

DESCRIPTIONS = {
    "outliers_d32": "10M x 32 fp32, k=64, 64-component mixture + 1% uniform outliers, k-means++ start",
    "blobs_d32": "100k x 32 fp32, k=64, 64-component mixture, k-means++ start",
    "lowd_d8": "10M x 8 fp32, k=8, 8-component diagonal mixture",
    "pixels_d4": "96M x 4 fp32, k=12, 12-class clipped correlated mixture",
    "embed_d768": "1M x 768 fp32, k=1024, unit-norm vMF-style embeddings",
    "embed_d1536": "1M x 1536 fp32, k=1024, unit-norm vMF-style embeddings",
    "blobs_d960": "1M x 960 fp32, k=1024, GIST-width 1024-blob mixture, k-means++ start",
    "blobs_d48": "10M x 48 fp32, k=64, 64-component mixture, k-means++ start",
    "blobs_d32_k128": "10M x 32 fp32, k=128, 128-component mixture, k-means++ start",
    "blobs_d96": "10M x 96 fp32, k=64, 64-component mixture, k-means++ start",
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def profile_summary(name):
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3 --pmc summary for this
    workload (FETCH_SIZE + WRITE_SIZE, each calibrated on a plain copy), or None if there is none."""
    path = os.path.join(ROOT, "profiles", f"traffic_{name}.md")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.startswith("traffic_bytes_per_launch:"):
                return float(line.split(":", 1)[1])
    return None


def cpu_threads():
    """-> (threads used, description): the host CPUs this process may run on, capped at OMP_NUM_THREADS (the
    share of a shared host's cores allotted to one GPU's jobs, 16 on the MI355X machines this runs on)."""
    host = os.cpu_count() or 1
    allowed = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else host
    cap = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or allowed
    used = max(1, min(allowed, cap))
    return used, (f"{used} threads: the host has {host} CPUs, this process may use {allowed}, and "
                  f"OMP_NUM_THREADS={os.environ.get('OMP_NUM_THREADS', 'unset')} is its share of a shared host")


def cpu_baseline(X, C, budget_s=12.0):
    import oracle
    cores, why = cpu_threads()
    n = len(X)
    rows = min(n, 2_000_000)
    sample = X[:rows]
    oracle.cpu_pass(sample[: min(rows, 50_000)], C, nthreads=cores)    # warm
    times = []
    t_all = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        oracle.cpu_pass(sample, C, nthreads=cores)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_all > budget_s or len(times) >= 20:
            break
    per_pass_ms = float(np.median(times)) * 1e3 * (n / rows)
    return {"value": round(per_pass_ms, 3), "unit": "ms/pass", "cores": cores, "kind": "port",
            "host_cpus": os.cpu_count(), "threads_note": why,
            "sample": f"first {rows:,} of {n:,} rows, {len(times)} passes, median scaled by {n / rows:g}; "
                      f"kmeans.mm CPU backend restated (oracle/kmeans_oracle.c orc_cpu_pass)"}


def cpu_baseline_numpy(X, C, budget_s=8.0):
    """The second CPU baseline: kmeans_simple.py:45-78 restated in numpy (expanded-form distances through the
    BLAS, argmin, scatter-add, float64 host totals), on a row sample scaled to the full workload."""
    import oracle
    cores, why = cpu_threads()
    n = len(X)
    rows = min(n, 1_000_000)
    sample = X[:rows]
    oracle.kmeans_simple_pass(sample[: min(rows, 20_000)], C)    # warm
    times = []
    t_all = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        oracle.kmeans_simple_pass(sample, C)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_all > budget_s or len(times) >= 10:
            break
    per_pass_ms = float(np.median(times)) * 1e3 * (n / rows)
    return {"value": round(per_pass_ms, 3), "unit": "ms/pass", "cores": cores, "kind": "port",
            "host_cpus": os.cpu_count(), "threads_note": "BLAS " + why,
            "sample": f"first {rows:,} of {n:,} rows, {len(times)} passes, median scaled by {n / rows:g}; "
                      f"kmeans_simple.py restated in numpy (oracle.kmeans_simple_pass)"}


def seed_probe(workload):
    """k-means++ seeding time at the workload's shape: the GPU seeding KMeans.fit uses, against the host float64
    greedy k-means++ the synthetic workloads use for their start centres (same sample size and trials)."""
    import torch
    from mlx_kmeans import core, synthetic
    w = synthetic.WORKLOADS[workload]()
    X, k = w["X"], w["k"]
    n = len(X)
    dd = core.DeviceData([X])
    core.kmeans_pp_init(dd, n, k, np.random.default_rng(1))   # warm
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    core.kmeans_pp_init(dd, n, k, np.random.default_rng(1))
    gpu_ms = (time.perf_counter() - t0) * 1e3
    dd.close()
    t0 = time.perf_counter()
    synthetic.kmeans_pp_init([X], n, k, np.random.default_rng(1))
    host_ms = (time.perf_counter() - t0) * 1e3
    m = min(n, min(200_000, max(20_000, 20 * k)))
    print(json.dumps({"seed_probe": workload, "k": k, "dims": X.shape[1], "sample_rows": m, "gpu_ms": round(gpu_ms, 2),
                      "host_f64_ms": round(host_ms, 1)}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=0,
                    help="untimed passes after the settling passes and before the timed ones (default 0)")
    ap.add_argument("--workload", default="outliers_d32", choices=sorted(DESCRIPTIONS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-bounds", action="store_true",
                    help="turn the per-centre bounds between passes off (every wide-row pass screens every pair)")
    ap.add_argument("--approx", action="store_true",
                    help="exact=False: the wide-row screen's minimiser taken on trust (other shapes run exact)")
    ap.add_argument("--seed-probe", action="store_true",
                    help="only time k-means++ seeding of the workload (GPU, and the host float64 version)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only copy 1 GiB with torch (a plain copy kernel of known size, for counter calibration)")
    ap.add_argument("--stream-probe", action="store_true",
                    help="only measure the HBM streaming-read rate (the library's probe kernel over 4 GiB)")
    a = ap.parse_args()
    if a.stream_probe:
        from mlx_kmeans import _lib
        ctx = _lib.Context(0)
        print(json.dumps({"stream_read_gbs": round(ctx.stream_probe(4 << 30, 20), 1), "bytes": 4 << 30}), flush=True)
        ctx.close()
        return
    if a.copy_probe:
        import torch
        x = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
        y = torch.empty_like(x)
        for _ in range(3):
            y.copy_(x)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": x.numel() * 4}), flush=True)
        return
    if a.seed_probe:
        seed_probe(a.workload)
        return
    if a.gpus != 1:
        print(f"bench.py runs on one GPU: --gpus {a.gpus} is not supported (the Lloyd pass shards by rows; "
              f"the multi-GPU exchange is design-only in this build)", file=sys.stderr)
        sys.exit(2)

    import torch
    from mlx_kmeans import _lib, synthetic

    log(f"[bench] generating {a.workload}")
    w = synthetic.WORKLOADS[a.workload]()
    X, C0, k = w["X"], w["C0"], w["k"]
    n, d = X.shape
    ctx = _lib.Context(0)
    ctx.set_parts([X])
    if a.no_bounds:
        ctx.bounds(0.0)
    log(f"[bench] data on device: {n} x {d}, k={k}")

    # the streaming-read rate the roofline is read against, measured first (it also brings the GPU's clocks up
    # before the warmup passes)
    stream_gbs = ctx.stream_probe(1 << 30, 10)
    log(f"[bench] streaming read probe: {stream_gbs:.1f} GB/s")
    # The reference's timing rule (quick_bench.py:34-45): at least 0.3 s of the same work before anything is
    # timed, since millisecond kernels timed while the GPU's clocks ramp read slow (a 20-pass fit here: 0.26-0.28
    # ms/pass after 5 passes of a fresh process, 0.245 after 0.3 s). These settling fits come first and are
    # reported apart; then the `warmup` untimed passes, then exactly `steps` Lloyd iterations timed by the host
    # clock around device synchronisations. tol = -1 never stops the loop, so a workload that reaches a fixed point
    # early still runs every pass.
    mode = _lib.KM_APPROX if a.approx else _lib.KM_EXACT
    settle, tw = 0, time.perf_counter()
    while settle < 3 or time.perf_counter() - tw < 0.3:
        ctx.fit(C0, 10, -1.0, mode=mode)
        torch.cuda.synchronize()
        settle += 10
    settle_s = time.perf_counter() - tw
    if a.warmup > 0:
        ctx.fit(C0, a.warmup, -1.0, mode=mode)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    C, inertia, iters, _ = ctx.fit(C0, a.steps, -1.0, mode=mode)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    assert iters == a.steps, (iters, a.steps)
    ms = elapsed * 1e3 / a.steps
    log(f"[bench] {a.steps} passes in {elapsed * 1e3:.3f} ms -> {ms:.4f} ms/pass, path {ctx.last_path()}")

    # dominant kernel: HIP events around every launch on the engine's stream, over the same loop
    ctx.profile(True)
    b0 = ctx.bounds_info()
    ctx.fit(C0, a.steps, -1.0, mode=mode)
    prof = ctx.profile_read()
    pass_ms = ctx.profile_passes()
    ctx.profile(False)
    b1 = ctx.bounds_info()
    bounds = {"passes_on_bounds": b1["on_bounds"] - b0["on_bounds"], "builds": b1["builds"] - b0["builds"],
              "tracked": b1["tracked"] - b0["tracked"], "last_fraction": b1["last_fraction"]}
    log("[bench] per-pass ms (events): " + " ".join(f"{t:.4f}" for t in pass_ms))
    kname, (kms, kcount) = max(prof.items(), key=lambda kv: kv[1][0])
    avg_ms = kms / kcount
    log("[bench] kernels: " + ", ".join(f"{k_}: {v[0] / v[1] * 1e3:.1f} us x{v[1]}" for k_, v in prof.items()))
    if a.workload.startswith("embed_d") or a.workload == "blobs_d960":
        flops = 2.0 * n * k * d
        # a pass on the per-centre bounds (or one that builds them, in its own kernel) leaves the plain screen at
        # its first instruction: only the launches that screened every pair count, and their time
        full = kcount
        if kname == "km_big_screen":
            full = max(kcount - bounds["passes_on_bounds"] - bounds["builds"], 0)
        avg_ms = kms / max(full, 1)
        achieved = flops / (avg_ms * 1e-3) / 1e12 if full else 0.0
        roof = {"bound": "mfma", "achieved": round(achieved, 2), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / BF16_PEAK_TFLOPS, 4), "traffic": profile_summary(a.workload),
                "kernel": kname, "kernel_avg_ms": round(avg_ms, 5), "flops_per_launch": flops,
                "full_screen_launches": full, "launches": kcount}
    else:
        bytes_alg = float(n) * d * 4
        achieved = bytes_alg / (avg_ms * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": profile_summary(a.workload),
                "kernel": kname, "kernel_avg_ms": round(avg_ms, 5), "bytes_per_launch": bytes_alg,
                "peak_measured": round(stream_gbs, 1), "frac_measured": round(achieved / stream_gbs, 4)}
    cpu = None if a.no_cpu else cpu_baseline(X, C0)
    cpu2 = None if a.no_cpu else cpu_baseline_numpy(X, C0)
    out = {
        "metric": METRIC,
        "value": round(ms, 5),
        "unit": "ms/pass",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "settle": {"passes": settle, "seconds": round(settle_s, 3),
                   "rule": "at least 0.3 s of the same fits before the warmup passes (quick_bench.py:34-45)"},
        "ms_per_step": round(ms, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"{a.workload}: {DESCRIPTIONS[a.workload]}", "rows": n, "dims": d, "k": k,
                   "mode": "exact=False" if a.approx else "exact",
                   "parallelism": "single GPU"},
        "rows_per_s": round(n / (ms * 1e-3)),
        "pass_ms_events": {"median": round(float(np.median(pass_ms)), 5), "min": round(float(pass_ms.min()), 5),
                           "max": round(float(pass_ms.max()), 5), "first": round(float(pass_ms[0]), 5),
                           "passes": int(len(pass_ms)),
                           "note": "HIP events at every pass boundary of a second timed loop; the first pass of "
                                   "a fit accumulates every row, later passes only the rows whose label changed "
                                   "(on the wide-row path, when at most half the rows changed)"},
        "stream_read_gbs": round(stream_gbs, 1),
        "bounds": bounds,
        "final_inertia": inertia,
        "roofline": roof,
        "cpu_baseline": cpu,
        "cpu_baseline_numpy": cpu2,
    }
    print(json.dumps(out), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
