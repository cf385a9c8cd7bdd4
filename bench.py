"""Benchmark of the fused per-point Vecchia refinement on one MI355X.

Workload (the headline configuration): N = 1,000,000 points uniform in the unit cube (seeded),
D = 3, n0 = 1000, k = 8, RBF table (variance 1, scale 0.05, 1000 log bins over [1e-4, 2],
jitter 1e-5) in Float32; xi and the cotangent vbar ~ N(0, 1). The graph is built with the
library's build_graph on the GPU (the same graph as the host build); inputs are resident in HBM
before timing starts.

A step is one pass of each op of the path over the batch: generate, generate_grad_xi and
generate_grad_vals (each recomputes the dense first layer and every per-point factorization,
as the reference does per call). value = N / step time (points through all three ops per
second); per-op rates are reported beside it.

The JSON line also carries:
  roofline     for the dominant per-point kernel (the factor pass), timed with HIP events on
               the stream it runs on, against 8 TB/s HBM (the bound for its algorithmic bytes);
  cpu_baseline the oracle (the C++/OpenMP restatement of the reference's CPU path) timed on
               this host's cores on the same workload.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "graphgp.jl_amd"))

METRIC = "points/s for generate, grad_xi, grad_vals at 1M pts k=8 fp32; % of roofline"
HBM_PEAK = 8.0e12
FP32_PEAK = 157.3e12


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def workload(N, D, n0, k, nbins, seed=20261201):
    import graphgp_hip as G
    rng = np.random.default_rng(seed)
    pts = rng.random((N, D))
    bins, vals = G.rbf_kernel(1.0, 0.05, 1e-4, 2.0, nbins, jitter=1e-5)
    t = time.perf_counter()
    prob = G.build_graph(pts, n0, k, bins.astype(np.float32), vals.astype(np.float32),
                         backend="hip")
    log(f"graph built on the GPU in {time.perf_counter() - t:.2f}s: N={N} n0={prob.n0} "
        f"levels={len(prob.offsets) - 1}")
    xi = np.random.default_rng(7).standard_normal(N).astype(np.float32)
    vb = np.random.default_rng(8).standard_normal(N).astype(np.float32)
    return prob, xi, vb


def factor_algorithmic(k, D, es=4):
    """Bytes and flops per refined point of the factor pass (mean_vec + std for one point):
    reads k int32 neighbour ids and (k+1)*D uint32 lattice coords, writes k+1 floats; flops by
    the convention FMA = 2, div/sqrt = 1: assembly 8P + Cholesky (n^3-n)/3 + P divides + n
    square roots + back-solve k(k-1) + k (n = k+1, P = n(n-1)/2)."""
    n = k + 1
    P = n * (n - 1) // 2
    bytes_ = 4 * k + 4 * (k + 1) * D + es * (k + 1)
    flops = 8 * P + (n ** 3 - n) // 3 + P + n + k * (k - 1) + k
    return bytes_, flops


def measured_traffic():
    """HBM bytes per k_factor launch from the committed counter summary (two rocprofv3 --pmc
    passes, FETCH_SIZE and WRITE_SIZE, calibrated against a copy of known size), or None."""
    path = os.path.join(ROOT, "profiles", "k_factor_pmc_1M_k8_f32.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def cpu_baseline(prob, xi, vb, nthreads):
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    ref = O.Problem(prob.coords, prob.neighbors, prob.offsets, prob.n0, prob.scale, prob.bins,
                    prob.vals, indices=prob.indices, dtype=np.float32, nthreads=nthreads)
    ops = {"generate": lambda: ref.generate(xi), "grad_xi": lambda: ref.generate_grad_xi(vb),
           "grad_vals": lambda: ref.generate_grad_vals(xi, vb)}
    t = {}
    for name, f in ops.items():   # one warm-up, then the best of three (whole op each)
        f()
        best = float("inf")
        for _ in range(3):
            s = time.perf_counter()
            f()
            best = min(best, time.perf_counter() - s)
        t[name] = best
    return t


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--n", type=int, default=1_000_000)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--ops", default="generate,grad_xi,grad_vals")
    ap.add_argument("--calib-copy", action="store_true",
                    help="run one 256 MiB device copy first (the known-size reference kernel for "
                         "calibrating HBM byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for {args.gpus}); the path's multi-GPU "
              "sharding is a design, not part of this build", file=sys.stderr)
        sys.exit(2)

    import torch
    import graphgp_hip as G
    from graphgp_hip import _native as nat

    if args.calib_copy:
        src = torch.ones(64 * 1024 * 1024, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    N, D, n0, k, nbins = args.n, 3, 1000, 8, 1000
    prob, xi_np, vb_np = workload(N, D, n0, k, nbins)
    hp = G.to_backend(prob)
    xi = torch.from_numpy(xi_np).cuda()
    vb = torch.from_numpy(vb_np).cuda()
    ops = args.ops.split(",")
    fns = {
        "generate": lambda: G.generate(hp, xi),
        "grad_xi": lambda: G.generate_grad_xi(hp, vb),
        "grad_vals": lambda: G.generate_grad_vals(hp, xi, vb),
    }
    for _ in range(args.warmup):
        for o in ops:
            fns[o]()
    torch.cuda.synchronize()
    # The timed region times the roofline kernel only: each HIP event pair costs the op a few
    # microseconds, so the other kernels are timed in a separate pass below.
    nat.call("ggp_kernel_timers", hp.handle, 1)
    per = {o: 0.0 for o in ops}
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        for o in ops:
            s = time.perf_counter()
            fns[o]()
            per[o] += time.perf_counter() - s
    torch.cuda.synchronize()
    total = time.perf_counter() - t0
    ms_step = total / args.steps * 1e3

    def timer(name):
        tot, cnt = C.c_double(), C.c_int64()
        nat.call("ggp_kernel_timer_read", hp.handle, name.encode(), C.byref(tot), C.byref(cnt))
        return tot.value, cnt.value

    tot, cnt = timer("factor")
    fac_ms = tot / cnt
    # per-kernel breakdown: a separate pass of a few steps with every timer on
    nat.call("ggp_kernel_timers", hp.handle, 63)
    kpass = 3
    for _ in range(kpass):
        for o in ops:
            fns[o]()
    torch.cuda.synchronize()
    kernels = {}
    for name in ("factor", "pullback", "sweep_fwd", "sweep_rev", "dense"):
        tot, cnt = timer(name)
        if cnt:
            kernels[name] = {"avg_ms": tot / cnt, "launch_groups": cnt,
                             "ms_per_step": tot / kpass}
    nat.call("ggp_kernel_timers", hp.handle, 0)
    M = prob.M
    fb, ff = factor_algorithmic(k, D)
    achieved = fb * M / (fac_ms * 1e-3)
    roofline = {"kernel": "k_factor (mean_vec + std for all refined points)", "bound": "hbm",
                "achieved": achieved / 1e9, "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                "frac": achieved / HBM_PEAK, "traffic": measured_traffic(), "traffic_unit": "bytes per launch",
                "algorithmic_bytes_per_point": fb, "points_per_launch": M,
                "flop_frac_fp32": ff * M / (fac_ms * 1e-3) / FP32_PEAK,
                "avg_launch_ms": fac_ms}
    per_op = {o: {"ms": per[o] / args.steps * 1e3, "points_per_s": N / (per[o] / args.steps)}
              for o in ops}
    line = {
        "metric": METRIC, "value": N / (total / args.steps), "unit": "points/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded uniform points, N(0,1) xi and cotangent)",
        "config": {"workload": "1M points uniform in [0,1)^3, n0=1000, k=8, RBF var 1 scale 0.05, "
                               "1000 log bins [1e-4,2], jitter 1e-5, f32; step = generate + "
                               "generate_grad_xi + generate_grad_vals",
                   "N": N, "n0": prob.n0, "k": k, "D": D, "levels": len(prob.offsets) - 1},
        "per_op": per_op, "kernels": kernels, "roofline": roofline,
    }
    if not args.no_cpu:
        # the host's CPU share: OMP_NUM_THREADS when the environment sets it, else the affinity
        nthreads = int(os.environ.get("OMP_NUM_THREADS") or
                       (len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()))
        log(f"cpu baseline on {nthreads} threads ...")
        t = cpu_baseline(prob, xi_np, vb_np, nthreads)
        tt = sum(t[o] for o in ("generate", "grad_xi", "grad_vals"))
        line["cpu_baseline"] = {
            "value": N / tt, "unit": "points/s", "cores": nthreads, "kind": "port",
            "sample": "the full 1M-point workload; each op timed whole, best of 3 after a warm-up",
            "per_op_s": t, "speedup": (N / (total / args.steps)) / (N / tt)}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
