"""Benchmark of the fused per-point Vecchia refinement on one MI355X.

Default workload (the headline configuration, --config 2): N = 1,000,000 points uniform in the
unit cube (seeded), D = 3, n0 = 1000, k = 8, RBF table (variance 1, scale 0.05, 1000 log bins over
[1e-4, 2], jitter 1e-5) in Float32; xi and the cotangent vbar ~ N(0, 1). The graph is built with
the library's build_graph on the GPU (the same graph as the host build); inputs are resident in
HBM before timing starts. The other benchmark configurations run with --config 1, 3, 4, 5.

A step is one pass of each op of the configuration over the batch (for the headline workload:
generate, generate_grad_xi and generate_grad_vals; each recomputes the dense first layer and
every per-point factorization, as the reference does per call). value = N / step time; per-op
rates and their fractions of the roofline are reported beside it.

The JSON line also carries:
  roofline      for the kernel with the most GPU time in a step (found in a pre-pass with every
                kernel timer on), timed with HIP events on the stream it runs on over the timed
                region; achieved = its algorithmic bytes or flops per launch / average launch
                time. traffic = its HBM bytes per launch from two rocprofv3 --pmc passes
                (FETCH_SIZE, WRITE_SIZE) of a short run of the same workload, each scaled by
                what the counter reads for a 1 GiB device copy (the known-size reference), or
                null (--no-traffic, or no profiler);
  kernels       every timed kernel's average launch time and its own roofline fraction;
  cpu_baseline  the oracle (the C++/OpenMP restatement of the reference's CPU path) timed on
                this host's cores on the same workload (headline and 10K-point configurations).
"""
from __future__ import annotations

import argparse
import csv
import ctypes as C
import glob
import json
import math
import os
import shutil
import subprocess
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "graphgp.jl_amd"))

METRIC = "points/s for generate, grad_xi, grad_vals at 1M pts k=8 fp32; % of roofline"
HBM_PEAK = 8.0e12
PEAK = {"f32": 157.3e12, "f64": 78.6e12}   # dense MFMA / vector peaks, MI355X
CALIB_BYTES = 1 << 30                      # the counter calibration copy (above the 256 MB MALL)

CONFIGS = {
    1: dict(desc="10K points, D=2, standard normal (seed 99), n0=100, k=10, RBF var 1 scale 0.3, "
                 "1000 log bins [1e-4,10], jitter 1e-5, f64",
            N=10_000, D=2, n0=100, k=10, dtype="f64", points="normal",
            table=("rbf", 1.0, 0.3, 1e-4, 10.0, 1000, 1e-5),
            ops=["generate", "generate_inv", "generate_logdet"], cpu=True),
    2: dict(desc="1M points uniform in [0,1)^3, n0=1000, k=8, RBF var 1 scale 0.05, 1000 log bins "
                 "[1e-4,2], jitter 1e-5, f32; step = generate + generate_grad_xi + "
                 "generate_grad_vals",
            N=1_000_000, D=3, n0=1000, k=8, dtype="f32", points="uniform",
            table=("rbf", 1.0, 0.05, 1e-4, 2.0, 1000, 1e-5),
            ops=["generate", "grad_xi", "grad_vals"], cpu=True),
    3: dict(desc="10M points, 256 Gaussian clusters (sigma 0.01) + 20% uniform in [0,1)^3, "
                 "n0=4096, k=16, Matern-3/2 var 2 scale 0.02, 2000 log bins [1e-4,2], f32",
            N=10_000_000, D=3, n0=4096, k=16, dtype="f32", points="clustered",
            table=("matern", 1, 2.0, 0.02, 1e-4, 2.0, 2000, 1e-5),
            ops=["generate", "generate_inv", "refine_logdet_grad_vals"], cpu=False),
    4: dict(desc="1M points uniform in [0,1)^3, n0=1000, k=30, Matern-5/2 var 1 scale 0.05, "
                 "1000 log bins [1e-4,2], jitter 1e-6, f64; generate_logdet with its d/dvals "
                 "and hyperparam_grad on (variance, scale)",
            N=1_000_000, D=3, n0=1000, k=30, dtype="f64", points="uniform",
            table=("matern", 2, 1.0, 0.05, 1e-4, 2.0, 1000, 1e-6),
            ops=["logdet_grad_hyper"], cpu=False),
    5: dict(desc="200M points, x,y uniform in [0,1), z uniform in [0,0.1), n0=16384, k=8, "
                 "anisotropic 256x64 grid exp(-ds/0.05) exp(-(dz/0.01)^2/2), f32",
            N=200_000_000, D=3, n0=16384, k=8, dtype="f32", points="slab",
            table=("aniso",), ops=["generate", "grad_xi"], cpu=False),
}

# Timer name (ggp_kernel_timers) -> kernel name prefix in profiles.
KERNELS = {"factor": "k_factor", "pullback": "k_pullback", "sweep_fwd": "k_sweep_fwd",
           "sweep_rev": "k_sweep_rev", "potrf": "k_potrf_walk"}
TIMER_BITS = {"factor": 1, "pullback": 2, "sweep_fwd": 4, "sweep_rev": 8, "dense": 16, "op": 32,
              "potrf": 64}


def log(msg):
    print(msg, file=sys.stderr, flush=True)


# ---- workloads --------------------------------------------------------------------------------
def make_points(cfg, N, seed=20261201):
    D = cfg["D"]
    if cfg["points"] == "normal":
        return np.random.default_rng(99).standard_normal((N, D))
    rng = np.random.default_rng(seed)
    if cfg["points"] == "uniform":
        return rng.random((N, D))
    if cfg["points"] == "clustered":
        cent = rng.random((256, D))
        pick = rng.integers(0, 256, N)
        pts = cent[pick] + 0.01 * rng.standard_normal((N, D))
        uni = rng.random(N) < 0.2
        pts[uni] = rng.random((int(uni.sum()), D))
        return pts
    if cfg["points"] == "slab":
        pts = rng.random((N, D))
        pts[:, 2] *= 0.1
        return pts
    raise ValueError(cfg["points"])


def make_table(cfg):
    import graphgp_hip as G
    t = cfg["table"]
    if t[0] == "rbf":
        return G.rbf_kernel(t[1], t[2], t[3], t[4], t[5], jitter=t[6])
    if t[0] == "matern":
        return G.matern_kernel(t[1], t[2], t[3], t[4], t[5], t[6], jitter=t[7])
    return G.rbf_kernel(1.0, 0.05, 1e-4, 2.0, 200)  # placeholder axes of the anisotropic problem


def aniso_cov(dt):
    import graphgp_hip as G
    sb = np.linspace(0.0, 1.5, 256)
    zb = np.linspace(0.0, 0.1, 64)
    grid = np.exp(-sb[:, None] / 0.05) * np.exp(-0.5 * (zb[None, :] / 0.01) ** 2)
    return G.build_anisotropic_covariance(sb, zb, grid, 1.0, jitter=1e-4, dtype=dt)


def workload(cfg, N):
    import graphgp_hip as G
    dt = np.float32 if cfg["dtype"] == "f32" else np.float64
    pts = make_points(cfg, N)
    bins, vals = make_table(cfg)
    t = time.perf_counter()
    prob = G.build_graph(pts, cfg["n0"], cfg["k"], bins.astype(dt), vals.astype(dt),
                         backend="hip")
    del pts
    log(f"graph built on the GPU in {time.perf_counter() - t:.2f}s: N={N} n0={prob.n0} "
        f"levels={len(prob.offsets) - 1}")
    if cfg["table"][0] == "aniso":
        prob = G.GraphGPProblem(prob.coords, prob.neighbors, prob.offsets, prob.n0, prob.scale,
                                indices=prob.indices, cov=aniso_cov(dt))
    xi = np.random.default_rng(7).standard_normal(N).astype(dt)
    vb = np.random.default_rng(8).standard_normal(N).astype(dt)
    return prob, xi, vb


def op_table(cfg, hp, xi, vb):
    import graphgp_hip as G
    t = cfg["table"]

    def hyper():
        ld, g = G.generate_logdet_and_grad_vals(hp)
        G.hyperparam_grad(g, lambda var, cut: G.matern_kernel(t[1], var, cut, t[4], t[5], t[6],
                                                               jitter=t[7]), [t[2], t[3]])
        return ld

    return {
        "generate": lambda: G.generate(hp, xi),
        "grad_xi": lambda: G.generate_grad_xi(hp, vb),
        "grad_vals": lambda: G.generate_grad_vals(hp, xi, vb),
        "generate_inv": lambda: G.generate_inv(hp, xi),
        "generate_logdet": lambda: G.generate_logdet(hp),
        "refine_logdet_grad_vals": lambda: G.refine_logdet_grad_vals(hp, as_numpy=False),
        "logdet_grad_hyper": hyper,
    }


# ---- algorithmic cost (bytes and flops per refined point) --------------------------------------
def per_point_cost(k, D, es):
    """Counting convention: gathered bytes with no reuse credit (int32 neighbours, uint32
    lattice coordinates, values of the element size es), flops with FMA = 2 and div/sqrt = 1.
    n = k+1, P = n(n-1)/2. The factorization (assembly, Cholesky, mean_vec back-solve) costs
    F_fac = 8P + (n^3-n)/3 + P + n + k(k-1) + k flops; one pass over the point reads
    B_pt = es(2k + D + kD + 2) bytes (neighbours, coordinates, the field values it gathers and
    its own input and output), plus 24 bytes of permutation gathers per op."""
    n = k + 1
    P = n * (n - 1) // 2
    f_fac = 8 * P + (n ** 3 - n) // 3 + P + n + k * (k - 1) + k
    b_pt = es * (2 * k + D + k * D + 2)
    f_pull = 4 * (n ** 3 - n) // 6 + 2 * n + 3 * P + 8 * P + 2 * k * k  # pullback pass
    return {
        "generate": (b_pt + 24, f_fac + 2 * k + 1),
        "generate_inv": (b_pt + 24, f_fac + 2 * k + 1),
        "grad_xi": (b_pt + 4 * k + 24, f_fac + 2 * k + 1),
        "grad_vals": (3 * b_pt + 4 * k + 24, 2 * (f_fac + 2 * k + 1) + f_pull + f_fac),
        "generate_logdet": (b_pt - es * k + 8, f_fac),
        "refine_logdet_grad_vals": (b_pt - es * k, f_fac + f_pull),
        "logdet_grad_hyper": (b_pt - es * k, f_fac + f_pull),
    }


def kernel_cost(name, k, D, es, n0, M, N):
    """(bytes, flops) per launch of each timed kernel, by the same convention."""
    n = k + 1
    P = n * (n - 1) // 2
    f_fac = 8 * P + (n ** 3 - n) // 3 + P + n + k * (k - 1) + k
    if name == "factor":      # nbr + joint coords in, mean_vec + std out
        return (4 * k + 4 * D * (k + 1) + es * (k + 1)) * M, f_fac * M
    if name == "pullback":    # nbr + coords + v gathers + vb + xi in
        return (4 * k + 4 * D * (k + 1) + es * (k + 2)) * M, (f_fac + 4 * (n ** 3 - n) // 6) * M
    if name == "sweep_fwd":   # nbr, mean_vec, std, xi, gathered v, two stores per point
        return (4 * k + es * (2 * k + 4)) * M, (2 * k + 1) * M
    if name == "sweep_rev":   # per list entry: entry, weight, consumer value; per point 3 words
        return (4 + 2 * es) * k * M + 3 * es * N, 2 * k * M
    if name == "potrf":       # the n0 x n0 Cholesky
        return 3 * es * n0 * n0, n0 ** 3 // 3
    raise KeyError(name)


# ---- counters ---------------------------------------------------------------------------------
def child_pmc(args, cfg):
    """Run under rocprofv3 --pmc by measure_traffic: the 1 GiB calibration copy, then one pass of
    every op of the configuration."""
    import torch
    import graphgp_hip as G
    src = torch.ones(CALIB_BYTES // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    prob, xi_np, vb_np = workload(cfg, args.n or cfg["N"])
    hp = G.to_backend(prob)
    xi, vb = torch.from_numpy(xi_np).cuda(), torch.from_numpy(vb_np).cuda()
    fns = op_table(cfg, hp, xi, vb)
    for o in cfg["ops"]:
        fns[o]()
    torch.cuda.synchronize()


def measure_traffic(args):
    """Per-dispatch HBM bytes of every library kernel from two rocprofv3 --pmc passes of a
    child run (FETCH_SIZE, then WRITE_SIZE), scaled by the counters of the 1 GiB copy.
    Returns ({kernel name: (fetch bytes, write bytes)}, note)."""
    if not shutil.which("rocprofv3"):
        return None, "rocprofv3 not found"
    out = {}
    scale = {}
    tmp = tempfile.mkdtemp(prefix="ggp_pmc_")
    try:
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            d = os.path.join(tmp, counter)
            cmd = ["rocprofv3", "--pmc", counter, "--output-format", "csv", "-d", d, "-o", "pmc",
                   "--", sys.executable, os.path.abspath(__file__), "--child-pmc",
                   "--config", str(args.config)]
            if args.n:
                cmd += ["--n", str(args.n)]
            env = dict(os.environ, TMPDIR="/tmp")
            log(f"counter pass {counter} ...")
            r = subprocess.run(cmd, cwd="/tmp", env=env, capture_output=True, text=True,
                               timeout=600)
            files = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
            if not files:
                return None, f"{counter}: no counter output (rocprofv3 exit {r.returncode})"
            per = {}  # kernel name -> per-dispatch bytes (KiB counters)
            for f in files:
                for row in csv.DictReader(open(f)):
                    name = row.get("Kernel_Name", "")
                    per.setdefault(name, []).append(float(row.get("Counter_Value", 0.0)) * 1024.0)
            # the calibration copy is the largest device copy of the run (the harness's other
            # copies are host <-> device transfers of a few bytes to a few MB)
            calib = [v for n, vs in per.items() if "copyBuffer" in n for v in vs]
            if not calib:
                return None, f"{counter}: calibration copy not found"
            scale[counter] = CALIB_BYTES / max(calib)
            for n, vs in per.items():
                out.setdefault(n, [0.0, 0.0])[0 if counter == "FETCH_SIZE" else 1] = \
                    float(np.mean(vs)) * scale[counter]
    except (subprocess.TimeoutExpired, OSError) as e:
        return None, f"counter pass failed: {e}"
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    note = (f"counter scale factors from the 1 GiB copy: FETCH_SIZE x{scale['FETCH_SIZE']:.3f}, "
            f"WRITE_SIZE x{scale['WRITE_SIZE']:.3f}")
    return out, note


def traffic_of(traffic, prefix):
    if not traffic:
        return None
    rows = [v for n, v in traffic.items() if n.split("(")[0].split("::")[-1].startswith(prefix)
            or f"::{prefix}<" in n or n.startswith(prefix)]
    if not rows:
        return None
    return float(np.mean([f + w for f, w in rows]))


# ---- CPU baseline -------------------------------------------------------------------------------
def cpu_baseline(cfg, prob, xi, vb, nthreads):
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    dt = np.float32 if cfg["dtype"] == "f32" else np.float64
    ref = O.Problem(prob.coords, prob.neighbors, prob.offsets, prob.n0, prob.scale, prob.bins,
                    prob.vals, indices=prob.indices, dtype=dt, nthreads=nthreads)
    ops = {"generate": lambda: ref.generate(xi), "grad_xi": lambda: ref.generate_grad_xi(vb),
           "grad_vals": lambda: ref.generate_grad_vals(xi, vb),
           "generate_inv": lambda: ref.generate_inv(xi),
           "generate_logdet": lambda: ref.generate_logdet()}
    t = {}
    for name in cfg["ops"]:   # one warm-up, then the best of three (whole op each)
        f = ops[name]
        f()
        best = float("inf")
        for _ in range(3):
            s = time.perf_counter()
            f()
            best = min(best, time.perf_counter() - s)
        t[name] = best
    return t


# ---- main ---------------------------------------------------------------------------------------
def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=2, choices=sorted(CONFIGS))
    ap.add_argument("--n", type=int, default=0, help="override the number of points")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-traffic", action="store_true", help="skip the counter passes")
    ap.add_argument("--child-pmc", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args()
    cfg = CONFIGS[args.config]
    if args.child_pmc:
        child_pmc(args, cfg)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for {args.gpus}); the path's multi-GPU "
              "sharding is a design, not part of this build", file=sys.stderr)
        sys.exit(2)

    # The counter passes run first, as child processes, before this process touches the GPU.
    traffic, traffic_note = (None, "skipped (--no-traffic)")
    if not args.no_traffic:
        traffic, traffic_note = measure_traffic(args)
        log(f"traffic: {traffic_note}")

    import torch
    import graphgp_hip as G
    from graphgp_hip import _native as nat

    N = args.n or cfg["N"]
    k, D, n0 = cfg["k"], cfg["D"], cfg["n0"]
    es = 4 if cfg["dtype"] == "f32" else 8
    prob, xi_np, vb_np = workload(cfg, N)
    hp = G.to_backend(prob)
    xi = torch.from_numpy(xi_np).cuda()
    vb = torch.from_numpy(vb_np).cuda()
    ops = cfg["ops"]
    fns = op_table(cfg, hp, xi, vb)
    for _ in range(args.warmup):
        for o in ops:
            fns[o]()
    torch.cuda.synchronize()

    def timer(name):
        tot, cnt = C.c_double(), C.c_int64()
        nat.call("ggp_kernel_timer_read", hp.handle, name.encode(), C.byref(tot), C.byref(cnt))
        return tot.value, cnt.value

    # Pre-pass with every kernel timer on: the per-kernel breakdown and the dominant kernel.
    nat.call("ggp_kernel_timers", hp.handle, 127)
    kpass = 3
    for _ in range(kpass):
        for o in ops:
            fns[o]()
    torch.cuda.synchronize()
    M = prob.M
    kernels = {}
    for name in ("factor", "pullback", "sweep_fwd", "sweep_rev", "potrf", "dense"):
        tot, cnt = timer(name)
        if not cnt:
            continue
        kernels[name] = {"avg_ms": tot / cnt, "launches_per_step": cnt / kpass,
                         "ms_per_step": tot / kpass}
        if name in KERNELS:
            b, f = kernel_cost(name, k, D, es, n0, M, N)
            t = tot / cnt * 1e-3
            kernels[name].update({
                "kernel": KERNELS[name], "bytes_per_launch": b, "flops_per_launch": f,
                "hbm_frac": b / t / HBM_PEAK, "flop_frac": f / t / PEAK[cfg["dtype"]]})
    dominant = max((n for n in kernels if n in KERNELS), key=lambda n: kernels[n]["ms_per_step"])

    # Timed region: only the dominant kernel's timer is on (every event pair costs the op a few
    # microseconds).
    nat.call("ggp_kernel_timers", hp.handle, TIMER_BITS[dominant])
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
    tot, cnt = timer(dominant)
    nat.call("ggp_kernel_timers", hp.handle, 0)
    dom_ms = tot / cnt
    ms_step = total / args.steps * 1e3

    b, f = kernel_cost(dominant, k, D, es, n0, M, N)
    hbm_frac = b / (dom_ms * 1e-3) / HBM_PEAK
    flop_frac = f / (dom_ms * 1e-3) / PEAK[cfg["dtype"]]
    if flop_frac > hbm_frac:
        roofline = {"bound": "mfma", "achieved": f / (dom_ms * 1e-3) / 1e12,
                    "peak": PEAK[cfg["dtype"]] / 1e12, "unit": "TFLOP/s", "frac": flop_frac}
    else:
        roofline = {"bound": "hbm", "achieved": b / (dom_ms * 1e-3) / 1e9,
                    "peak": HBM_PEAK / 1e9, "unit": "GB/s", "frac": hbm_frac}
    tr = traffic_of(traffic, KERNELS[dominant])
    roofline.update({"traffic": tr, "traffic_unit": "bytes per launch", "traffic_note": traffic_note,
                     "kernel": KERNELS[dominant], "avg_launch_ms": dom_ms,
                     "algorithmic_bytes_per_launch": b, "algorithmic_flops_per_launch": f,
                     "launches_timed": cnt})
    for name, v in kernels.items():
        if name in KERNELS:
            v["traffic_bytes_per_launch"] = traffic_of(traffic, KERNELS[name])

    cost = per_point_cost(k, D, es)
    per_op = {}
    for o in ops:
        t = per[o] / args.steps
        per_op[o] = {"ms": t * 1e3, "points_per_s": N / t}
        if o in cost:
            bo, fo = cost[o]
            per_op[o].update({"bytes_per_point": bo, "flops_per_point": fo,
                              "roofline_frac": max(bo * M / t / HBM_PEAK,
                                                   fo * M / t / PEAK[cfg["dtype"]])})
    step_bytes = sum(cost[o][0] for o in ops if o in cost) * M
    line = {
        "metric": METRIC if args.config == 2 and N == cfg["N"] else
        f"points/s for {', '.join(ops)} ({cfg['desc'].split(';')[0]})",
        "value": N / (total / args.steps), "unit": "points/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": cfg["dtype"],
        "data": "synthetic (seeded points, N(0,1) xi and cotangent)",
        "config": {"workload": cfg["desc"], "N": N, "n0": prob.n0, "k": k, "D": D,
                   "levels": len(prob.offsets) - 1, "config_id": args.config},
        "per_op": per_op, "step_roofline_frac_hbm": step_bytes / (total / args.steps) / HBM_PEAK,
        "kernels": kernels, "roofline": roofline,
    }
    if cfg["cpu"] and not args.no_cpu:
        # the host's CPU share: OMP_NUM_THREADS when the environment sets it, else the affinity
        nthreads = int(os.environ.get("OMP_NUM_THREADS") or
                       (len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity")
                        else os.cpu_count()))
        log(f"cpu baseline on {nthreads} threads ...")
        t = cpu_baseline(cfg, prob, xi_np, vb_np, nthreads)
        tt = sum(t.values())
        line["cpu_baseline"] = {
            "value": N / tt, "unit": "points/s", "cores": nthreads, "kind": "port",
            "sample": f"the full {N}-point workload; each op timed whole, best of 3 after a "
                      "warm-up (the dense factor is the oracle's column-by-column Cholesky)",
            "per_op_s": t, "speedup": (N / (total / args.steps)) / (N / tt)}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
