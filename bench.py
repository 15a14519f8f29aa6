#!/usr/bin/env python3
"""All-points FRNN (grid build + neighbour search) on one MI355X.

    python bench.py [--steps K] [--warmup W] [--config metric|C1..C5|refD<D>N<N>] [--no-cpu]

A step is one FRNNEngine.search_gpu call (reference: frnn_engine.cu:195-250)
over the configuration's synthetic cloud, with the SoA input already resident
in HBM and the outputs left in HBM -- the timing the reference's harness uses
(Tests/scripts/benchmark_vs_libfrnn.py:146-169).  Prints ONE JSON line on stdout:

  value            mean ms per step over exactly K steps, each step one
                   synchronous call timed on its own (ms_per_step_wall: the
                   whole timed loop, which also holds the reads of the search
                   kernel's event times between steps)
  roofline         dominant kernel (the neighbour search), its mean HIP-event
                   duration on the engine's stream over the timed steps (the
                   only events recorded there):
                   grid paths: bound "hbm", the search's algorithmic bytes
                   8DN + 4(C+1) + 4N + 8KN (read the rows, the cell offsets and
                   the index map; write K keys per query; C = the plan's cells)
                   per launch / duration vs 8 TB/s;
                   brute force: bound "mfma", 2 * N * N * D flops / duration vs
                   the fp32 MFMA peak.  The other view is reported beside it
                   (mfma_view: 2*D flops per (query, candidate) pair streamed
                   through the MFMA filter, counted by the kernel; hbm_view).
                   traffic: HBM bytes per launch from the committed rocprofv3
                   PMC summary for this config, when present.
  build_hbm        grid-build kernels: algorithmic bytes / event time vs 8 TB/s
                   (events around every stage, in a profiled pass after the
                   timed region)
  refD<D>N<N>      a cell of the reference's own published K=16 sweep (A100
                   latency reported beside ours; frnn_workloads.REF_SWEEP)
  cpu_baseline     the C++/OpenMP restatement of the reference (oracle/: the
                   reference's own grid, i.e. its first-coordinate grid on the
                   raw coordinates for D > 4) on every host core this job may
                   use, on a bounded query sample timed on this host and scaled
                   to all N queries; the same sample is compared bit-exactly with
                   the GPU rows
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "pure_cuda-c-_frnn_amd"), os.path.join(ROOT, "oracle")]

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0
MFMA_F32_PEAK_TFLOPS = 157.3
METRIC = "ms per all-points FRNN (build+search) + HBM GB/s frac, D=16 N=1M K=64"


def eprint(*a):
    print(*a, file=sys.stderr, flush=True)


def build_bytes(N, D, ds, g, C, framed, zero_filled):
    """Algorithmic HBM bytes of each build kernel (4-byte ints and floats); ds is
    the padded row length of the AoS rows the reorder writes, C the grid's cells
    (a frame's actual cells), zero_filled the count entries the build filled
    (0 once a previous call's count scan has left the array zero)."""
    T = min(D, 32)
    b = {
        "zero_fill": 4 * zero_filled,
        "stats": 4 * D * N,
        "bin_count": 4 * (T if framed else g) * N + 8 * N + 8 * (C + 1),
        # read the counts, write the offsets, zero the counts
        "scan": 12 * (C + 1),
        "reorder": 20 * N + 4 * D * N + (8 if ds >= 64 else 4) * ds * N,
    }
    if framed:
        # frame: covariance sample over the T projection terms (512 tiles of 256
        # points)
        b["frame"] = 4 * T * min(N, 512 * 256)
    return b


def traffic_from_profiles(config):
    path = os.path.join(ROOT, "profiles", f"search_pmc_{config}.json")
    if not os.path.exists(path):
        return None, None
    with open(path) as f:
        p = json.load(f)
    return p.get("hbm_bytes_per_dispatch"), os.path.relpath(path, ROOT)


def cpu_baseline(w, gi, gd, target_s, threads):
    import frnn_oracle as O
    rs = np.random.RandomState(99)
    # calibration run on a small sample, then one run sized to ~target_s of search work
    q0 = min(w.N, 1000)
    t = []
    O.search(w.X, w.K, w.radius, nthreads=threads,
             query_ids=np.sort(rs.choice(w.N, q0, replace=False)).astype(np.int32), timings=t)
    per_q = max(t[1] / q0, 1e-9)
    nq = int(min(w.N, max(q0, target_s / per_q)))
    q = np.sort(rs.choice(w.N, nq, replace=False)).astype(np.int32)
    t = []
    ri, rd = O.search(w.X, w.K, w.radius, nthreads=threads, query_ids=q, timings=t)
    build_s, search_s = t
    full_ms = 1e3 * (build_s + search_s * w.N / nq)
    same = np.all(gi[q] == ri, 1) & np.all(gd[q].view(np.uint32) == rd.view(np.uint32), 1)
    return {
        "value": round(full_ms, 3), "unit": "ms", "cores": threads, "kind": "port",
        "algorithm": "the reference's (oracle/frnn_oracle.cpp): its grid on the raw coordinates (for D > 4 the "
                     "first-coordinate grid, g = 4), the full 3^g cell shell per query, sequential-fma distances",
        "sample": f"{nq} of {w.N} queries (random, seed 99) against the full database, with the "
                  f"full grid build; search time scaled by N/{nq}: build {build_s * 1e3:.1f} ms + "
                  f"search {search_s:.2f} s",
        "speedup_vs_gpu": None, "parity_sample_rows": nq,
        "parity_mismatched_rows": int(np.sum(~same)),
    }


def host_cores():
    """CPUs this process may run on (the job's share of the host)."""
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def bench_queries(args, w):
    """Separate queries against a reused grid: the config's points are built
    once (frnn_engine_build), then each timed step is one query() of M queries
    (points near random points of the set, offsets of norm ~0.3 r)."""
    import torch
    import frnn_cuda
    M = args.queries
    rs = np.random.RandomState(78)
    Q = (w.X[rs.randint(0, w.N, M)] + (0.3 * w.radius / np.sqrt(w.D)) * rs.standard_normal((M, w.D)))
    Q = np.ascontiguousarray(Q.astype(np.float32).T)
    dp = torch.from_numpy(w.soa()).to("cuda:0")
    dq = torch.from_numpy(Q).to("cuda:0")
    torch.cuda.synchronize()
    eng = frnn_cuda.FRNNEngine(max_points=max(w.N, M))
    builds = []
    for _ in range(max(args.warmup // 4, 2)):
        t0 = time.perf_counter()
        eng.build(dp.data_ptr(), w.N, w.D, w.K, w.radius)
        builds.append(time.perf_counter() - t0)
    for _ in range(args.warmup):
        eng.query(dq.data_ptr(), M)
    torch.cuda.synchronize()
    times = []
    for _ in range(args.steps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        eng.query(dq.data_ptr(), M)
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    ms = 1e3 * float(np.mean(times))
    # one profiled query() with the plain kernel for the stage times, then one
    # with the counting build for the work counters
    eng.set_profiling(True, counters=False)
    eng.query(dq.data_ptr(), M)
    st = eng.stage_times()
    eng.set_profiling(True, counters=True)
    eng.query(dq.data_ptr(), M)
    ct = eng.counters()
    plan = eng.last_plan()
    eng.close()
    print(json.dumps({
        "metric": f"ms per query() call of {M} separate queries against a reused grid",
        "value": round(ms, 4), "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_median": round(1e3 * float(np.median(times)), 4), "higher_is_better": False,
        "queries_per_s": round(M / (ms / 1e3), 1), "build_ms_median": round(1e3 * float(np.median(builds)), 4),
        "dtype": "f32", "data": "synthetic (the config's points; queries near random points of the set)",
        "config": {"workload": w.name, "N": w.N, "M": M, "D": w.D, "K": w.K, "radius": w.radius,
                   "path": plan["path"]},
        "search_kernel_ms": round(st["search"], 4),
        "query_build_ms": round(st["reorder"], 4),
        "counters": {k: int(v) for k, v in ct.items()},
    }))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="metric")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run three 256 MiB device copies (calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--queries", type=int, default=0,
                    help="instead of the all-points search: build the config's grid once and time "
                         "query() calls of this many separate queries against it")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        eprint(f"bench.py: --gpus {args.gpus} (WORLD_SIZE={world}) requested, but this engine runs on "
               f"one GPU only; there is no multi-GPU path to measure. Run with --gpus 1.")
        sys.exit(2)

    import torch
    import frnn_cuda
    import frnn_workloads as W

    if args.copy_probe:
        n = 256 * 1024 * 1024 // 4
        a = torch.ones(n, device="cuda:0")
        b = torch.empty_like(a)
        torch.cuda.synchronize()
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        eprint(f"[bench] copy probe: 3 copies of {n * 4} bytes")
        return

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    t_gen = time.perf_counter()
    w = W.config(args.config)
    if args.queries > 0:
        bench_queries(args, w)
        return
    eprint(f"[bench] {w.name}: N={w.N} D={w.D} K={w.K} r={w.radius:.6f} "
           f"(data {time.perf_counter() - t_gen:.1f}s)")
    plan = frnn_cuda.plan(w.N, w.D, w.K, w.radius)
    d = torch.from_numpy(w.soa()).to("cuda:0")
    torch.cuda.synchronize()
    eng = frnn_cuda.FRNNEngine(max_points=w.N)
    ptr = d.data_ptr()
    for _ in range(args.warmup):
        eng.search_gpu(ptr, w.N, w.D, w.K, w.radius)
    eprint(f"[bench] warmup done ({args.warmup} steps), path={plan['path']}")

    # Timed region: each step is one synchronous search_gpu() call, timed on
    # its own; HIP events around the search kernel only (the dominant kernel's
    # duration for the roofline) are read between steps.  Events around every
    # stage cost ~0.03-0.04 ms per call, so the per-stage breakdown comes from
    # a separate profiled pass after the timed region, and the counting build
    # of the search from one more call after that.
    eng.set_profiling(True, counters=False, search_only=True)
    steps_ms, search_ms = [], []
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        s0 = time.perf_counter()
        eng.search_gpu(ptr, w.N, w.D, w.K, w.radius)   # synchronous
        steps_ms.append((time.perf_counter() - s0) * 1e3)
        search_ms.append(eng.stage_times()["search"])
    torch.cuda.synchronize()
    total_s = time.perf_counter() - t0
    ms_per_step = float(np.sum(steps_ms)) / args.steps
    eng.set_profiling(True, counters=False)
    stage_sum = {}
    n_prof = min(args.steps, 5)
    for _ in range(n_prof):
        eng.search_gpu(ptr, w.N, w.D, w.K, w.radius)
        for k, v in eng.stage_times().items():
            stage_sum[k] = stage_sum.get(k, 0.0) + v
    cwork = eng.count_work()
    eng.set_profiling(True, counters=True)
    eng.search_gpu(ptr, w.N, w.D, w.K, w.radius)
    ctr = eng.counters()
    eng.set_profiling(False)
    stages = {k: v / n_prof for k, v in stage_sum.items()}
    stages["search"] = float(np.mean(search_ms))   # the timed region's
    eprint(f"[bench] {args.steps} steps: {ms_per_step:.3f} ms/step; stages " +
           ", ".join(f"{k}={v:.3f}" for k, v in stages.items()))

    idx, dist = eng.get_results_numpy(w.N, w.K)
    gi = idx.reshape(w.K, w.N).T
    gd = dist.reshape(w.K, w.N).T

    # dominant kernel (the search): algorithmic work per launch / its mean
    # HIP-event duration.  Grid paths are priced on HBM bytes, brute force on
    # fp32 MFMA flops; the other view is reported beside it.
    search_s = stages["search"] / 1e3
    pairs = ctr["streamed_pairs"]
    filt_flops = 2.0 * w.D * pairs
    filt_tf = filt_flops / search_s / 1e12
    mfma_view = {"flops_per_launch": filt_flops, "filtered_pairs": pairs,
                 "TFLOPs": round(filt_tf, 3), "frac": round(filt_tf / MFMA_F32_PEAK_TFLOPS, 4),
                 "unit_of_work": "2*D flops per (query, candidate) pair streamed through the MFMA filter"}
    traffic, traffic_src = traffic_from_profiles(args.config)
    C = plan["cells"] if plan["path"] != "bruteforce" else 0
    alg_bytes = 8 * w.D * w.N + 4 * (C + 1) + 4 * w.N + 8 * w.K * w.N
    alg_gbs = alg_bytes / search_s / 1e9
    hbm_view = {"algorithmic_bytes": alg_bytes, "GBps": round(alg_gbs, 1),
                "frac": round(alg_gbs / HBM_PEAK_GBS, 5),
                "bytes_formula": "8DN + 4(C+1) + 4N + 8KN, C = the plan's cells"}
    if plan["path"] == "bruteforce":
        bf_flops = 2.0 * w.N * w.N * w.D
        tf = bf_flops / search_s / 1e12
        roofline = {"kernel": "search_kernel (tiled brute force, fp32 MFMA distance filter)", "bound": "mfma",
                    "achieved": round(tf, 3), "peak": MFMA_F32_PEAK_TFLOPS, "unit": "TFLOP/s",
                    "frac": round(tf / MFMA_F32_PEAK_TFLOPS, 4), "traffic": traffic,
                    "flops_per_launch": bf_flops, "mean_kernel_ms": round(stages["search"], 4),
                    "traffic_source": traffic_src, "hbm_view": hbm_view}
    else:
        roofline = {"kernel": "search_kernel (neighbour search)", "bound": "hbm",
                    "achieved": round(alg_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(alg_gbs / HBM_PEAK_GBS, 5), "traffic": traffic,
                    "algorithmic_bytes": alg_bytes, "mean_kernel_ms": round(stages["search"], 4),
                    "traffic_source": traffic_src, "mfma_view": mfma_view,
                    "shell_candidate_pairs": ctr["shell_candidates"]}

    if plan["path"] != "bruteforce":
        bb = build_bytes(w.N, w.D, frnn_cuda.aos_stride(w.D), plan["grid_dim"], cwork["scanned"] - 1,
                         frnn_cuda.frame_workspace_bytes(w.N, w.D, w.K, w.radius) > 0, cwork["zero_filled"])
    else:
        ds = frnn_cuda.aos_stride(w.D)
        bb = {"stats": 4 * w.D * w.N, "reorder": 4 * w.D * w.N + (8 if ds >= 64 else 4) * ds * w.N}
    build = {}
    tot_b, tot_ms = 0, 0.0
    for k, b in bb.items():
        ms = stages[k]
        if b == 0:
            continue    # a stage with no work this call (the count fill after the first)
        gbs = b / (ms / 1e3) / 1e9 if ms > 0 else 0.0
        build[k] = {"bytes": b, "ms": round(ms, 4), "GBps": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
        tot_b += b
        tot_ms += ms
    if tot_ms > 0:
        g = tot_b / (tot_ms / 1e3) / 1e9
        build["total"] = {"bytes": tot_b, "ms": round(tot_ms, 4), "GBps": round(g, 1),
                          "frac": round(g / HBM_PEAK_GBS, 4)}
    end_to_end_bytes = tot_b + 8 * w.D * w.N + 16 * w.K * w.N
    e2e_gbs = end_to_end_bytes / (ms_per_step / 1e3) / 1e9

    cpu = None
    if not args.no_cpu:
        threads = host_cores()
        eprint(f"[bench] cpu baseline with {threads} threads (~{args.cpu_seconds:.0f}s sample)")
        cpu = cpu_baseline(w, gi, gd, args.cpu_seconds, threads)
        cpu["speedup_vs_gpu"] = round(cpu["value"] / ms_per_step, 1)
        eprint(f"[bench] cpu {cpu['value']:.1f} ms (x{cpu['speedup_vs_gpu']}), parity mismatched rows "
               f"{cpu['parity_mismatched_rows']}/{cpu['parity_sample_rows']}")

    line = {
        "metric": METRIC, "value": round(ms_per_step, 4), "unit": "ms", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4),
        "ms_median": round(float(np.median(steps_ms)), 4),
        "ms_per_step_wall": round(total_s * 1e3 / args.steps, 4), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (numpy RandomState 1234, recipe in frnn_workloads.py)",
        "config": {"workload": w.name, "N": w.N, "D": w.D, "K": w.K, "radius": w.radius,
                   "raw_radius": w.notes.get("raw_radius"), "path": plan["path"],
                   "grid_dim": plan["grid_dim"], "res": plan["res"], "cells": plan["cells"],
                   "queries_per_s": round(w.N / (ms_per_step / 1e3), 1),
                   **({"reference_a100_ms": round(w.notes["a100_ms"], 4),
                       "speedup_vs_reference_a100": round(w.notes["a100_ms"] / ms_per_step, 2)}
                      if "a100_ms" in w.notes else {})},
        "roofline": roofline,
        "build_hbm": build,
        "end_to_end_hbm": {"bytes": end_to_end_bytes, "GBps": round(e2e_gbs, 1),
                           "frac": round(e2e_gbs / HBM_PEAK_GBS, 5)},
        "stages_ms": {k: round(v, 4) for k, v in stages.items()},
        "counters": ctr,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    eng.close()


if __name__ == "__main__":
    main()
