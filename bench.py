"""Benchmark of the MI355X CWLB-SpMM mean aggregation on one GPU.

Workload: the skewed R-MAT configuration (N = 2^22 nodes, 2^26 R-MAT samples
a=.57 b=c=.19 d=.05 relabelled and deduplicated, unit edge values, K = 128
FP32 features in U[-1,1)), degree-reordered and cost-weighted partitioned
with the committed gfx950 cost coefficients; S is chosen among the three
wave-based candidates as the reference's --candidates mode does.

A step is one SpMM call (split-row clearing + aggregation kernel) over the
whole graph with all inputs resident in HBM.  W warm-up steps, then K timed
steps between synchronisations, timed with HIP events on the launch stream.

Prints one JSON line: GFLOP/s (2 nnz K / t) as `value`, the aggregation
kernel's roofline (algorithmic bytes per launch / mean event-timed kernel
duration vs 8 TB/s) and the CPU baseline (the reference kernel's semantics
restated with OpenMP, on this host's cores, over a sample of the tasks).
"""
import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "cwlb-spmm_amd"))

METRIC = "SpMM GFLOP/s (2·nnz·K/t) + achieved HBM GB/s vs peak, FP32 mean agg"
HBM_PEAK_GBS = 8000.0
COST_FILE = os.path.join(ROOT, "cwlb-spmm_amd", "resources", "spmm_costs_gfx950.txt")
GOLDEN = os.path.join(ROOT, "tests", "golden", "partition_golden.json")
# Committed rocprofv3 PMC summaries per workload configuration (traffic per
# aggregation launch, FETCH_SIZE + WRITE_SIZE scaled by a known-size copy).
PMC_SUMMARY = {
    4: os.path.join(ROOT, "profiles", "spmm_mean_runs_rmat22_k128_pmc.txt"),
    5: os.path.join(ROOT, "profiles", "spmm_mean_runs_mesh16m_k32_trace_pmc.md"),
    3: os.path.join(ROOT, "profiles", "spmm_mean_runs_sbm240k_k600_trace_pmc.md"),
    2: os.path.join(ROOT, "profiles", "spmm_mean_runs_chunglu1m_k64_trace_pmc.md"),
}


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def measured_traffic(cfg, S):
    """HBM bytes per aggregation launch from the committed rocprofv3 PMC
    summary: the figure measured at segment size S
    ("traffic_bytes_per_launch[S=63]: ..."), or None when the summary has no
    figure for this S."""
    try:
        text = open(PMC_SUMMARY[cfg]).read()
    except (KeyError, OSError):
        return None
    found = dict(re.findall(r"traffic_bytes_per_launch(?:\[S=(\d+)\])?:\s*([0-9.eE+]+)", text))
    value = found.get(str(S))
    return float(value) if value is not None else None


def reference_partition_match(cfg, S, costs, tasks):
    """Whether the task list equals, by SHA-256, the one the reference's own
    costWeightedTaskPartitioning produced for this graph, S and cost vector
    (tests/golden/partition_golden.json); None when the fixture has no such
    case."""
    import hashlib

    import numpy as np
    try:
        golden = json.load(open(GOLDEN))
    except OSError:
        return None
    rec = golden["full"].get(str(cfg))
    if rec is None:
        return None
    for p in rec["partitions"]:
        if p["S"] == S and golden["costs"][p["costs"]] == list(costs):
            digest = hashlib.sha256(np.ascontiguousarray(tasks).astype("<i4").tobytes())
            return digest.hexdigest() == p["tasks_sha256"]
    return None


def segment_size_sweep(ctx, call, tune, dev, tasks_for, cfg, costs, S, trials):
    """Aggregation kernel time at segment size S: mean of `trials`
    event-timed launches with the automatic schedule, then with the schedule
    cwlb_ctx_tune_schedule keeps for this S (outside the timed launches)."""
    import numpy as np
    tk = tasks_for(S)
    d_t = dev(tk.reshape(-1))
    ctx.set_schedule(0, 0)
    ctx.set_locality(0, 0)
    ctx.set_cache_hints(0)
    ctx.set_occupancy(0)
    for _ in range(3):
        call(d_t, len(tk), False)
    auto_us = float(np.mean([call(d_t, len(tk), True).main_us for _ in range(trials)]))
    m, sl, (order, xcd) = tune(d_t, len(tk))
    for _ in range(3):
        call(d_t, len(tk), False)
    tuned_us = float(np.mean([call(d_t, len(tk), True).main_us for _ in range(trials)]))
    return {"S": S, "tasks": int(len(tk)), "automatic_us": round(auto_us, 1),
            "tuned_us": round(tuned_us, 1),
            "schedule": {"tasks_per_wave": m, "feature_slices": sl, "run_order": order,
                         "xcd_blocks": xcd, "hot_bytes": ctx.cache_hints(),
                         "occupancy": ctx.occupancy()},
            "tasks_match_reference_fixture": reference_partition_match(cfg, S, costs, tk)}


def preprocessing_times(ctx, g, rp, costs, S, tasks, reorder_host_ms):
    """Wall times (ms) of the degree reordering and the partition at S, on
    the host and on the GPU (outside the timed region; results checked
    equal)."""
    import numpy as np
    import torch

    from cwlb_amd import capi

    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    n, nnz = g.n, g.nnz
    d_rp0, d_ci0, d_v0 = dev(g.row_ptr), dev(g.col_idx), dev(g.val)
    outs = [torch.empty(n, dtype=torch.int32, device="cuda"),
            torch.empty(n + 1, dtype=torch.int32, device="cuda"),
            torch.empty(max(nnz, 1), dtype=torch.int32, device="cuda"),
            torch.empty(max(nnz, 1), dtype=torch.float32, device="cuda")]
    ctx.reorder_device(n, nnz, d_rp0, d_ci0, d_v0, *outs)  # warm-up
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ctx.reorder_device(n, nnz, d_rp0, d_ci0, d_v0, *outs)
    reorder_dev_ms = (time.perf_counter() - t0) * 1e3
    same_rp = bool(np.array_equal(outs[1].cpu().numpy(), rp))
    del d_ci0, d_v0, outs
    cap = capi.capacity_from_s(S, costs)
    t0 = time.perf_counter()
    host_tasks = capi.partition(rp, costs, cap)
    part_host_ms = (time.perf_counter() - t0) * 1e3
    d_rp = dev(rp)
    out = torch.empty((len(host_tasks), 4), dtype=torch.int32, device="cuda")
    try:
        ctx.partition_device(d_rp, n, costs, cap, out, len(host_tasks))  # warm-up
        t0 = time.perf_counter()
        ctx.partition_device(d_rp, n, costs, cap, out, len(host_tasks))
        part_dev_ms = round((time.perf_counter() - t0) * 1e3, 2)
        same_tasks = bool(np.array_equal(out.cpu().numpy(), host_tasks))
    except capi.CwlbError as e:
        part_dev_ms, same_tasks = str(e), None
    return {"reorder_host_ms": round(reorder_host_ms, 1), "reorder_device_ms": round(reorder_dev_ms, 2),
            "reorder_identical": same_rp, "partition_host_ms": round(part_host_ms, 1),
            "partition_device_ms": part_dev_ms, "partition_identical": same_tasks,
            "tasks_identical_to_bench_tasks": bool(np.array_equal(host_tasks, tasks))}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cfg", type=int, default=4, help="workload configuration (default: R-MAT)")
    ap.add_argument("--s", type=int, default=0, help="fixed segment size (0 = best candidate)")
    ap.add_argument("--k", type=int, default=0,
                    help="feature width instead of the workload's (above the device's maximum "
                         "work-group size the large-K entry runs, as the reference's driver "
                         "picks spmmKernelLargeKFallback)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--tasks-per-wave", type=int, default=0,
                    help="fixed launch schedule (with --slices) instead of tuning")
    ap.add_argument("--slices", type=int, default=0)
    ap.add_argument("--occupancy", type=int, default=0, choices=(0, 6),
                    help="fixed schedule: 6 = the 6-waves-per-SIMD kernel variant")
    ap.add_argument("--run-order", type=int, default=0,
                    help="fixed run order (cwlb_ctx_set_locality: 1 task order, 2 by output row)")
    ap.add_argument("--xcd-blocks", type=int, default=0,
                    help="fixed XCD placement (1 interleaved, 2 contiguous)")
    ap.add_argument("--s-sweep", default=None,
                    help="comma-separated segment sizes timed after the measured step, each "
                         "with the automatic and the tuned schedule (default: 32,64,128,256,512 "
                         "for the mesh workload, none otherwise; 'none' for none)")
    ap.add_argument("--hot-mb", type=int, default=0,
                    help="fixed cache hints: hot set of this many MB of feature rows "
                         "(cwlb_ctx_set_cache_hints; with --tasks-per-wave etc.)")
    ap.add_argument("--no-tune", action="store_true",
                    help="keep the automatic launch schedule (no cwlb_ctx_tune_schedule)")
    ap.add_argument("--no-host-call", action="store_true",
                    help="skip the one host-pointer call (inputs copied in, C copied out)")
    ap.add_argument("--costs", default=COST_FILE, help="cost file (four coefficients)")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="also run one device-to-device copy of this many MiB (a known-size "
                         "reference for the HBM traffic counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(the multi-GPU sharding is a design note, not a build target)", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import oracle
    from cwlb_amd import capi, synth, workloads

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    cfg = args.cfg
    K = args.k or workloads.FEATURE_DIM[cfg]
    workload = workloads.NAMES[cfg] if not args.k else f"{workloads.NAMES[cfg].rsplit('_k', 1)[0]}_k{K}"
    t0 = time.time()
    g = workloads.graph(cfg)
    log(f"graph {workloads.NAMES[cfg]}: n={g.n} nnz={g.nnz} ({time.time() - t0:.1f}s)")
    t0 = time.perf_counter()
    origin, rp, ci, val = capi.reorder_by_degree(g.row_ptr, g.col_idx, g.val)
    reorder_host_ms = (time.perf_counter() - t0) * 1e3
    costs = capi.read_costs(args.costs)
    log(f"reordered on the host in {reorder_host_ms:.0f} ms; costs {costs}")

    stream = torch.cuda.current_stream()
    ctx = capi.Context(0, stream.cuda_stream)
    info = ctx.info()
    large_k = K > info.max_work_group_size
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    d_rp, d_ci, d_v, d_o = dev(rp), dev(ci), dev(val), dev(origin)
    H = torch.empty((g.n, K), dtype=torch.float32, device="cuda")
    ctx.fill_features(H, g.n, K, workloads.FEATURE_SEED)
    C = torch.empty((g.n, K), dtype=torch.float32, device="cuda")

    def tasks_for(S):
        cap = capi.capacity_from_s(S, costs)
        return capi.partition(rp, costs, cap)

    def call(d_t, n_t, timed):
        return ctx.spmm(d_rp, d_ci, d_v, d_o, g.n, g.nnz, H, g.n, K, d_t, n_t, C, timed=timed,
                        large_k=large_k)

    def tune(d_t, n_t):
        return ctx.tune_schedule(d_rp, d_ci, d_v, d_o, g.n, g.nnz, H, g.n, K, d_t, n_t, C,
                                 trials=3, locality=True)

    # S: the best of the three wave-based candidates (main.cpp:534-577), or fixed.
    # S: the best of the three wave-based candidates (main.cpp:534-577), or
    # fixed.  As in the drop-in driver's candidate search (run_single_s per
    # S), each S gets its launch schedule tuned once (cwlb_ctx_tune_schedule,
    # outside the timed region), and the S with the fastest tuned aggregation
    # is kept.  A fixed schedule (--tasks-per-wave etc.) or --no-tune ranks
    # the S by the automatic schedule instead.
    fixed = bool(args.tasks_per_wave or args.slices or args.run_order or args.xcd_blocks
                 or args.hot_mb or args.occupancy)
    tuning = not fixed and not args.no_tune
    cands = [args.s] if args.s else workloads.candidate_s(g.nnz, info.compute_units)
    best = None
    s_candidates = []
    t_tune = 0.0
    for S in cands:
        tk = tasks_for(S)
        d_t = dev(tk.reshape(-1))
        ctx.set_schedule(0, 0)
        ctx.set_locality(0, 0)
        ctx.set_cache_hints(0)
        ctx.set_occupancy(0)
        for _ in range(5):
            call(d_t, len(tk), False)
        us = float(np.mean([call(d_t, len(tk), True).total_us for _ in range(10)]))
        rec = {"S": S, "tasks": int(len(tk)), "automatic_us": round(us, 1)}
        rank = us
        if tuning:
            t0 = time.perf_counter()
            m, sl, (order, xcd) = tune(d_t, len(tk))
            t_tune += time.perf_counter() - t0
            rec["schedule"] = {"tasks_per_wave": m, "feature_slices": sl, "run_order": order,
                               "xcd_blocks": xcd, "hot_bytes": ctx.cache_hints(),
                               "occupancy": ctx.occupancy()}
            for _ in range(3):
                call(d_t, len(tk), False)
            rank = float(np.mean([call(d_t, len(tk), True).total_us for _ in range(10)]))
            rec["tuned_us"] = round(rank, 1)
        log(f"candidate S={S}: {rec}")
        s_candidates.append(rec)
        if best is None or rank < best[1]:
            best = (S, rank, tk, d_t, us, rec.get("schedule"))
    S, _, tasks, d_t, auto_us, tuned = best
    T = len(tasks)
    prep = preprocessing_times(ctx, g, rp, costs, S, tasks, reorder_host_ms)
    prep["tasks_match_reference_fixture"] = reference_partition_match(cfg, S, costs, tasks)
    log(f"preprocessing: {prep}")
    # Launch schedule for this graph and S (0, 0 = the automatic choice).
    schedule = {"tasks_per_wave": 0, "feature_slices": 0, "tuned": False,
                "automatic_schedule_us": round(float(auto_us), 1)}
    if fixed:
        ctx.set_schedule(args.tasks_per_wave, args.slices)
        ctx.set_locality(args.run_order, args.xcd_blocks)
        ctx.set_cache_hints(args.hot_mb << 20)
        ctx.set_occupancy(args.occupancy)
        schedule.update(tasks_per_wave=args.tasks_per_wave, feature_slices=args.slices,
                        run_order=args.run_order, xcd_blocks=args.xcd_blocks,
                        hot_bytes=args.hot_mb << 20, occupancy=args.occupancy)
        log(f"fixed schedule: {schedule}")
    elif tuning:
        ctx.set_schedule(tuned["tasks_per_wave"], tuned["feature_slices"])
        ctx.set_locality(tuned["run_order"], tuned["xcd_blocks"])
        ctx.set_cache_hints(tuned["hot_bytes"])
        ctx.set_occupancy(tuned["occupancy"])
        schedule.update(tuned, tuned=True, tuning_ms=round(t_tune * 1e3, 1))
        log(f"tuned schedule: {schedule}")
    else:
        ctx.set_schedule(0, 0)
        ctx.set_locality(0, 0)
        ctx.set_cache_hints(0)
        ctx.set_occupancy(0)

    # Timed region: W warm-ups, K steps, synchronised on both sides.
    for _ in range(args.warmup):
        call(d_t, T, False)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.steps):
        call(d_t, T, False)
    e1.record(stream)
    torch.cuda.synchronize()
    ms_per_step = e0.elapsed_time(e1) / args.steps
    # Per-kernel durations: the reference protocol (event-timed launches).
    times = [call(d_t, T, True) for _ in range(args.steps)]
    main_us = float(np.mean([t.main_us for t in times]))
    zero_us = float(np.mean([t.zero_us for t in times]))
    # The schedule those launches resolved to (automatic choices included).
    schedule["launched"] = ctx.last_launch()
    # The reference's structure (one task per wave, one atomic add per
    # partial segment), for comparison.
    pt = [ctx.spmm(d_rp, d_ci, d_v, d_o, g.n, g.nnz, H, g.n, K, d_t, T, C,
                   flags=capi.PER_TASK, large_k=large_k) for _ in range(10)]
    per_task_us = float(np.mean([t.total_us for t in pt]))
    log(f"S={S} T={T} ms/step={ms_per_step:.3f} main_us={main_us:.1f} zero_us={zero_us:.1f}")

    # The host-pointer boundary (the drop-in spmmKernel's transfers): one
    # call with inputs in host memory, copied in and out (pageable).
    host_call_ms = None
    if not args.no_host_call:
        Hh = H.cpu().numpy()
        t1 = time.perf_counter()
        ctx.spmm_host(rp, ci, val, origin, Hh, tasks)
        host_call_ms = (time.perf_counter() - t1) * 1e3
        del Hh
        log(f"host-pointer call {host_call_ms:.1f} ms (PCIe transfers included)")

    if args.copy_probe_mib:
        nb = args.copy_probe_mib << 20
        src = torch.ones(nb // 4, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy probe: {nb} bytes read and written")
        del src, dst

    sweep_arg = args.s_sweep if args.s_sweep is not None else (
        "32,64,128,256,512" if cfg == 5 and not args.k else "")
    s_sweep = [segment_size_sweep(ctx, call, tune, dev, tasks_for, cfg, costs, int(x), trials=10)
               for x in sweep_arg.split(",") if x.strip() and x.strip() != "none"]
    if s_sweep:
        log(f"S sweep: {s_sweep}")
        ctx.set_schedule(0, 0)
        ctx.set_locality(0, 0)
        ctx.set_cache_hints(0)
        ctx.set_occupancy(0)

    flops = 2.0 * g.nnz * K
    gflops = flops / (ms_per_step * 1e-3) / 1e9
    b_alg = workloads.algorithmic_bytes(g.n, g.nnz, K, T)
    achieved = b_alg / (main_us * 1e-6) / 1e9
    traffic = measured_traffic(cfg, S) if not args.k else None

    cpu = None
    if not args.no_cpu:
        # Bounded CPU sample: every 8th task of the same task list.
        sample = np.ascontiguousarray(tasks[::8])
        Hh = synth.features(g.n, K, workloads.FEATURE_SEED)
        Ch = np.zeros((g.n, K), np.float32)
        nnz_s = 0
        rpl = rp.astype(np.int64)
        for rs, re_, fo, ln in sample:
            lo = rpl[rs] + fo
            hi = rpl[re_ - 1] + ln if ln > 0 else rpl[re_]
            nnz_s += int(hi - lo)
        threads = oracle.max_threads()
        oracle.spmm_mean_f32_omp(rp, ci, val, origin, Hh, sample, threads, out=Ch)
        runs, tc = 0, 0.0
        while tc < args.cpu_seconds and runs < 50:
            t1 = time.perf_counter()
            oracle.spmm_mean_f32_omp(rp, ci, val, origin, Hh, sample, threads, out=Ch)
            tc += time.perf_counter() - t1
            runs += 1
        cpu_gflops = 2.0 * nnz_s * K * runs / tc / 1e9
        cpu = {"value": round(cpu_gflops, 3), "unit": "GFLOP/s", "cores": threads,
               "kind": "port",
               "sample": f"every 8th task of the same R-MAT task list ({len(sample)} tasks, "
                         f"{nnz_s} nonzeros, K={K}), {runs} timed passes after 1 warm-up; "
                         "reference kernel semantics restated in C/OpenMP"}
        log(f"cpu baseline {cpu_gflops:.2f} GFLOP/s on {threads} threads")

    out = {
        "metric": METRIC,
        "value": round(gflops, 2),
        "unit": "GFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": workload, "n": g.n, "nnz": g.nnz, "K": K, "S": S,
                   "tasks": T, "costs": list(costs), "device": info.name.decode(),
                   "main_kernel_us": round(main_us, 2), "zero_pass_us": round(zero_us, 2),
                   "per_task_mode_us": round(per_task_us, 2),
                   "host_pointer_call_ms": None if host_call_ms is None else round(host_call_ms, 1),
                   "preprocessing": prep,
                   "schedule": schedule,
                   "s_candidates": s_candidates,
                   **({"s_sweep": s_sweep} if s_sweep else {}),
                   "algorithmic_bytes": b_alg,
                   # measured HBM-side traffic per launch / the same launch time
                   "traffic_gbs": None if traffic is None else round(traffic / (main_us * 1e-6) / 1e9, 1)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
