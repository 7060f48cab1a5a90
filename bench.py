"""Benchmark of the MI355X CWLB-SpMM mean aggregation on one GPU.

Workload: the skewed R-MAT configuration (N = 2^22 nodes, 2^26 R-MAT samples
a=.57 b=c=.19 d=.05 relabelled and deduplicated, unit edge values, K = 128
FP32 features in U[-1,1)), degree-reordered and cost-weighted partitioned
with the committed gfx950 cost coefficients; S is chosen among the three
wave-based candidates as the reference's --candidates mode does.

A step is one SpMM call (split-row clearing + aggregation kernel) over the
whole graph with all inputs resident in HBM.  W warm-up steps, then K timed
steps between synchronisations, timed with HIP events on the launch stream.
C is cleared once before the steps, as the reference clears its output
outside its timed kernel; every step rewrites each row with nonzeros and,
as the reference's kernel, leaves the rows without nonzeros at that 0
(CWLB_SPMM_KEEP_EMPTY_ROWS).

Prints one JSON line: GFLOP/s (2 nnz K / t) as `value`; the aggregation
kernel's roofline: its algorithmic bytes per launch over its mean
event-timed duration against 8 TB/s (`achieved`, `frac`), and the
L2-to-fabric traffic of one launch (rocprofv3 FETCH_SIZE + WRITE_SIZE;
Infinity Cache hits are included, so it is an upper bound on the HBM bytes),
measured on a replay of the very launch that was timed (child processes
running this file with --pmc-child), with its rate and fraction
(`traffic`, `traffic_gbs`, `traffic_frac`), next to the compulsory bytes
per launch, the L2 hit rate and the occupancy; the CPU
baseline (the reference kernel's semantics restated with OpenMP, on this
host's cores, over a sample of the tasks); and the parity of the timed
launch: the whole of C after the last timed step against the oracle, at
1e-5 relative / 1e-6 absolute per element.  Exits with status 1, after the
line, when that check fails.
"""
import argparse
import csv
import glob
import json
import os
import re
import shutil
import subprocess
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "cwlb-spmm_amd"))

METRIC = "SpMM GFLOP/s (2·nnz·K/t) + achieved HBM GB/s vs peak, FP32 mean agg"
HBM_PEAK_GBS = 8000.0
COST_FILE = os.path.join(ROOT, "cwlb-spmm_amd", "resources", "spmm_costs_gfx950.txt")
GOLDEN = os.path.join(ROOT, "tests", "golden", "partition_golden.json")
# Counter passes of the traffic measurement, one rocprofv3 run each (a run
# holds at most 4 TCC counters: FETCH_SIZE takes 3 and WRITE_SIZE 2).
PMC_PASSES = [["FETCH_SIZE"], ["WRITE_SIZE"], ["TCC_HIT_sum", "TCC_MISS_sum"],
              ["MeanOccupancyPerCU"]]
PROBE_MIB = 1024  # the known-size device-to-device copy that scales the counters


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


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


def cpu_model():
    """The host CPU's model name and logical core count."""
    name = None
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                name = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return name, os.cpu_count()


# ----------------------------------------------------------------- counters
def schedule_args(S, sched):
    """Command-line arguments that fix the launch: segment size and schedule."""
    return ["--s", str(S), "--tasks-per-wave", str(sched["tasks_per_wave"]),
            "--slices", str(sched["feature_slices"]), "--run-order", str(sched["run_order"]),
            "--xcd-blocks", str(sched["xcd_blocks"]), "--hot-mb", str(sched["hot_bytes"] >> 20),
            "--occupancy", str(sched["occupancy"]), "--phases", str(sched.get("phases", 0)),
            "--tiling", str(sched.get("tiling", 0))]


def read_counter_csv(path):
    """{(kernel name, counter): [value per dispatch]} in dispatch order, and
    the dispatch order of the copy kernels."""
    rows = list(csv.DictReader(open(path)))
    key = "Dispatch_Id" if rows and "Dispatch_Id" in rows[0] else None
    if key:
        rows.sort(key=lambda r: int(r[key]))
    vals = {}
    for r in rows:
        vals.setdefault((r["Kernel_Name"], r["Counter_Name"]), []).append(float(r["Counter_Value"]))
    return vals


# Counters that add up over the dispatches of one call (a column-phased call
# dispatches the aggregation kernel once per phase).
ADDITIVE = {"FETCH_SIZE", "WRITE_SIZE", "TCC_HIT_sum", "TCC_MISS_sum"}


def per_call_value(counter, values, per_call):
    """One call's value of a counter read on every dispatch: the mean over
    the dispatches, times the dispatches of one call when it adds up."""
    mean = sum(values) / len(values)
    return mean * per_call if counter in ADDITIVE else mean


def measure_counters(args, cfg, K, S, sched, per_call=1):
    """Replays the timed launch (same workload, S and schedule) in child
    processes under rocprofv3, one counter pass each, each with a 1 GiB
    device-to-device copy as the known-size reference.  Returns the
    aggregation kernel's counter values per call (the mean over its
    dispatches, times the per_call dispatches of one call for the additive
    counters), the copy's, and the kernel's name; raises RuntimeError when a
    pass fails."""
    rocprof = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    if not os.path.exists(rocprof):
        raise RuntimeError("rocprofv3 not found")
    out = {"kernel": {}, "copy": {}, "name": None, "dispatches": 0}
    env = dict(os.environ, TMPDIR="/tmp")
    child = [sys.executable, os.path.abspath(__file__), "--pmc-child", "--cfg", str(cfg),
             "--k", str(K), "--costs", args.costs, "--copy-probe-mib", str(PROBE_MIB)]
    child += schedule_args(S, sched)
    for counters in PMC_PASSES:
        tmp = tempfile.mkdtemp(prefix="cwlb_pmc_", dir="/tmp")
        cmd = ["timeout", "-s", "KILL", "240", rocprof, "--pmc", *counters, "--output-format",
               "csv", "-d", tmp, "-o", "run", "--", *child]
        t0 = time.perf_counter()
        r = subprocess.run(cmd, cwd="/tmp", env=env, stdout=subprocess.PIPE,
                           stderr=subprocess.STDOUT, text=True)
        files = glob.glob(os.path.join(tmp, "**", "*counter_collection.csv"), recursive=True)
        done = "[bench] pmc child done" in r.stdout
        if r.returncode in (124, 137, -9) or not files or not done:
            tail = "\n".join(r.stdout.splitlines()[-8:])
            shutil.rmtree(tmp, ignore_errors=True)
            raise RuntimeError(f"counter pass {counters} failed (rc {r.returncode}): {tail}")
        vals = read_counter_csv(files[0])
        shutil.rmtree(tmp, ignore_errors=True)
        for (kname, cname), v in vals.items():
            if "spmm_mean_runs" in kname:
                out["kernel"][cname] = per_call_value(cname, v, per_call)
                out["dispatches"] = len(v)
                out["dispatches_per_call"] = per_call
                out["name"] = kname
            elif "copyBuffer" in kname:
                out["copy"][cname] = v[-1]  # the probe is the last copy of the run
        log(f"counter pass {counters}: {time.perf_counter() - t0:.1f} s (rc {r.returncode})")
    return out


def kernel_template(name):
    """'spmm_mean_runs<...>' from a demangled kernel name."""
    m = re.search(r"spmm_mean_runs<[^>]*>", name or "")
    return m.group(0).replace(" ", "") if m else name


def pmc_child(args):
    """--pmc-child: one workload and fixed schedule, 1 + steps launches and
    the 1 GiB copy probe; the parent reads the counters."""
    import numpy as np
    import torch

    from cwlb_amd import capi, workloads
    cfg, K = args.cfg, args.k or workloads.FEATURE_DIM[args.cfg]
    g = workloads.graph(cfg)
    origin, rp, ci, val = capi.reorder_by_degree(g.row_ptr, g.col_idx, g.val)
    costs = capi.read_costs(args.costs)
    tasks = capi.partition(rp, costs, capi.capacity_from_s(args.s, costs))
    stream = torch.cuda.current_stream()
    ctx = capi.Context(0, stream.cuda_stream)
    large_k = K > ctx.info().max_work_group_size
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    d = [dev(x) for x in (rp, ci, val, origin, tasks.reshape(-1))]
    H = torch.empty((g.n, K), dtype=torch.float32, device="cuda")
    ctx.fill_features(H, g.n, K, workloads.FEATURE_SEED)
    # Cleared once before the steps, as the reference clears its output
    # outside its timed kernel (parallelMatrix.cpp:112): the rows without
    # nonzeros, which its kernel never writes (:166), stay 0 -- the steps
    # leave them (KEEP_EMPTY_ROWS) -- and so do the rows the partition
    # leaves out (empty rows costlier than the capacity).
    C = torch.zeros((g.n, K), dtype=torch.float32, device="cuda")
    ctx.set_schedule(args.tasks_per_wave, args.slices)
    ctx.set_locality(args.run_order, args.xcd_blocks)
    ctx.set_cache_hints(args.hot_mb << 20)
    ctx.set_occupancy(args.occupancy)
    ctx.set_column_phases(args.phases)
    ctx.set_lane_tiling(args.tiling)
    for _ in range(1 + args.steps):
        ctx.spmm(d[0], d[1], d[2], d[3], g.n, g.nnz, H, g.n, K, d[4], len(tasks), C,
                 flags=capi.KEEP_EMPTY_ROWS, large_k=large_k)
    nb = args.copy_probe_mib << 20
    src = torch.ones(nb // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    ctx.close()
    print("[bench] pmc child done", flush=True)


def roofline_record(counters, err, b_alg, b_min, main_us, launched):
    """The roofline object of the aggregation kernel: `achieved` is its
    algorithmic bytes per launch (4(N+1) + 8 nnz + 4 nnz K + 4 N K + 4 N + 16 T,
    every feature-row gather counted as a read) over its mean duration, and
    `frac` that rate against 8 TB/s; gathers the caches serve let it exceed 1.
    `traffic` is the measured traffic per launch (L2-to-fabric bytes,
    Infinity Cache hits included: an upper bound on the HBM bytes), with its
    rate and fraction beside it (`traffic_gbs`, `traffic_frac`), and the
    compulsory bytes (CSR, each referenced feature row and C once)."""
    t = main_us * 1e-6
    achieved = b_alg / t / 1e9
    rec = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
           "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None, "kernel_us": round(main_us, 2),
           "achieved_kind": "algorithmic bytes per launch (every feature-row gather counted as a "
                            "read) over the kernel's mean duration",
           "algorithmic_bytes": b_alg, "traffic_gbs": None, "traffic_frac": None,
           "compulsory_bytes": b_min, "compulsory_gbs": round(b_min / t / 1e9, 1),
           "compulsory_frac": round(b_min / t / 1e9 / HBM_PEAK_GBS, 4),
           "max_waves_per_cu": launched.get("max_waves_per_cu")}
    if counters is None:
        rec["counters_error"] = err
        return rec
    k, c = counters["kernel"], counters["copy"]
    probe = PROBE_MIB << 20
    fetch_scale = probe / (c["FETCH_SIZE"] * 1024.0)
    write_scale = probe / (c["WRITE_SIZE"] * 1024.0)
    read_b = k["FETCH_SIZE"] * 1024.0 * fetch_scale
    write_b = k["WRITE_SIZE"] * 1024.0 * write_scale
    traffic = read_b + write_b
    traffic_gbs = traffic / t / 1e9
    hits, misses = k.get("TCC_HIT_sum"), k.get("TCC_MISS_sum")
    rec.update({
        "traffic": round(traffic), "traffic_read": round(read_b), "traffic_write": round(write_b),
        "traffic_gbs": round(traffic_gbs, 1), "traffic_frac": round(traffic_gbs / HBM_PEAK_GBS, 4),
        "traffic_kind": "L2-to-fabric bytes (FETCH_SIZE + WRITE_SIZE), Infinity Cache hits "
                        "included: an upper bound on the HBM bytes",
        "kernel": kernel_template(counters["name"]),
        "l2_hit_rate": None if not hits else round(hits / (hits + misses), 4),
        "waves_per_cu": None if k.get("MeanOccupancyPerCU") is None
        else round(k["MeanOccupancyPerCU"], 2),
        "counters": {"FETCH_SIZE_kib": round(k["FETCH_SIZE"], 1),
                     "WRITE_SIZE_kib": round(k["WRITE_SIZE"], 1),
                     "fetch_scale": round(fetch_scale, 5), "write_scale": round(write_scale, 5),
                     "copy_probe_bytes": probe, "dispatches": counters["dispatches"],
                     "dispatches_per_call": counters.get("dispatches_per_call", 1),
                     "how": "rocprofv3 --pmc, one pass per counter group, on a replay of the "
                            "timed launch in a child process; scales from a 1 GiB "
                            "device-to-device copy in the same runs"}})
    return rec


# ------------------------------------------------------------------- parity
RTOL, ATOL = 1e-5, 1e-6  # per element: |C - ref| <= ATOL + RTOL |ref|
PARITY_COLS = 256  # feature columns per oracle block


def parity_check(torch, C, H, rp, ci, val, origin, tasks, threads):
    """The whole of C, as the timed launch left it, against the oracle (the
    reference kernel's semantics, parallelMatrix.cpp:148-236: per task row
    chunk, fp32 FMA sum in nonzero order, divided by the full row degree,
    stored for whole rows and added atomically for split rows) on the same
    device-resident H, at ATOL + RTOL |ref| per element.  Mean aggregation
    is independent per feature column, so the oracle runs on blocks of
    PARITY_COLS columns of H copied back from the device, and each block is
    compared on the device.  Returns the record for the JSON line."""
    import numpy as np

    import oracle
    n, K = C.shape
    t0 = time.perf_counter()
    worst, nan_rows, oracle_s = -float("inf"), 0, 0.0
    for j0 in range(0, K, PARITY_COLS):
        j1 = min(K, j0 + PARITY_COLS)
        Hb = np.ascontiguousarray(H[:, j0:j1].cpu().numpy())
        t1 = time.perf_counter()
        ref = oracle.spmm_mean_f32_omp(rp, ci, val, origin, Hb, tasks, threads)
        oracle_s += time.perf_counter() - t1
        del Hb
        ref_dev = torch.from_numpy(ref).to(C.device)
        del ref
        for r0 in range(0, n, 1 << 20):
            c = C[r0:r0 + (1 << 20), j0:j1]
            r = ref_dev[r0:r0 + (1 << 20)]
            nan_rows += int(torch.isnan(c).any(dim=1).sum().item())
            excess = ((c - r).abs() - (ATOL + RTOL * r.abs())).max().item()
            worst = max(worst, excess)
        del ref_dev
    ok = nan_rows == 0 and worst <= 0.0
    return {"ok": ok, "max_excess": worst, "nan_rows": nan_rows,
            "elements": int(n) * int(K), "rtol": RTOL, "atol": ATOL,
            "oracle_threads": threads, "oracle_s": round(oracle_s, 2),
            "check_s": round(time.perf_counter() - t0, 2),
            "how": "whole C after the last timed step, against the oracle's OpenMP "
                   "restatement of the reference kernel on the same H and task list, "
                   f"in blocks of {PARITY_COLS} feature columns"}


# ------------------------------------------------------------ preprocessing
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
    ctx.set_column_phases(0)
    ctx.set_lane_tiling(0)
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
                         "occupancy": ctx.occupancy(), "phases": ctx.column_phases(),
                         "tiling": ctx.lane_tiling()},
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


def schedule_build_times(call_fresh, sched):
    """Wall time (ms) that the chosen schedule's one-off builds add to the
    first call on a new context: the cache hints (column in-degrees, their
    histogram, one bit per nonzero), the run order sorted by output row and
    the column phases' buffers (their allocation: the band sort itself runs
    in every call, inside the step).  Each is the first call's time minus
    the second's, on a context that has only that setting."""
    out = {"cache_hint_build_ms": None, "run_order_build_ms": None,
           "column_phase_alloc_ms": None}
    if sched.get("phases", 0) > 1:
        first, second = call_fresh({"phases": sched["phases"]})
        out["column_phase_alloc_ms"] = round(first - second, 2)
    if sched["hot_bytes"] > 0:
        first, second = call_fresh({"hot_bytes": sched["hot_bytes"]})
        out["cache_hint_build_ms"] = round(first - second, 2)
    if sched["run_order"] == 2:
        first, second = call_fresh({"run_order": 2})
        out["run_order_build_ms"] = round(first - second, 2)
    return out


# --------------------------------------------------------------------- main
def parse_args():
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
    ap.add_argument("--no-pmc", action="store_true",
                    help="skip the rocprofv3 counter passes (traffic, L2 hit rate, occupancy)")
    ap.add_argument("--pmc-child", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--tasks-per-wave", type=int, default=0,
                    help="fixed launch schedule (with --slices) instead of tuning")
    ap.add_argument("--slices", type=int, default=0)
    ap.add_argument("--occupancy", type=int, default=0, choices=(0, 6),
                    help="fixed schedule: 6 = the 6-waves-per-SIMD kernel variant")
    ap.add_argument("--phases", type=int, default=0,
                    help="fixed schedule: column phases (cwlb_ctx_set_column_phases)")
    ap.add_argument("--tiling", type=int, default=0, choices=(0, 1, 2),
                    help="fixed schedule: lane tiling (cwlb_ctx_set_lane_tiling: 1 power-of-two "
                         "slots, 2 packed slots)")
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
    return ap.parse_args()


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(the multi-GPU sharding is a design note, not a build target)", file=sys.stderr)
        sys.exit(2)
    if args.pmc_child:
        pmc_child(args)
        return

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
    # Cleared once before the steps, as the reference clears its output
    # outside its timed kernel (parallelMatrix.cpp:112): the rows without
    # nonzeros, which its kernel never writes (:166), stay 0 -- the steps
    # leave them (KEEP_EMPTY_ROWS) -- and so do the rows the partition
    # leaves out (empty rows costlier than the capacity).
    C = torch.zeros((g.n, K), dtype=torch.float32, device="cuda")

    def tasks_for(S):
        cap = capi.capacity_from_s(S, costs)
        return capi.partition(rp, costs, cap)

    def call(d_t, n_t, timed, c=ctx):
        return c.spmm(d_rp, d_ci, d_v, d_o, g.n, g.nnz, H, g.n, K, d_t, n_t, C, timed=timed,
                      flags=capi.KEEP_EMPTY_ROWS, large_k=large_k)

    def tune(d_t, n_t):
        return ctx.tune_schedule(d_rp, d_ci, d_v, d_o, g.n, g.nnz, H, g.n, K, d_t, n_t, C,
                                 trials=3, locality=True)

    # S: the best of the three wave-based candidates (main.cpp:534-577), or
    # fixed.  As in the drop-in driver's candidate search (run_single_s per
    # S), each S gets its launch schedule tuned once (cwlb_ctx_tune_schedule,
    # outside the timed region), and the S with the fastest tuned aggregation
    # is kept.  A fixed schedule (--tasks-per-wave etc.) or --no-tune ranks
    # the S by the automatic schedule instead.
    fixed = bool(args.tasks_per_wave or args.slices or args.run_order or args.xcd_blocks
                 or args.hot_mb or args.occupancy or args.phases or args.tiling)
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
        ctx.set_column_phases(0)
        ctx.set_lane_tiling(0)
        for _ in range(5):
            call(d_t, len(tk), False)
        us = float(np.mean([call(d_t, len(tk), True).total_us for _ in range(10)]))
        rec = {"S": S, "tasks": int(len(tk)), "automatic_us": round(us, 1)}
        rank = us
        if tuning:
            t0 = time.perf_counter()
            m, sl, (order, xcd) = tune(d_t, len(tk))
            rec["tuning_ms"] = round((time.perf_counter() - t0) * 1e3, 1)
            t_tune += rec["tuning_ms"]
            rec["schedule"] = {"tasks_per_wave": m, "feature_slices": sl, "run_order": order,
                               "xcd_blocks": xcd, "hot_bytes": ctx.cache_hints(),
                               "occupancy": ctx.occupancy(), "phases": ctx.column_phases(),
                               "tiling": ctx.lane_tiling()}
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
    schedule = {"tasks_per_wave": 0, "feature_slices": 0, "run_order": 0, "xcd_blocks": 0,
                "hot_bytes": 0, "occupancy": 0, "phases": 0, "tiling": 0, "tuned": False,
                "automatic_schedule_us": round(float(auto_us), 1)}
    if fixed:
        schedule.update(tasks_per_wave=args.tasks_per_wave, feature_slices=args.slices,
                        run_order=args.run_order, xcd_blocks=args.xcd_blocks,
                        hot_bytes=args.hot_mb << 20, occupancy=args.occupancy,
                        phases=args.phases, tiling=args.tiling)
        log(f"fixed schedule: {schedule}")
    elif tuning:
        # One cwlb_ctx_tune_schedule call per S candidate (each candidate's
        # own time is in s_candidates).
        schedule.update(tuned, tuned=True, tuning_ms_all_candidates=round(t_tune, 1))
        log(f"tuned schedule: {schedule}")

    def apply(c, sched):
        c.set_schedule(sched["tasks_per_wave"], sched["feature_slices"])
        c.set_locality(sched["run_order"], sched["xcd_blocks"])
        c.set_cache_hints(sched["hot_bytes"])
        c.set_occupancy(sched["occupancy"])
        c.set_column_phases(sched["phases"])
        c.set_lane_tiling(sched.get("tiling", 0))

    apply(ctx, schedule)

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
    # Outside the timed region: the output of the last timed step, checked
    # whole against the oracle (the launch and schedule it ran with beside).
    timed_launch = ctx.last_launch()
    parity = parity_check(torch, C, H, rp, ci, val, origin, tasks, oracle.max_threads())
    parity["launch"] = {"S": S, **timed_launch}
    log(f"parity of the timed launch: ok={parity['ok']} max_excess={parity['max_excess']:.3g} "
        f"({parity['check_s']} s)")
    # Per-kernel durations: the reference protocol (event-timed launches).
    times = [call(d_t, T, True) for _ in range(args.steps)]
    main_us = float(np.mean([t.main_us for t in times]))
    zero_us = float(np.mean([t.zero_us for t in times]))
    # The schedule those launches resolved to (automatic choices included).
    launched = ctx.last_launch()
    schedule["launched"] = launched
    log(f"S={S} T={T} ms/step={ms_per_step:.3f} main_us={main_us:.1f} zero_us={zero_us:.1f}")

    # What the chosen schedule's one-off builds cost a first call on a new
    # graph (outside the timed steps, like the reorder and the partition).
    def call_fresh(setting):
        c = capi.Context(0, stream.cuda_stream)
        try:
            only = dict(schedule)
            only.update(hot_bytes=0, run_order=0, phases=0)
            only.update(setting)
            apply(c, only)
            walls = []
            for _ in range(2):
                torch.cuda.synchronize()
                t1 = time.perf_counter()
                call(d_t, T, False, c)
                torch.cuda.synchronize()
                walls.append((time.perf_counter() - t1) * 1e3)
            return walls
        finally:
            c.close()

    prep.update(schedule_build_times(call_fresh, schedule))
    log(f"schedule builds: hints {prep['cache_hint_build_ms']} ms, "
        f"run order {prep['run_order_build_ms']} ms, "
        f"phase buffers {prep['column_phase_alloc_ms']} ms")
    # The reference's structure (one task per wave, one atomic add per
    # partial segment, rows without nonzeros left), for comparison.
    pt = [ctx.spmm(d_rp, d_ci, d_v, d_o, g.n, g.nnz, H, g.n, K, d_t, T, C,
                   flags=capi.PER_TASK | capi.KEEP_EMPTY_ROWS, large_k=large_k)
          for _ in range(10)]
    per_task_us = float(np.mean([t.total_us for t in pt]))

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
    ctx.close()

    flops = 2.0 * g.nnz * K
    gflops = flops / (ms_per_step * 1e-3) / 1e9
    b_alg = workloads.algorithmic_bytes(g.n, g.nnz, K, T)
    n_empty = int(np.count_nonzero(np.diff(rp) == 0))
    referenced = int(np.count_nonzero(np.bincount(g.col_idx, minlength=g.n)))
    b_min = workloads.compulsory_bytes(referenced, g.n, g.nnz, K) + 16 * T

    counters, pmc_err = None, "skipped (--no-pmc)"
    if not args.no_pmc:
        # The device buffers of the timed run are released first: the child
        # processes build the same workload again.
        del d_rp, d_ci, d_v, d_o, H, C, d_t
        torch.cuda.empty_cache()
        try:
            counters = measure_counters(args, cfg, K, S, schedule,
                                        per_call=launched.get("column_phases", 1))
            pmc_err = None
        except (RuntimeError, OSError, KeyError, ZeroDivisionError) as e:
            pmc_err = str(e)
            log(f"counters: {e}")
    roofline = roofline_record(counters, pmc_err, b_alg, b_min, main_us, launched)
    log(f"roofline: {roofline}")

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
        model, logical = cpu_model()
        cpu = {"value": round(cpu_gflops, 3), "unit": "GFLOP/s", "cores": threads,
               "kind": "port", "cpu_model": model, "host_logical_cpus": logical,
               "sample": f"every 8th task of the same {workload} task list ({len(sample)} "
                         f"tasks, {nnz_s} nonzeros, K={K}), {runs} timed passes after 1 "
                         "warm-up; reference kernel semantics restated in C/OpenMP"}
        log(f"cpu baseline {cpu_gflops:.2f} GFLOP/s on {threads} threads ({model})")

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
                   "empty_rows": "C cleared once before the timed steps, as the reference "
                                 "clears it outside its timed kernel; the steps write every "
                                 "row with nonzeros and leave the rows without "
                                 f"({n_empty} of {g.n}), as the reference's kernel does",
                   "host_pointer_call_ms": None if host_call_ms is None else round(host_call_ms, 1),
                   "preprocessing": prep,
                   "schedule": schedule,
                   "s_candidates": s_candidates,
                   **({"s_sweep": s_sweep} if s_sweep else {})},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "parity": parity,
    }
    print(json.dumps(out), flush=True)
    if not parity["ok"]:
        log("the timed launch's C does not match the oracle")
        sys.exit(1)


if __name__ == "__main__":
    main()
