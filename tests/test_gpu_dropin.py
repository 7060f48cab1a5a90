"""GPU tests of the device degree reordering, the calibration, the C++17
drop-in layer (through tests/cxx/bin/dropin_probe) and the cwlb-spmm /
costWrite executables.

Parity bar: the reordering is bit-exact with the oracle (the reference's
(degree, id) order); aggregated features within 1e-5 relative + 1e-6
absolute of the reference-order oracle and of the fp64 closed form.
"""
import os
import subprocess

import numpy as np
import pytest

import oracle
from conftest import SKEWED_COSTS, UNIT_COSTS
from cwlb_amd import capi, synth, workloads
from dropin_util import (BIN, ProbeError, probe, read_order, write_csr, write_f32, write_order,
                         write_tasks)

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-5, 1e-6


def dev(a):
    import torch
    a = np.ascontiguousarray(a)
    if a.size == 0:
        a = np.zeros(1, a.dtype)
    return torch.from_numpy(a).cuda()


def reorder_on_device(ctx, rp, ci, val):
    import torch
    n = len(rp) - 1
    nnz = len(ci)
    origin = torch.full((max(n, 1),), -7, dtype=torch.int32, device="cuda")
    rp_out = torch.full((n + 1,), -7, dtype=torch.int32, device="cuda")
    ci_out = torch.full((max(nnz, 1),), -7, dtype=torch.int32, device="cuda")
    v_out = torch.full((max(nnz, 1),), -7.0, dtype=torch.float32, device="cuda")
    ctx.reorder_device(n, nnz, dev(rp), dev(ci), dev(val), origin, rp_out, ci_out, v_out)
    return (origin.cpu().numpy()[:n], rp_out.cpu().numpy(), ci_out.cpu().numpy()[:nnz],
            v_out.cpu().numpy()[:nnz])


def assert_same_order(got, exp):
    for a, b in zip(got, exp):
        assert np.array_equal(a, b)


# ------------------------------------------------------ device reordering
@pytest.mark.parametrize("cfg", [1, 2, 3, 4, 5])
def test_device_reorder_small(gpu_ctx, cfg):
    g = workloads.small(cfg)
    got = reorder_on_device(gpu_ctx, g.row_ptr, g.col_idx, g.val)
    assert_same_order(got, oracle.reorder_by_degree(g.row_ptr, g.col_idx, g.val))


@pytest.mark.parametrize("cfg", [4, 5])
def test_device_reorder_full(gpu_ctx, cfg):
    """Full-size R-MAT (max degree ~1e5) and mesh (N = 16M): bit-exact with
    the host reordering, which the CPU tests pin to the oracle."""
    g = workloads.graph(cfg)
    print(f"cfg={cfg} n={g.n} nnz={g.nnz}", flush=True)
    got = reorder_on_device(gpu_ctx, g.row_ptr, g.col_idx, g.val)
    exp = capi.reorder_by_degree(g.row_ptr, g.col_idx, g.val)
    assert_same_order(got, exp)
    assert np.array_equal(got[0], np.argsort(np.diff(g.row_ptr), kind="stable"))


def test_device_reorder_edge_cases(gpu_ctx, rng):
    # no rows
    got = reorder_on_device(gpu_ctx, np.zeros(1, np.int32), np.zeros(0, np.int32),
                            np.zeros(0, np.float32))
    assert list(got[1]) == [0]
    # all rows empty, then hub rows next to empty and short rows, values kept
    # the long rows (more than 16 entries) are copied in chunks of 4,096
    # output entries: rows ending on, just before and just after a chunk end
    chunked = np.array([17] * 300 + [4095, 4096, 4097, 12289, 16, 0, 1] + [40] * 77, np.int64)
    for degs in (np.zeros(1000, np.int64), np.array([0, 3000, 1, 17, 16, 0, 64, 65, 3000, 2]),
                 chunked, np.array([9000], np.int64), np.array([17], np.int64)):
        rp = np.concatenate([[0], np.cumsum(degs)]).astype(np.int32)
        ci = rng.integers(0, 50, rp[-1]).astype(np.int32)
        val = rng.normal(size=rp[-1]).astype(np.float32)
        got = reorder_on_device(gpu_ctx, rp, ci, val)
        assert_same_order(got, oracle.reorder_by_degree(rp, ci, val))


def test_device_reorder_rejects_bad_offsets(gpu_ctx):
    ci = np.zeros(4, np.int32)
    val = np.ones(4, np.float32)
    with pytest.raises(capi.CwlbError) as e:
        reorder_on_device(gpu_ctx, np.array([0, 3, 2, 4], np.int32), ci, val)
    assert e.value.status == capi.INVALID_ARG
    with pytest.raises(capi.CwlbError) as e:
        reorder_on_device(gpu_ctx, np.array([0, 1, 2, 3], np.int32), ci, val)
    assert e.value.status == capi.RUNTIME_ERROR


# ------------------------------------------------------------- calibration
@pytest.mark.parametrize("K,WI,writers", [(128, 131072, 8), (64, 8192, 8), (40, 1000, 3)])
def test_calibration_normalisation(gpu_ctx, K, WI, writers):
    """Each coefficient is the reference's normalisation of its benchmark's
    measured mean launch time: (ms * 1e6) / WI / K * 10 for compute, load
    and store, (ms * 1e6) / ops * 10 for the atomic with ops = writer groups
    x feature block (utils.cpp:419-421, 522-524, 583-585, 791-806), equal
    bit for bit to the oracle's restatement applied to the reported times.
    The times obey the hardware's limits: the stores and loads move at most
    8 TB/s (40 bytes / coefficient per ns), the fma chains run below the
    157.3 TFLOP/s FP32 peak, and a contended atomic costs more than a
    coalesced store (the default shapes, the costWrite defaults with fewer
    repeats)."""
    c, rep = gpu_ctx.calibrate_report(K=K, repeat=20, WI=WI, load_MB=64, atomic_writers=writers)
    ms = (rep.compute_ms, rep.load_ms, rep.store_ms, rep.atomic_ms)
    assert all(np.isfinite(ms)) and all(m > 0 for m in ms), ms
    want, ops = oracle.cost_coefficients(ms, K, WI, writers)
    assert list(c.tuple4()) == want, (c.tuple4(), want)
    assert [rep.compute_ops, rep.load_ops, rep.store_ops, rep.atomic_ops] == ops
    assert rep.load_bytes == rep.store_bytes == 4 * WI * K
    assert (c.K, c.WI, c.repeat, c.atomic_writers_per_addr) == (K, WI, 20, writers)
    if K == 128:
        store_gbs, load_gbs = 40.0 / c.C_store_ns, 40.0 / c.C_load_ns
        assert store_gbs == pytest.approx(rep.store_bytes / (rep.store_ms * 1e6), rel=1e-12)
        assert store_gbs <= 8000.0 and load_gbs <= 8000.0, (store_gbs, load_gbs)
        assert 2.0 * WI * K / (rep.compute_ms * 1e-3) <= 157.3e12
        assert c.C_atomic_ns > c.C_store_ns, c.tuple4()
    print(f"K={K} WI={WI}: coefficients {c.tuple4()} from ms {ms}", flush=True)


def test_calibration_arguments(gpu_ctx):
    c = gpu_ctx.calibrate(K=64, repeat=3, WI=8192, load_MB=16, atomic_writers=8)
    vals = c.tuple4()
    assert all(np.isfinite(vals)) and all(v > 0 for v in vals), vals
    assert (c.K, c.WI, c.repeat, c.atomic_writers_per_addr) == (64, 8192, 3, 8)
    with pytest.raises(capi.CwlbError) as e:
        gpu_ctx.calibrate(K=0, repeat=3, WI=8192, load_MB=16, atomic_writers=8)
    assert e.value.status == capi.INVALID_ARG
    with pytest.raises(capi.CwlbError) as e:
        gpu_ctx.calibrate(K=1 << 20, repeat=1, WI=64, load_MB=1, atomic_writers=1)
    assert e.value.status == capi.RUNTIME_ERROR  # data_MB_for_load too small for K


# ------------------------------------------------------- drop-in C++ layer
def test_dropin_device_properties():
    out = probe("device").split()
    props = dict(zip(out[::2], out[1::2]))
    assert props["wg"] == "1024" and props["wave"] == "64"
    assert props["arch"].startswith("gfx950")
    assert int(props["cu"]) > 0


@pytest.mark.parametrize("cfg", [1, 4])
def test_dropin_reorder_gpu(tmp_path, cfg):
    g = workloads.small(cfg)
    write_csr(tmp_path / "in", g.row_ptr, g.col_idx, g.val)
    probe("reorder-gpu", tmp_path / "in", tmp_path / "out")
    assert_same_order(read_order(tmp_path / "out"),
                      oracle.reorder_by_degree(g.row_ptr, g.col_idx, g.val))


def spmm_case(tmp_path, cfg, K, S, costs=SKEWED_COSTS, seed=None):
    g = workloads.small(cfg, seed)
    p = workloads.prepare(g, costs, S)
    H = synth.features(g.n, K, 7)
    write_order(tmp_path / "ord", p.origin, p.row_ptr, p.col_idx, p.val)
    write_f32(tmp_path / "H", H)
    write_tasks(tmp_path / "tasks", p.tasks)
    return g, p, H


def oracle_check(got, g, p, H):
    ref32 = oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H, p.tasks)
    ref64 = oracle.spmm_mean_f64(g.row_ptr, g.col_idx, g.val, H)
    np.testing.assert_allclose(got, ref32, rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(got, ref64, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("cfg,K,S", [(1, 32, 4), (2, 64, 16), (3, 600, 8), (4, 128, 32),
                                     (5, 32, 2)])
def test_dropin_spmm_kernel(tmp_path, cfg, K, S):
    g, p, H = spmm_case(tmp_path, cfg, K, S)
    out = probe("spmm", tmp_path / "ord", tmp_path / "H", g.n, K, tmp_path / "tasks",
                tmp_path / "C").split()
    assert float(out[1]) > 0 and out[3] == str(g.n) and out[5] == str(K)
    got = np.fromfile(tmp_path / "C", np.float32).reshape(g.n, K)
    oracle_check(got, g, p, H)


def test_dropin_large_k(tmp_path):
    g, p, H = spmm_case(tmp_path, 1, 1100, 5, UNIT_COSTS, seed=9)
    with pytest.raises(ProbeError) as e:
        probe("spmm", tmp_path / "ord", tmp_path / "H", g.n, 1100, tmp_path / "tasks",
              tmp_path / "C")
    assert e.value.kind == "invalid_argument"
    assert "use spmmKernelLargeKFallback for larger K" in e.value.msg
    probe("spmm-large", tmp_path / "ord", tmp_path / "H", g.n, 1100, tmp_path / "tasks",
          tmp_path / "C")
    got = np.fromfile(tmp_path / "C", np.float32).reshape(g.n, 1100)
    oracle_check(got, g, p, H)
    g, p, H = spmm_case(tmp_path, 1, 64, 5, UNIT_COSTS, seed=9)
    with pytest.raises(ProbeError) as e:
        probe("spmm-large", tmp_path / "ord", tmp_path / "H", g.n, 64, tmp_path / "tasks",
              tmp_path / "C")
    assert e.value.msg == "spmmKernelLargeKFallback requires K > device max work-group size."


def test_dropin_degenerate_calls(tmp_path):
    g, p, H = spmm_case(tmp_path, 1, 32, 4)
    # no tasks: zero matrix, time 0 (parallelMatrix.cpp:101-104)
    write_tasks(tmp_path / "none", np.zeros((0, 4), np.int32))
    out = probe("spmm", tmp_path / "ord", tmp_path / "H", g.n, 32, tmp_path / "none",
                tmp_path / "C").split()
    assert float(out[1]) == 0.0
    assert not np.fromfile(tmp_path / "C", np.float32).any()
    # K == 0 (parallelMatrix.cpp:80-83)
    out = probe("spmm", tmp_path / "ord", tmp_path / "H", g.n, 0, tmp_path / "tasks",
                tmp_path / "C").split()
    assert float(out[1]) == 0.0 and out[5] == "0"
    # a column index outside H
    ci = p.col_idx.copy()
    ci[0] = g.n + 3
    write_order(tmp_path / "bad", p.origin, p.row_ptr, ci, p.val)
    with pytest.raises(ProbeError) as e:
        probe("spmm", tmp_path / "bad", tmp_path / "H", g.n, 32, tmp_path / "tasks",
              tmp_path / "C")
    assert e.value.kind == "invalid_argument"


@pytest.mark.parametrize("tune", ["1", "0"], ids=["tuned", "automatic"])
def test_dropin_run_single_s(tmp_path, tune):
    """run_single_s: 50 timed launches after 20 warm-ups, the reference's
    tasks, the oracle's features; the launch schedule tuned first unless
    CWLB_TUNE_SCHEDULE=0."""
    g = workloads.small(4, seed=6)
    K, S = 128, 16
    order = capi.reorder_by_degree(g.row_ptr, g.col_idx, g.val)
    H = synth.features(g.n, K, 11)
    write_order(tmp_path / "ord", *order)
    write_f32(tmp_path / "H", H)
    out = probe("run-single-s", tmp_path / "ord", tmp_path / "H", g.n, K, *SKEWED_COSTS, S,
                tmp_path / "C", env={"CWLB_TUNE_SCHEDULE": tune})
    last = out.strip().splitlines()[-1].split()
    rec = dict(zip(last[::2], last[1::2]))
    assert float(rec["average"]) > 0 and rec["samples"] == "50"
    m, sl, run_order, xcd = map(int, rec["schedule"].split(","))
    if tune == "0":
        assert (m, sl, run_order, xcd, rec["hints"], rec["occupancy"], rec["phases"],
                rec["tiling"]) == (0, 0, 0, 0, "0", "0", "0", "0")
    else:
        assert m in (0, 1, 2, 4, 8, 16, 32, 64) and sl in (0, 1, 2, 4)
        assert (run_order, xcd) in ((0, 0), (2, 1), (2, 2))
        assert int(rec["hints"]) in (0, 24 << 20, 48 << 20, 96 << 20)
        assert rec["occupancy"] in ("0", "6")
        assert rec["phases"] == "0"  # a 128 KB feature matrix: phases cannot pay
        assert rec["tiling"] in ("0", "2")
    assert len([ln for ln in out.splitlines() if ln.startswith("[Iteration ")]) == 50
    cap = capi.capacity_from_s(S, SKEWED_COSTS)
    tasks = oracle.partition(order[1], SKEWED_COSTS, cap)
    assert int(rec["tasks"]) == len(tasks)
    got = np.fromfile(tmp_path / "C", np.float32).reshape(g.n, K)
    ref32 = oracle.spmm_mean_f32(order[1], order[2], order[3], order[0], H, tasks)
    np.testing.assert_allclose(got, ref32, rtol=RTOL, atol=ATOL)


# ------------------------------------------------------------- executables
def cli_tree(tmp_path, g, costs=SKEWED_COSTS):
    build = tmp_path / "build"
    data = tmp_path / "resources" / "datasets"
    build.mkdir()
    data.mkdir(parents=True)
    text = ",".join(map(str, g.row_ptr)) + "\n" + ",".join(map(str, g.col_idx)) + "\n"
    (data / "g.csr").write_text(text)
    capi.save_costs(costs, tmp_path / "resources" / "spmm_costs.txt")
    return build


def run_exe(name, *args, cwd=None, stdin=""):
    r = subprocess.run([os.path.join(BIN, name), *map(str, args)], capture_output=True, text=True,
                       cwd=cwd, input=stdin, timeout=300)
    print(r.stdout[-3000:], r.stderr[-2000:], flush=True)
    return r


def test_cli_single_s_and_wave(tmp_path):
    g = workloads.small(4, seed=2)
    build = cli_tree(tmp_path, g)
    r = run_exe("cwlb-spmm", "g", 64, "--S", 8, cwd=build)
    assert r.returncode == 0
    lines = r.stdout.splitlines()
    assert sum(ln.startswith("[Warm-up ") for ln in lines) == 20
    assert sum(ln.startswith("[Iteration ") for ln in lines) == 50
    assert f"V: {g.n}, E: {g.nnz}" in r.stdout
    t = float([ln for ln in lines if ln.startswith("SpMM time: ")][0].split()[2])
    assert t > 0
    r = run_exe("cwlb-spmm", "g.csr", 64, 64, cwd=build)
    assert r.returncode == 0 and "Dataset: g.csr" in r.stdout


def test_cli_missing_cost_file(tmp_path):
    g = workloads.small(1)
    build = cli_tree(tmp_path, g)
    os.remove(tmp_path / "resources" / "spmm_costs.txt")
    r = run_exe("cwlb-spmm", "g", 32, "--S", 8, cwd=build)
    assert r.returncode == 1
    assert ("Cannot read microbenchmark cost file: ../resources/spmm_costs.txt. "
            "Run ./costWrite first.") in r.stderr


def test_cli_candidates_and_search(tmp_path):
    g = workloads.small(2, seed=3)
    build = cli_tree(tmp_path, g)
    r = run_exe("cwlb-spmm", "g", 32, "--candidates", cwd=build)
    assert r.returncode == 0
    assert "=== Candidate summary (SpMM kernel time, us) ===" in r.stdout
    assert "best_candidate=S" in r.stdout
    assert not (tmp_path / "resources" / "results.txt").exists()
    # declined search: nothing written
    r = run_exe("cwlb-spmm", "g", 32, "--candidate-search", 3, cwd=build, stdin="maybe\nno\n")
    assert r.returncode == 0
    assert "Please enter yes or no." in r.stdout
    assert "Search cancelled; results.txt unchanged." in r.stdout
    assert not (tmp_path / "resources" / "results.txt").exists()
    # EOF at the prompt is a cancellation too
    r = run_exe("cwlb-spmm", "g", 32, "--candidate-search", cwd=build, stdin="")
    assert r.returncode == 0 and "Search cancelled" in r.stdout
    # confirmed search: both blocks appended
    r = run_exe("cwlb-spmm", "g", 32, "--candidate-search", "--step", 5, cwd=build,
                stdin=" YES \n")
    assert r.returncode == 0
    assert "final_best_S=" in r.stdout and "Results appended to ../resources/results.txt" in r.stdout
    text = (tmp_path / "resources" / "results.txt").read_text().splitlines()
    assert text[0] == "cwlb-spmm-candidates\tg\t32"
    assert text[4] == "cwlb-spmm-candidate-search\tg\t32"
    plan = [ln for ln in r.stdout.splitlines() if ln.startswith("[Search plan] S values:")][0]
    assert len(text) == 5 + len(plan.split()[4:])


def test_cli_range_sweep(tmp_path):
    g = workloads.small(5)
    build = cli_tree(tmp_path, g)
    r = run_exe("cwlb-spmm", "g", 32, 2, 7, 2, cwd=build)
    assert r.returncode == 0
    text = (tmp_path / "resources" / "results.txt").read_text().splitlines()
    assert text[0] == "cwlb-spmm\tg\t32"
    assert [ln.split("\t")[0] for ln in text[1:]] == ["2", "4", "6"]
    assert "best_S=" in r.stdout


def test_cost_write_small(tmp_path):
    build = tmp_path / "build"
    build.mkdir()
    r = run_exe("costWrite", 64, 3, 8192, 16, 8, cwd=build)
    assert r.returncode == 0
    assert "Saved cost parameters to: ../resources/spmm_costs.txt" in r.stdout
    vals = [float(x) for x in (tmp_path / "resources" / "spmm_costs.txt").read_text().split()]
    assert len(vals) == 4 and all(v > 0 for v in vals)


# ------------------------------------------------------------ GPU partition
def device_partition(ctx, rp, costs, cap):
    import torch
    n = len(rp) - 1
    d_rp = dev(np.asarray(rp, np.int32))
    T = ctx.partition_device_count(d_rp, n, costs, cap)
    out = torch.full((max(T, 1), 4), -9, dtype=torch.int32, device="cuda")
    T2 = ctx.partition_device(d_rp, n, costs, cap, out, T)
    assert T2 == T
    return out.cpu().numpy()[:T]


@pytest.mark.parametrize("cfg", [1, 2, 3, 4, 5])
def test_device_partition_small(gpu_ctx, cfg):
    g = workloads.small(cfg)
    _, rp, _, _ = capi.reorder_by_degree(g.row_ptr, g.col_idx, g.val)
    for costs in (UNIT_COSTS, SKEWED_COSTS, (0.004519, 0.015617, 0.010667, 0.540499)):
        for S in workloads.candidate_s(g.nnz, 256) + [1, 3]:
            cap = capi.capacity_from_s(S, costs)
            got = device_partition(gpu_ctx, rp, costs, cap)
            assert np.array_equal(got, capi.partition(rp, costs, cap)), (cfg, costs, S)


@pytest.mark.parametrize("cfg", [2, 3, 4, 5])
def test_device_partition_full(gpu_ctx, cfg):
    """Full-size graphs at the three wave-based S (and the mesh's S sweep)
    with the gfx950 costs: task-for-task identical to the host partition,
    and SHA-256-identical to the reference partition's fixture
    (tests/golden/partition_golden.json)."""
    import time
    from test_golden import GOLDEN, sha
    rec = GOLDEN["full"][str(cfg)]
    g = workloads.graph(cfg)
    d_origin, d_rp, _, _ = reorder_on_device(gpu_ctx, g.row_ptr, g.col_idx, g.val)
    assert sha(d_origin) == rec["origin_sha256"] and sha(d_rp) == rec["sorted_row_ptr_sha256"]
    _, rp, _, _ = capi.reorder_by_degree(g.row_ptr, g.col_idx, g.val)
    assert np.array_equal(rp, d_rp)
    costs = GOLDEN["costs"]["gfx950"]
    for p in rec["partitions"]:
        S = p["S"]
        cap = capi.capacity_from_s(S, costs)
        assert cap == float.fromhex(p["capacity"])
        t0 = time.perf_counter()
        got = device_partition(gpu_ctx, rp, costs, cap)
        t1 = time.perf_counter()
        exp = capi.partition(rp, costs, cap)
        t2 = time.perf_counter()
        print(f"cfg={cfg} S={S} T={len(exp)} device {1e3 * (t1 - t0):.1f} ms (two calls) "
              f"host {1e3 * (t2 - t1):.1f} ms", flush=True)
        assert np.array_equal(got, exp)
        assert (len(got), sha(got)) == (p["n_tasks"], p["tasks_sha256"])


def test_device_partition_random_fixture(gpu_ctx):
    """The reference partition's random fixture cases (sorted and unsorted
    degree sequences, assorted costs) on the GPU partition; cases whose
    costs have no row bound are refused and stay with the host."""
    from test_golden import GOLDEN, random_case, sha
    ran = 0
    for c in GOLDEN["random"]:
        rp, costs, cap = random_case(c)
        try:
            got = device_partition(gpu_ctx, rp, costs, cap)
        except capi.CwlbError as e:
            assert e.status == capi.UNSUPPORTED
            continue
        assert (len(got), sha(got)) == (c["n_tasks"], c["tasks_sha256"]), c
        ran += 1
    print(f"random fixture cases on the GPU: {ran} of {len(GOLDEN['random'])}", flush=True)
    assert ran >= 40


def test_device_partition_random(gpu_ctx, rng):
    for trial in range(60):
        n = int(rng.integers(1, 3000))
        degs = rng.geometric(0.05, n) - 1
        if trial % 2:
            degs = np.sort(degs)
        degs[rng.random(n) < 0.3] = 0
        rp = np.concatenate([[0], np.cumsum(degs)]).astype(np.int32)
        costs = (UNIT_COSTS, SKEWED_COSTS)[trial % 2]
        S = int(rng.integers(1, 60))
        cap = capi.capacity_from_s(S, costs)
        assert np.array_equal(device_partition(gpu_ctx, rp, costs, cap),
                              capi.partition(rp, costs, cap)), (trial, S)


def test_device_partition_edge_cases(gpu_ctx):
    import torch
    # no rows
    assert gpu_ctx.partition_device_count(dev(np.zeros(1, np.int32)), 0, UNIT_COSTS, 4.5) == 0
    # one row, a single hub row, all rows empty
    for degs in ([0], [7], [100000], [0] * 500, [3, 0, 0, 9, 1000, 5]):
        rp = np.concatenate([[0], np.cumsum(degs)]).astype(np.int32)
        cap = capi.capacity_from_s(4, UNIT_COSTS)
        assert np.array_equal(device_partition(gpu_ctx, rp, UNIT_COSTS, cap),
                              capi.partition(rp, UNIT_COSTS, cap))
    # a buffer too small reports the count
    rp = np.concatenate([[0], np.cumsum([5] * 50)]).astype(np.int32)
    out = torch.zeros((2, 4), dtype=torch.int32, device="cuda")
    with pytest.raises(capi.CwlbError) as e:
        gpu_ctx.partition_device(dev(rp), 50, UNIT_COSTS, 4.5, out, 2)
    assert e.value.status == capi.INSUFFICIENT
    # costs with no bound on a task's row count stay with the host partition
    for costs in ((0.25, 0.75, 0.0, 0.5), (0.25, -0.75, 0.5, 0.5), (0.25, 0.75, 1e-9, 0.5)):
        with pytest.raises(capi.CwlbError) as e:
            gpu_ctx.partition_device_count(dev(rp), 50, costs, capi.capacity_from_s(4, costs))
        assert e.value.status == capi.UNSUPPORTED


@pytest.mark.parametrize("costs", [SKEWED_COSTS, (0.25, 0.75, 0.0, 0.5)], ids=["gpu", "host"])
def test_dropin_partition_hip(tmp_path, costs):
    """costWeightedTaskPartitioning_HIP: identical tasks, on the GPU or (for
    costs with C_store = 0) through the host partition."""
    g = workloads.small(4, seed=5)
    order = oracle.reorder_by_degree(g.row_ptr, g.col_idx, g.val)
    write_order(tmp_path / "ord", *order)
    for S in (1, 7, 40):
        probe("partition-gpu", tmp_path / "ord", *costs, S, tmp_path / "tasks")
        raw = open(tmp_path / "tasks", "rb").read()
        got = np.frombuffer(raw[8:], np.int32).reshape(-1, 4)
        cap = oracle.capacity_from_s(S, costs)
        assert np.array_equal(got, oracle.partition(order[1], costs, cap))
