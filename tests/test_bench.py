"""bench.py's host-side helpers (no GPU): the roofline record computed from
counter values, the counter CSV reader, the launch arguments handed to the
counter passes, the algorithmic / compulsory byte formulas, and the check of
the timed launch's C against the oracle (on CPU tensors, with planted
mistakes in C)."""
import importlib
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def bench():
    sys.path.insert(0, ROOT)
    return importlib.import_module("bench")


KERNEL = ("void cwlb::(anonymous namespace)::spmm_mean_runs<4, 16, 1, 8, 2, true, false>"
          "(int const*, int const*, float const*, int const*, int, long long, ...)")


def counters(fetch_kib, write_kib, probe_fetch_kib, probe_write_kib, hits=1.0, misses=3.0,
             occ=17.5):
    return {"kernel": {"FETCH_SIZE": fetch_kib, "WRITE_SIZE": write_kib, "TCC_HIT_sum": hits,
                       "TCC_MISS_sum": misses, "MeanOccupancyPerCU": occ},
            "copy": {"FETCH_SIZE": probe_fetch_kib, "WRITE_SIZE": probe_write_kib},
            "name": KERNEL, "dispatches": 4}


def test_roofline_from_counters(bench):
    """achieved = algorithmic bytes / kernel time, frac = achieved / 8 TB/s
    (36 GB in 4 ms: 9 TB/s, 1.125); traffic_frac = (FETCH x read scale +
    WRITE x write scale) / kernel time / 8 TB/s, with the scales from the
    1 GiB copy (24 GB in 4 ms: 6 TB/s = 0.75); the compulsory rate beside."""
    probe_kib = 1 << 20  # 1 GiB
    # FETCH_SIZE reads half of the copy's bytes: read scale 2; WRITE exact.
    c = counters(fetch_kib=10e9 / 1024 / 2, write_kib=14e9 / 1024, probe_fetch_kib=probe_kib / 2,
                 probe_write_kib=probe_kib)
    rec = bench.roofline_record(c, None, b_alg=36e9, b_min=4.8e9, main_us=4000.0,
                                launched={"max_waves_per_cu": 28})
    assert rec["traffic"] == pytest.approx(24e9)
    assert rec["traffic_read"] == pytest.approx(10e9) and rec["traffic_write"] == pytest.approx(14e9)
    assert rec["traffic_gbs"] == pytest.approx(6000.0) and rec["traffic_frac"] == pytest.approx(0.75)
    assert rec["traffic_frac"] == pytest.approx(rec["traffic"] / (rec["kernel_us"] * 1e-6) / 8e12)
    assert rec["achieved"] == pytest.approx(9000.0) and rec["frac"] == pytest.approx(1.125)
    assert rec["frac"] == pytest.approx(rec["algorithmic_bytes"] / (rec["kernel_us"] * 1e-6) / 8e12)
    assert rec["compulsory_gbs"] == pytest.approx(1200.0)
    assert rec["compulsory_frac"] == pytest.approx(0.15)
    assert rec["l2_hit_rate"] == pytest.approx(0.25)
    assert rec["waves_per_cu"] == 17.5 and rec["max_waves_per_cu"] == 28
    assert rec["kernel"] == "spmm_mean_runs<4,16,1,8,2,true,false>"
    assert rec["counters"]["fetch_scale"] == pytest.approx(2.0)
    assert (rec["bound"], rec["unit"], rec["peak"]) == ("hbm", "GB/s", 8000.0)


def test_roofline_without_counters(bench):
    rec = bench.roofline_record(None, "rocprofv3 not found", 36e9, 4.8e9, 4000.0, {})
    assert rec["traffic"] is None and rec["traffic_frac"] is None and rec["traffic_gbs"] is None
    assert rec["counters_error"] == "rocprofv3 not found"
    assert rec["achieved"] == pytest.approx(9000.0) and rec["frac"] == pytest.approx(1.125)


def test_counter_csv_reader(bench, tmp_path):
    """Rows grouped per (kernel, counter) in dispatch order."""
    path = tmp_path / "run_counter_collection.csv"
    path.write_text(
        "Correlation_Id,Dispatch_Id,Agent_Id,Queue_Id,Process_Id,Thread_Id,Grid_Size,Kernel_Id,"
        "Kernel_Name,Workgroup_Size,LDS_Block_Size,Scratch_Size,VGPR_Count,Accum_VGPR_Count,"
        "SGPR_Count,Counter_Name,Counter_Value,Start_Timestamp,End_Timestamp\n"
        f'3,3,1,1,9,9,4096,7,"{KERNEL}",256,0,0,72,0,96,FETCH_SIZE,30.0,0,1\n'
        f'1,1,1,1,9,9,4096,7,"{KERNEL}",256,0,0,72,0,96,FETCH_SIZE,10.0,0,1\n'
        '2,2,1,1,9,9,4096,8,"__amd_rocclr_copyBuffer",256,0,0,8,0,16,FETCH_SIZE,5.0,0,1\n'
        '4,4,1,1,9,9,4096,8,"__amd_rocclr_copyBuffer",256,0,0,8,0,16,FETCH_SIZE,7.0,0,1\n')
    vals = bench.read_counter_csv(str(path))
    assert vals[(KERNEL, "FETCH_SIZE")] == [10.0, 30.0]
    assert vals[("__amd_rocclr_copyBuffer", "FETCH_SIZE")] == [5.0, 7.0]


def test_schedule_args_fix_the_launch(bench):
    sched = {"tasks_per_wave": 64, "feature_slices": 2, "run_order": 0, "xcd_blocks": 0,
             "hot_bytes": 48 << 20, "occupancy": 0}
    args = bench.schedule_args(63, sched)
    assert args == ["--s", "63", "--tasks-per-wave", "64", "--slices", "2", "--run-order", "0",
                    "--xcd-blocks", "0", "--hot-mb", "48", "--occupancy", "0", "--phases", "0",
                    "--tiling", "0"]
    sched["phases"] = 16
    sched["tiling"] = 2
    assert bench.schedule_args(63, sched)[-4:] == ["--phases", "16", "--tiling", "2"]


def test_counters_per_call(bench):
    """A call of P column phases dispatches the kernel P times: traffic and
    L2 accesses add up over them, the occupancy is a mean."""
    assert bench.per_call_value("FETCH_SIZE", [10.0, 30.0], 16) == pytest.approx(320.0)
    assert bench.per_call_value("TCC_MISS_sum", [4.0], 3) == pytest.approx(12.0)
    assert bench.per_call_value("MeanOccupancyPerCU", [10.0, 30.0], 16) == pytest.approx(20.0)
    assert bench.per_call_value("WRITE_SIZE", [5.0, 7.0], 1) == pytest.approx(6.0)


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True)
    assert r.returncode == 2 and "one GPU only" in r.stderr


def test_algorithmic_bytes_formula():
    """4(N+1) + 8 nnz + 4 nnz K + 4 N K + 4 N + 16 T, the per-unit figures
    stated next to the roofline: 8 B + 4K B per nonzero, 4 B + 4K B + 4 B per
    row, 16 B per task."""
    from cwlb_amd import workloads
    n, nnz, K, T = 7, 11, 3, 5
    assert workloads.algorithmic_bytes(n, nnz, K, T) == (
        4 * (n + 1) + 8 * nnz + 4 * nnz * K + 4 * n * K + 4 * n + 16 * T)
    assert workloads.algorithmic_bytes(4194304, 65245138, 128, 1084009) == 36125853988


def test_compulsory_bytes_formula():
    """CSR once, each referenced feature row once, C once: the R-MAT bound
    with every row referenced is 4.85 GB (CSR, H and C once each)."""
    from cwlb_amd import workloads
    n, nnz, K = 4194304, 65245138, 128
    b = workloads.compulsory_bytes(n, n, nnz, K)
    assert b == 4 * (n + 1) + 8 * nnz + 4 * n * K + 4 * n * K + 4 * n
    assert 4.8e9 < b < 4.9e9


def _parity_case(K):
    """A small graph, its task list and the oracle's output at width K."""
    import numpy as np

    import oracle
    from cwlb_amd import synth, workloads
    g = workloads.small(4, seed=7)
    p = workloads.prepare(g, (0.125, 1.375, 0.75, 3.5), S=8)
    H = synth.features(g.n, K, 11)
    ref = oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H, p.tasks)
    return p, H, ref


@pytest.mark.parametrize("cols", [256, 7])
def test_parity_check_accepts_the_oracle_output(bench, monkeypatch, cols):
    """The bench's own check of the timed launch (whole C against the oracle,
    in blocks of feature columns) passes on the sequential oracle's output,
    also when the columns fall into several blocks."""
    import torch
    monkeypatch.setattr(bench, "PARITY_COLS", cols)
    p, H, ref = _parity_case(20)
    rec = bench.parity_check(torch, torch.from_numpy(ref.copy()), torch.from_numpy(H), p.row_ptr,
                             p.col_idx, p.val, p.origin, p.tasks, 2)
    assert rec["ok"] and rec["max_excess"] <= 0.0 and rec["nan_rows"] == 0
    assert rec["elements"] == ref.size


@pytest.mark.parametrize("plant", ["offset", "nan", "zero_row"])
def test_parity_check_rejects_a_wrong_c(bench, monkeypatch, plant):
    """A C off by a few ulps beyond the tolerance in one element of the last
    column block, a NaN, or one aggregated row left at zero fails the check."""
    import numpy as np
    import torch
    monkeypatch.setattr(bench, "PARITY_COLS", 8)
    p, H, ref = _parity_case(20)
    bad = ref.copy()
    deg = np.diff(p.row_ptr)[np.argsort(p.origin)]
    r = int(np.flatnonzero(deg > 0)[3])
    if plant == "offset":
        bad[r, 19] += 2e-6 + 2e-5 * abs(bad[r, 19])
    elif plant == "nan":
        bad[r, 19] = np.nan
    else:
        bad[r, :] = 0.0
    rec = bench.parity_check(torch, torch.from_numpy(bad), torch.from_numpy(H), p.row_ptr,
                             p.col_idx, p.val, p.origin, p.tasks, 2)
    assert not rec["ok"], rec
