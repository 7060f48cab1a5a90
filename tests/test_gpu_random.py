"""Seeded random cross-product of graph family, K, S, costs and launch
schedule (run length, feature slices, run order, XCD placement, cache hints,
occupancy variant, column phases, lane tiling, flags, feature-view
alignment) against the oracle.

The structured tests in test_gpu_spmm.py cover each setting on fixed graphs;
these cases draw combinations that no structured test names, with the same
bar: every output row within 1e-5 relative / 1e-6 absolute of the oracle in
the reference's value order, and the schedule the library reports for the
launch consistent with the settings.  The reference's kernel is
src/parallelMatrix.cpp:63-254 (K <= 1024) and :264-683 (larger K).
Further drawn cases go through the host-pointer entry (shuffled lists
included) and the allocation-free entry (drawn flags, run length, slices).
"""
import numpy as np
import pytest

import oracle
from conftest import SKEWED_COSTS, UNIT_COSTS
from cwlb_amd import capi, synth, workloads
from test_gpu_spmm import expected_tiling

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-5, 1e-6
N_CASES = 256
K_CHOICES = [1, 2, 3, 4, 7, 8, 12, 16, 31, 32, 48, 60, 64, 96, 100, 128, 200, 256, 300, 384,
             512, 600, 1024, 1028, 1100]


def draw_case(i):
    """The i-th case: a dict of every setting, reproducible from i alone."""
    r = np.random.default_rng(1000 + i)
    costs = [UNIT_COSTS, SKEWED_COSTS,
             tuple(float(x) for x in np.round(r.uniform(0.05, 4.0, 4), 3))][int(r.integers(3))]
    return {
        "family": int(r.integers(1, 6)),
        "seed": int(r.integers(1, 1 << 20)),
        "K": K_CHOICES[int(r.integers(len(K_CHOICES)))],
        "S": int(np.exp(r.uniform(0, np.log(400)))),
        "costs": costs,
        "M": [0, 1, 2, 3, 4, 7, 8, 16, 32, 64][int(r.integers(10))],
        "SL": [0, 1, 2, 4, 8][int(r.integers(5))],
        "order": int(r.integers(3)),
        "xcd": int(r.integers(3)),
        "hot_rows": [0, 0, 16, 256, 4096][int(r.integers(5))],
        "flags": [0, 0, 0, capi.ZERO_OUTPUT, capi.PER_TASK][int(r.integers(5))],
        "h_offset": [0, 0, 0, 1, 2][int(r.integers(5))],  # floats past the allocation start
        "occupancy": [0, 0, 6][int(r.integers(3))],
        # drawn from its own stream, so the other settings of a case do not
        # depend on it
        "phases": [0, 0, 2, 5, 16][int(np.random.default_rng(5000 + i).integers(5))],
        "keep_empty": bool(np.random.default_rng(7000 + i).integers(3) == 0),
        "tiling": [0, 0, 2][int(np.random.default_rng(9000 + i).integers(3))],
    }


def uncovered_rows(tasks, origin, n):
    """Output ids of the rows no task's row range covers (reordered row r
    is written to output row origin[r])."""
    cover = np.zeros(n + 1, np.int64)
    t = np.asarray(tasks, np.int64).reshape(-1, 4)
    np.add.at(cover, np.clip(t[:, 0], 0, n), 1)
    np.add.at(cover, np.clip(t[:, 1], 0, n), -1)
    return np.asarray(origin)[np.cumsum(cover[:n]) == 0]


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_schedule_case(gpu_ctx, i):
    import torch
    c = draw_case(i)
    print(f"case {i}: {c}", flush=True)
    g = workloads.small(c["family"], seed=c["seed"])
    K = c["K"]
    p = workloads.prepare(g, c["costs"], c["S"])
    H = synth.features(g.n, K, c["seed"] % 997)
    large_k = K > 1024

    d_rp = torch.from_numpy(p.row_ptr).cuda()
    d_ci = torch.from_numpy(p.col_idx).cuda()
    d_v = torch.from_numpy(p.val).cuda()
    d_o = torch.from_numpy(p.origin).cuda()
    d_t = torch.from_numpy(np.ascontiguousarray(p.tasks, np.int32).reshape(-1)).cuda()
    # A feature view starting h_offset floats past a 256-byte boundary.
    flat = torch.empty(g.n * K + 4, dtype=torch.float32, device="cuda")
    d_H = flat[c["h_offset"]:c["h_offset"] + g.n * K].view(g.n, K)
    d_H.copy_(torch.from_numpy(H))
    C = torch.full((g.n, K), float("nan"), dtype=torch.float32, device="cuda")

    gpu_ctx.set_schedule(c["M"], c["SL"])
    gpu_ctx.set_locality(c["order"], c["xcd"])
    gpu_ctx.set_cache_hints(c["hot_rows"] * 4 * K)
    gpu_ctx.set_occupancy(c["occupancy"])
    gpu_ctx.set_column_phases(c["phases"])
    gpu_ctx.set_lane_tiling(c["tiling"])
    flags = c["flags"] | (capi.KEEP_EMPTY_ROWS if c["keep_empty"] else 0)
    try:
        gpu_ctx.spmm(d_rp, d_ci, d_v, d_o, g.n, g.nnz, d_H, g.n, K, d_t, len(p.tasks), C,
                     flags=flags, large_k=large_k)
        info = gpu_ctx.last_launch()
    finally:
        gpu_ctx.set_schedule(0, 0)
        gpu_ctx.set_locality(0, 0)
        gpu_ctx.set_cache_hints(0)
        gpu_ctx.set_occupancy(0)
        gpu_ctx.set_column_phases(0)
        gpu_ctx.set_lane_tiling(0)

    ref = oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H, p.tasks)
    if not c["flags"] & capi.ZERO_OUTPUT:
        # Rows no task covers keep their contents.  The partition leaves out
        # the rows without nonzeros when their slot cost exceeds the capacity
        # (utils.cpp:972-976); the reference's cleared C holds 0 for them.
        ref[uncovered_rows(p.tasks, p.origin, g.n)] = np.nan
        if c["keep_empty"]:
            # Rows without nonzeros are left too (the reference's kernel
            # skips them, parallelMatrix.cpp:166).
            ref[p.origin[np.diff(p.row_ptr) == 0]] = np.nan
    np.testing.assert_allclose(C.cpu().numpy(), ref, rtol=RTOL, atol=ATOL, err_msg=str(c))

    per_task = bool(c["flags"] & capi.PER_TASK)
    if len(p.tasks) and K:
        assert info["grid_blocks"] > 0, info
    if per_task:
        assert (info["tasks_per_wave"], info["feature_slices"]) == (1, 1), info
        assert (info["run_order"], info["cache_hints"]) == (1, 0), info
    elif c["M"]:
        assert info["tasks_per_wave"] == c["M"], info
    if c["SL"] and not per_task:
        # Slices are whole 4-float vectors (as even as K allows): 16-byte
        # lanes and at least one vector per slice.
        sliced = info["vector_width"] == 4 and K // 4 >= c["SL"]
        assert info["feature_slices"] == (c["SL"] if sliced else 1), (info, c)
    if c["hot_rows"] == 0:
        assert info["cache_hints"] == 0, info
    if c["order"] != 2:
        assert info["run_order"] == 1, info
    expect_vec = 4 if K % 4 == 0 and c["h_offset"] % 4 == 0 else (
        2 if K % 2 == 0 and c["h_offset"] % 2 == 0 else 1)
    assert info["vector_width"] == expect_vec, info
    f4 = -(-(K // 4) // info["feature_slices"])  # vectors of the widest slice
    # Column phases: 16-byte lanes, at most 64 vectors per slice; they
    # replace the occupancy variant and the cache hints.
    phased = c["phases"] > 1 and not per_task and expect_vec == 4 and f4 <= 64
    assert info["column_phases"] == (c["phases"] if phased else 1), (info, c)
    o6 = (c["occupancy"] == 6 and not per_task and expect_vec == 4 and 2 < f4 <= 16
          and not phased)
    assert info["waves_per_simd"] == (6 if o6 else 0), (info, c)
    if phased:
        assert info["cache_hints"] == 0, (info, c)
    if K and len(p.tasks):
        packed = c["tiling"] == 2 and not per_task and expect_vec == 4 and not o6
        wide = info["cache_hints"] == 0 and info["column_phases"] == 1
        assert (info["slot_lanes"], info["lane_vectors"]) == expected_tiling(
            K, info["feature_slices"], packed, wide, vec=expect_vec), (info, c)


N_ENTRY_CASES = 64


def entry_case(i):
    """A drawn case's graph, prepared problem and features (seeds apart from
    the device-entry cases)."""
    c = draw_case(300000 + i)
    g = workloads.small(c["family"], seed=c["seed"])
    p = workloads.prepare(g, c["costs"], c["S"])
    H = synth.features(g.n, c["K"], c["seed"] % 997)
    return c, g, p, H


@pytest.mark.parametrize("i", range(N_ENTRY_CASES))
def test_random_host_entry_case(gpu_ctx, i):
    """The host-pointer entry (the drop-in spmmKernel): always the
    reference's zeroed C; a shuffled list (about a third of the cases) is
    run one task per wave, as it does not tile the nonzeros in order."""
    c, g, p, H = entry_case(i)
    r = np.random.default_rng(400000 + i)
    tasks = np.asarray(p.tasks, np.int32).reshape(-1, 4)
    if len(tasks) and r.random() < 0.3:
        tasks = tasks[r.permutation(len(tasks))]
    print(f"case {i}: {c} shuffled={not np.array_equal(tasks, p.tasks)}", flush=True)
    got, _ = gpu_ctx.spmm_host(p.row_ptr, p.col_idx, p.val, p.origin, H, tasks)
    ref = oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H, tasks)
    np.testing.assert_allclose(got, ref, rtol=RTOL, atol=ATOL, err_msg=str(c))


@pytest.mark.parametrize("i", range(N_ENTRY_CASES))
def test_random_noalloc_entry_case(gpu_ctx, i):
    """The allocation-free entry with drawn flags, run length and slices."""
    import torch
    c, g, p, H = entry_case(i)
    r = np.random.default_rng(500000 + i)
    flags = [0, capi.ZERO_OUTPUT, capi.PER_TASK, capi.KEEP_EMPTY_ROWS,
             capi.ZERO_OUTPUT | capi.KEEP_EMPTY_ROWS][int(r.integers(5))]
    m = [0, 1, 2, 8, 64][int(r.integers(5))]
    sl = [0, 1, 2, 4, 8][int(r.integers(5))]
    K = c["K"]
    print(f"case {i}: {c} flags={flags} m={m} sl={sl}", flush=True)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    tk = np.ascontiguousarray(p.tasks, np.int32).reshape(-1)
    C = torch.full((g.n, K), float("nan"), dtype=torch.float32, device="cuda")
    capi.spmm_noalloc(torch.cuda.current_stream().cuda_stream, dev(p.row_ptr), dev(p.col_idx),
                      dev(p.val), dev(p.origin), g.n, g.nnz, dev(H), g.n, K,
                      dev(tk if tk.size else np.zeros(4, np.int32)), len(p.tasks), C,
                      flags=flags, tasks_per_wave=m, feature_slices=sl)
    ref = oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H, p.tasks)
    if not flags & capi.ZERO_OUTPUT:
        ref[uncovered_rows(p.tasks, p.origin, g.n)] = np.nan
        if flags & capi.KEEP_EMPTY_ROWS:
            ref[p.origin[np.diff(p.row_ptr) == 0]] = np.nan
    np.testing.assert_allclose(C.cpu().numpy(), ref, rtol=RTOL, atol=ATOL, err_msg=str(c))
