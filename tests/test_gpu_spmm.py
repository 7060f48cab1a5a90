"""GPU parity of the HIP mean-aggregation SpMM against the oracle.

Every case runs the C ABI (libcwlb.so) on an MI355X and compares with
  * oracle.spmm_mean_f32: the reference kernel's value order
    (parallelMatrix.cpp:148-236) on the CPU, and
  * oracle.spmm_mean_f64: the closed form (A H)[i] / deg(i) on the original
    CSR, independent of the permutation and the partition.
Tolerance (from the parity contract): |gpu - ref| <= 1e-6 + 1e-5 * |ref|
per element.  Full-size configurations are checked on the whole of C
against the OpenMP form of the reference-order oracle (the large-K widths in
blocks of feature columns, since each column aggregates independently), and
through properties: all-ones features give exactly 1 (unit values) or 0
(degree-0 rows), and sampled rows match the fp64 closed form.
"""
import subprocess
import sys
import textwrap

import numpy as np
import pytest

import oracle
from conftest import PKG, ROOT, SKEWED_COSTS, UNIT_COSTS
from cwlb_amd import capi, paths, synth, workloads

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-5, 1e-6


def torch_mod():
    import torch
    return torch


def dev(a, dtype=None):
    torch = torch_mod()
    a = np.ascontiguousarray(a)
    if a.size == 0:
        a = np.zeros(1, a.dtype if dtype is None else dtype)
    return torch.from_numpy(a).cuda()


def run_gpu(ctx, p, H, flags=0, c_fill=float("nan"), large_k=False, h_dev=None):
    """Runs the device-pointer SpMM on prepared problem p; returns (C, timing)."""
    torch = torch_mod()
    K = H.shape[1] if H is not None else h_dev.shape[1]
    h_rows = H.shape[0] if H is not None else h_dev.shape[0]
    d_rp, d_ci, d_v, d_o = dev(p.row_ptr), dev(p.col_idx), dev(p.val), dev(p.origin)
    d_t = dev(np.ascontiguousarray(p.tasks, np.int32).reshape(-1))
    d_H = dev(H) if h_dev is None else h_dev
    C = torch.full((max(p.n, 1), max(K, 1)), c_fill, dtype=torch.float32, device="cuda")
    t = ctx.spmm(d_rp, d_ci, d_v, d_o, p.n, p.nnz, d_H, h_rows, K, d_t, len(p.tasks), C,
                 flags=flags, large_k=large_k)
    return C[:p.n, :K].cpu().numpy(), t


# (tasks_per_wave, feature_slices, flags, run_order, xcd_blocks, hot_bytes,
# waves_per_simd): automatic, the reference's one task per wave, forced
# task-run fusion / XCD feature slicing (small graphs do not trigger them
# automatically), runs sorted by output row, contiguous XCD stretches, cache
# hints (hot sets of 64 KB / 256 KB of feature rows: a few hundred hot
# columns, the rest cold, on these small graphs) and the 6-waves-per-SIMD
# kernel variant (it applies where a feature slice has 9 to 64 floats).
SCHEDULES = [(0, 0, 0, 0, 0, 0, 0), (0, 0, capi.PER_TASK, 0, 0, 0, 0), (3, 1, 0, 1, 1, 0, 0),
             (8, 2, 0, 1, 1, 0, 0), (16, 4, 0, 1, 1, 0, 0), (64, 4, 0, 1, 1, 0, 0),
             (2, 1, 0, 2, 1, 0, 0), (5, 1, 0, 1, 2, 0, 0), (8, 4, 0, 2, 2, 0, 0),
             (1, 2, 0, 2, 2, 0, 0), (0, 0, 0, 0, 0, 1 << 16, 0), (8, 2, 0, 1, 1, 1 << 18, 0),
             (2, 1, 0, 2, 2, 1 << 16, 0), (0, 0, capi.PER_TASK, 0, 0, 1 << 16, 0),
             (0, 0, 0, 0, 0, 0, 6), (3, 2, 0, 2, 2, 0, 6), (8, 1, 0, 1, 1, 1 << 16, 6)]
SCHED_IDS = ["auto", "per_task", "m3", "m8s2", "m16s4", "m64s4", "m2ord", "m5xcd", "m8s4ordxcd",
             "m1s2ordxcd", "hints64k", "m8s2_hints256k", "m2ordxcd_hints64k", "per_task_hints",
             "occ6", "m3s2ordxcd_occ6", "m8_hints64k_occ6"]


@pytest.fixture(params=SCHEDULES, ids=SCHED_IDS)
def sched(request, gpu_ctx):
    m, sl, flags, order, xcd, hot, occ = request.param
    gpu_ctx.set_schedule(m, sl)
    gpu_ctx.set_locality(order, xcd)
    gpu_ctx.set_cache_hints(hot)
    gpu_ctx.set_occupancy(occ)
    yield flags
    gpu_ctx.set_schedule(0, 0)
    gpu_ctx.set_locality(0, 0)
    gpu_ctx.set_cache_hints(0)
    gpu_ctx.set_occupancy(0)


def check(got, ref):
    np.testing.assert_allclose(got, ref, rtol=RTOL, atol=ATOL)


def problem(g, costs, S):
    return workloads.prepare(g, costs, S)


def oracle_pair(p, g, H):
    ref32 = oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H, p.tasks)
    ref64 = oracle.spmm_mean_f64(g.row_ptr, g.col_idx, g.val, H)
    return ref32, ref64


def custom_graph(rp, ci, val=None):
    rp = np.asarray(rp, np.int32)
    ci = np.asarray(ci, np.int32)
    val = np.ones(len(ci), np.float32) if val is None else np.asarray(val, np.float32)
    return synth.Graph(len(rp) - 1, rp, ci, val)


# --------------------------------------------------------------- small configs
@pytest.mark.parametrize("cfg", [1, 2, 3, 4, 5])
@pytest.mark.parametrize("which", [0, 1, 2])
def test_small_config_candidates(gpu_ctx, sched, cfg, which):
    """Each configuration family at reduced size, at the three wave-based S."""
    g = workloads.small(cfg)
    K = workloads.FEATURE_DIM[cfg]
    S = workloads.candidate_s(g.nnz, 256)[which]
    p = problem(g, SKEWED_COSTS, S)
    H = synth.features(g.n, K, workloads.FEATURE_SEED)
    print(f"cfg={cfg} S={S} n={g.n} nnz={g.nnz} tasks={len(p.tasks)}", flush=True)
    got, t = run_gpu(gpu_ctx, p, H, flags=sched)
    ref32, ref64 = oracle_pair(p, g, H)
    check(got, ref32)
    check(got, ref64)
    assert t.total_us > 0


@pytest.mark.parametrize("S", [1, 2, 3, 7, 32, 1000])
def test_small_rmat_segment_sizes(gpu_ctx, sched, S):
    """Heavy splitting (S=1) through no splitting (S=1000) on a skewed graph."""
    g = workloads.small(4, seed=11)
    H = synth.features(g.n, 128, 7)
    p = problem(g, UNIT_COSTS, S)
    got, _ = run_gpu(gpu_ctx, p, H, flags=sched)
    ref32, ref64 = oracle_pair(p, g, H)
    check(got, ref32)
    check(got, ref64)


def test_config1_full(gpu_ctx):
    """The CPU plumbing configuration at full size (N=4,096, K=32)."""
    g = workloads.graph(1)
    H = synth.features(g.n, 32, workloads.FEATURE_SEED)
    for S in workloads.candidate_s(g.nnz, 256):
        p = problem(g, SKEWED_COSTS, S)
        got, _ = run_gpu(gpu_ctx, p, H)
        ref32, ref64 = oracle_pair(p, g, H)
        check(got, ref32)
        check(got, ref64)


def test_config2_full(gpu_ctx):
    """Chung-Lu N=1M K=64 at full size against the full CPU oracle."""
    g = workloads.graph(2)
    H = synth.features(g.n, 64, workloads.FEATURE_SEED)
    S = workloads.candidate_s(g.nnz, 256)[0]
    p = problem(g, SKEWED_COSTS, S)
    got, _ = run_gpu(gpu_ctx, p, H)
    ref32 = oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H, p.tasks)
    check(got, ref32)


# ------------------------------------------------------ full-size properties
def features_rows(rows, K, seed):
    """Host restatement of the feature generator for selected rows (numpy uint64)."""
    def mix64(z):
        z = z + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))
    with np.errstate(over="ignore"):
        s = mix64(np.uint64(seed))
        idx = (np.asarray(rows, np.uint64)[:, None] * np.uint64(K)
               + np.arange(K, dtype=np.uint64)[None, :])
        x = mix64(s + idx)
    u = (x >> np.uint64(40)).astype(np.int64) - 8388608
    return (u.astype(np.float32) * np.float32(2.0**-23)).astype(np.float32)


def sampled_rows_check(g, C_dev, H_host, rng, n_sample=3000):
    """Compare sampled rows (random + highest degree) with the fp64 closed form."""
    torch = torch_mod()
    deg = np.diff(g.row_ptr)
    top = np.argsort(deg, kind="stable")[-200:]
    rows = np.unique(np.concatenate([rng.integers(0, g.n, n_sample), top]))
    got = C_dev[torch.from_numpy(rows).cuda()].cpu().numpy()
    exp = np.zeros((len(rows), H_host.shape[1]), np.float64)
    for i, r in enumerate(rows):
        lo, hi = g.row_ptr[r], g.row_ptr[r + 1]
        if hi > lo:
            vals = g.val[lo:hi].astype(np.float64)
            exp[i] = (vals[:, None] * H_host[g.col_idx[lo:hi]].astype(np.float64)).sum(0) / (hi - lo)
    np.testing.assert_allclose(got, exp, rtol=RTOL, atol=ATOL)


def split_rows(p):
    """Reordered rows that some task covers only partly."""
    t = np.asarray(p.tasks, np.int64).reshape(-1, 4)
    deg = np.diff(p.row_ptr).astype(np.int64)
    rs, re, fo, ln = t[:, 0], t[:, 1], t[:, 2], t[:, 3]
    single = re - rs == 1
    first = (fo > 0) | (single & (ln > 0) & (ln < deg[rs]))
    last = (~single) & (ln > 0) & (ln < deg[re - 1])
    return np.unique(np.concatenate([rs[first], re[last] - 1]))


def tasks_per_row(p):
    """Number of tasks that touch each reordered row."""
    t = np.asarray(p.tasks, np.int64).reshape(-1, 4)
    cnt = np.zeros(p.n + 1, np.int64)
    np.add.at(cnt, t[:, 0], 1)
    np.add.at(cnt, t[:, 1], -1)
    return np.cumsum(cnt)[:-1]


@pytest.mark.parametrize("cfg", [3, 4, 5])
@pytest.mark.parametrize("per_task", [False, True], ids=["auto", "per_task"])
def test_full_config_properties(gpu_ctx, cfg, per_task):
    torch = torch_mod()
    flags = capi.PER_TASK if per_task else 0
    g = workloads.graph(cfg)
    K = workloads.FEATURE_DIM[cfg]
    S = workloads.candidate_s(g.nnz, 256)[0]
    p = problem(g, SKEWED_COSTS, S)
    print(f"cfg={cfg} n={g.n} nnz={g.nnz} K={K} S={S} tasks={len(p.tasks)}", flush=True)
    d_rp, d_ci, d_v, d_o = dev(p.row_ptr), dev(p.col_idx), dev(p.val), dev(p.origin)
    d_t = dev(np.ascontiguousarray(p.tasks, np.int32).reshape(-1))
    C = torch.full((g.n, K), float("nan"), dtype=torch.float32, device="cuda")
    # All-ones features: rows that no task splits average to exactly 1 (or
    # 0 without edges).  A split row sums per-segment means in float, as the
    # reference's atomics do; on hub rows with thousands of equal segment
    # means that drifts from 1 by more than the parity tolerance, in the
    # reference as much as here, so split rows are held to the rounding
    # bound (touching tasks + 1) * 2^-23, which the reference-order oracle
    # must meet too.
    ones = torch.ones((g.n, K), dtype=torch.float32, device="cuda")
    gpu_ctx.spmm(d_rp, d_ci, d_v, d_o, g.n, g.nnz, ones, g.n, K, d_t, len(p.tasks), C,
                 flags=flags)
    del ones
    got = C.cpu().numpy()
    touch = np.zeros(g.n, np.int64)
    touch[p.origin] = tasks_per_row(p)
    split = np.zeros(g.n, bool)
    split[p.origin[split_rows(p)]] = True
    deg = np.diff(g.row_ptr)
    exact = np.where(deg > 0, 1.0, 0.0).astype(np.float32)
    assert np.array_equal(got[~split], np.broadcast_to(exact[~split, None], got[~split].shape))
    bound = (touch[split] + 1) * 2.0**-23
    assert np.all(np.abs(got[split] - 1.0) <= bound[:, None])
    ref1 = oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin,
                                np.ones((g.n, 1), np.float32), p.tasks)
    assert np.all(np.abs(ref1[split, 0] - 1.0) <= bound)
    if per_task:
        np.testing.assert_allclose(got, np.broadcast_to(ref1, got.shape), rtol=RTOL, atol=ATOL)
    del got
    # Seeded U[-1,1) features: sampled rows against the fp64 closed form.
    H = torch.empty((g.n, K), dtype=torch.float32, device="cuda")
    gpu_ctx.fill_features(H, g.n, K, workloads.FEATURE_SEED)
    C.fill_(float("nan"))
    t = gpu_ctx.spmm(d_rp, d_ci, d_v, d_o, g.n, g.nnz, H, g.n, K, d_t, len(p.tasks), C,
                     flags=flags)
    assert not torch.isnan(C).any().item()
    H_host = synth.features(g.n, K, workloads.FEATURE_SEED)
    sampled_rows_check(g, C, H_host, np.random.default_rng(cfg))
    print(f"cfg={cfg} total_us={t.total_us:.1f} zero_us={t.zero_us:.1f}", flush=True)


def _whole_c_vs_oracle_in_column_blocks(torch, C, H, p, what, cols=1024):
    """The whole of C against the reference-order oracle, one block of
    feature columns at a time: mean aggregation is independent per column,
    so the oracle on columns j0:j1 of H (copied back from the device) is the
    oracle's value for those columns of C.  Keeps host buffers at n x cols."""
    K = C.shape[1]
    for j0 in range(0, K, cols):
        j1 = min(K, j0 + cols)
        Hb = np.ascontiguousarray(H[:, j0:j1].cpu().numpy())
        ref = oracle.spmm_mean_f32_omp(p.row_ptr, p.col_idx, p.val, p.origin, Hb, p.tasks)
        del Hb
        ref_dev = torch.from_numpy(ref).cuda()
        del ref
        _assert_close_on_device(torch, C[:, j0:j1], ref_dev, f"{what} columns {j0}:{j1}")
        del ref_dev


@pytest.mark.parametrize("K", [1028, 4096])
def test_full_chunglu_large_k_vs_oracle(gpu_ctx, K):
    """The large-K entry (K above the 1,024-lane work-group limit) on the
    full-size Chung-Lu graph (1M rows, 9.1M nonzeros; H and C of 4-16 GB):
    all-ones features give exactly 1 (0 for empty rows) on rows no task
    splits and stay within the rounding bound on split rows; with seeded
    features the whole of C matches the reference-order oracle
    (parallelMatrix.cpp:148-236) at 1e-5 relative / 1e-6 absolute, checked
    in blocks of 1,024 feature columns."""
    torch = torch_mod()
    g = workloads.graph(2)
    S = workloads.candidate_s(g.nnz, 256)[2]
    p = problem(g, SKEWED_COSTS, S)
    print(f"K={K} n={g.n} nnz={g.nnz} S={S} tasks={len(p.tasks)}", flush=True)
    d_rp, d_ci, d_v, d_o = dev(p.row_ptr), dev(p.col_idx), dev(p.val), dev(p.origin)
    d_t = dev(np.ascontiguousarray(p.tasks, np.int32).reshape(-1))
    C = torch.full((g.n, K), float("nan"), dtype=torch.float32, device="cuda")
    ones = torch.ones((g.n, K), dtype=torch.float32, device="cuda")
    gpu_ctx.spmm(d_rp, d_ci, d_v, d_o, g.n, g.nnz, ones, g.n, K, d_t, len(p.tasks), C,
                 large_k=True)
    del ones
    touch = np.zeros(g.n, np.int64)
    touch[p.origin] = tasks_per_row(p)
    split = np.zeros(g.n, bool)
    split[p.origin[split_rows(p)]] = True
    deg = np.diff(g.row_ptr)
    exact = torch.from_numpy(np.where(deg > 0, 1.0, 0.0).astype(np.float32)).cuda()
    whole = torch.from_numpy(~split).cuda()
    assert bool((C[whole] == exact[whole, None]).all().item())
    bound = torch.from_numpy(((touch + 1) * 2.0**-23).astype(np.float32)).cuda()
    sp = torch.from_numpy(split).cuda()
    assert bool(((C[sp] - 1.0).abs() <= bound[sp, None]).all().item())
    del whole, sp
    H = torch.empty((g.n, K), dtype=torch.float32, device="cuda")
    gpu_ctx.fill_features(H, g.n, K, workloads.FEATURE_SEED)
    C.fill_(float("nan"))
    t = gpu_ctx.spmm(d_rp, d_ci, d_v, d_o, g.n, g.nnz, H, g.n, K, d_t, len(p.tasks), C,
                     large_k=True)
    print(f"K={K} total_us={t.total_us:.1f}", flush=True)
    _whole_c_vs_oracle_in_column_blocks(torch, C, H, p, f"chunglu K={K} S={S}")


# ------------------------------------------------------------------ edge cases
@pytest.mark.parametrize("K", [1, 2, 3, 4, 6, 12, 20, 36, 64, 100, 128, 192, 256, 260, 512, 600,
                               1000, 1024])
@pytest.mark.parametrize("m,sl", [(1, 1), (8, 2), (8, 4), (4, 8)])
def test_feature_widths(gpu_ctx, K, m, sl):
    g = workloads.small(4, seed=3)
    H = synth.features(g.n, K, 5)
    p = problem(g, SKEWED_COSTS, 8)
    gpu_ctx.set_schedule(m, sl)
    try:
        got, _ = run_gpu(gpu_ctx, p, H)
    finally:
        gpu_ctx.set_schedule(0, 0)
    ref32, ref64 = oracle_pair(p, g, H)
    check(got, ref32)
    check(got, ref64)


@pytest.mark.parametrize("K", [1025, 1100, 2052, 4100])
def test_large_k_entry(gpu_ctx, K):
    """K above the work-group limit goes through the large-K entry point."""
    g = workloads.small(1, seed=9)
    H = synth.features(g.n, K, 5)
    p = problem(g, UNIT_COSTS, 5)
    got, _ = run_gpu(gpu_ctx, p, H, large_k=True)
    ref32, ref64 = oracle_pair(p, g, H)
    check(got, ref32)
    check(got, ref64)
    with pytest.raises(capi.CwlbError) as e:
        run_gpu(gpu_ctx, p, H, large_k=False)
    assert e.value.status == capi.INVALID_ARG


def expected_tiling(K, SL, packed, wide, vec=4):
    """(slot lanes G, vectors per lane R) of a K-float row in SL slices of
    vec-float vectors: the restatement of cwlb_ctx_set_lane_tiling's rule
    (packed slots take 16-byte lanes only)."""
    F = -(-(K // vec) // SL)
    if F <= 64:
        G, R = 1 << max(0, (F - 1).bit_length()), 1
    else:
        G, R = 64, (min(-(-F // 64), 8) if SL == 1 else 1)
    if not packed:
        return G, R

    def key(g, r):
        passes = -(-F // (g * r))
        return passes, passes * g * r, r
    if F <= 64:
        cands = [(g, r) for g, r in ((4, 3), (4, 5), (8, 3), (8, 5), (16, 3)) if g * r >= F]
    elif wide:
        cands = [(g, r) for g, r in ((16, 5), (32, 3), (32, 5), (64, 3), (64, 5))
                 if g < 64 or SL == 1]
    else:
        cands = []
    for g, r in cands:
        if key(g, r) < key(G, R):
            G, R = g, r
    return G, R


def test_expected_tiling_examples():
    """The packed tilings the kernel's slices get: K = 96 in 8 x 3, K = 600 in
    4 slices (38 vectors) in 8 x 5, in 8 slices (19) in 4 x 5, in 2 slices
    (75) in 16 x 5 and in one (150) in 32 x 5; power-of-two widths keep
    one vector per lane."""
    assert expected_tiling(96, 1, True, True) == (8, 3)
    assert expected_tiling(96, 1, False, True) == (32, 1)
    assert expected_tiling(600, 4, True, True) == (8, 5)
    assert expected_tiling(600, 8, True, True) == (4, 5)
    assert expected_tiling(600, 2, True, True) == (16, 5)
    assert expected_tiling(600, 1, True, True) == (32, 5)
    assert expected_tiling(600, 1, False, True) == (64, 3)
    assert expected_tiling(600, 4, True, False) == (8, 5)  # hints and phases: one pass
    assert expected_tiling(2052, 1, True, True) == (64, 5)  # 513 vectors: 2 x 320, not 2 x 512
    assert expected_tiling(128, 2, True, True) == (16, 1)
    assert expected_tiling(64, 1, True, True) == (16, 1)


# (K, feature slices, variant): widths whose slices the packed tiling
# covers with fewer idle lanes (and power-of-two ones it leaves), with
# slices, cache hints and column phases.
PACKED_CASES = [(K, sl, v) for K in (12, 20, 36, 48, 96, 100, 152, 300, 600, 1000)
                for sl in (1, 2, 4, 8) for v in ("plain", "hints", "phases")
                if K // 4 >= sl]
_PACKED = {}


def _packed_problem(K):
    """The graph, task list, features and oracle results of width K (kept
    for the cases of one K, which run one after the other)."""
    if K not in _PACKED:
        _PACKED.clear()
        g = workloads.small(4, seed=5)
        H = synth.features(g.n, K, 7)
        p = problem(g, SKEWED_COSTS, 8)
        _PACKED[K] = (g, H, p, oracle_pair(p, g, H))
    return _PACKED[K]


@pytest.mark.parametrize("K,sl,variant", PACKED_CASES)
def test_packed_lane_tiling(gpu_ctx, K, sl, variant):
    """Packed slots (cwlb_ctx_set_lane_tiling(2)) against the oracle in
    reference order and the fp64 closed form, with the tiling the launch
    reports checked against the rule's restatement."""
    g, H, p, (ref32, ref64) = _packed_problem(K)
    gpu_ctx.set_schedule(8, sl)
    gpu_ctx.set_lane_tiling(2)
    gpu_ctx.set_cache_hints(1 << 16 if variant == "hints" else 0)
    gpu_ctx.set_column_phases(5 if variant == "phases" else 0)
    try:
        got, _ = run_gpu(gpu_ctx, p, H)
        info = gpu_ctx.last_launch()
    finally:
        gpu_ctx.set_schedule(0, 0)
        gpu_ctx.set_lane_tiling(0)
        gpu_ctx.set_cache_hints(0)
        gpu_ctx.set_column_phases(0)
    wide = info["cache_hints"] == 0 and info["column_phases"] == 1
    assert (info["slot_lanes"], info["lane_vectors"]) == expected_tiling(K, sl, True, wide), info
    if variant == "phases" and -(-(K // 4) // sl) <= 64:
        assert info["column_phases"] == 5, info
    check(got, ref32)
    check(got, ref64)


@pytest.mark.parametrize("K", [1100, 2052, 4100])
def test_packed_lane_tiling_large_k(gpu_ctx, K):
    """The large-K entry with packed slots (K = 2,052: 513 vectors in two
    passes of 64 x 5 instead of 64 x 8)."""
    g = workloads.small(1, seed=9)
    H = synth.features(g.n, K, 5)
    p = problem(g, UNIT_COSTS, 5)
    gpu_ctx.set_lane_tiling(2)
    try:
        got, _ = run_gpu(gpu_ctx, p, H, large_k=True)
        info = gpu_ctx.last_launch()
    finally:
        gpu_ctx.set_lane_tiling(0)
    assert (info["slot_lanes"], info["lane_vectors"]) == expected_tiling(
        K, info["feature_slices"], True, True), info
    ref32, ref64 = oracle_pair(p, g, H)
    check(got, ref32)
    check(got, ref64)


def test_lane_tiling_argument(gpu_ctx):
    for bad in (-1, 3):
        with pytest.raises(capi.CwlbError) as e:
            gpu_ctx.set_lane_tiling(bad)
        assert e.value.status == capi.INVALID_ARG
    gpu_ctx.set_lane_tiling(1)
    assert gpu_ctx.lane_tiling() == 1
    gpu_ctx.set_lane_tiling(0)


def test_large_k_entry_rejects_small_k(gpu_ctx):
    g = workloads.small(1, seed=9)
    H = synth.features(g.n, 64, 5)
    p = problem(g, UNIT_COSTS, 5)
    with pytest.raises(capi.CwlbError) as e:
        run_gpu(gpu_ctx, p, H, large_k=True)
    assert e.value.status == capi.INVALID_ARG


def test_hub_row_and_empty_rows(gpu_ctx, sched, rng):
    """One row of degree 5,000 among degree-0 and degree-1 rows, tiny S."""
    n = 6000
    deg = np.zeros(n, np.int64)
    deg[17] = 5000
    deg[rng.integers(0, n, 300)] = 1
    rp = np.concatenate([[0], np.cumsum(deg)]).astype(np.int32)
    ci = rng.integers(0, n, rp[-1]).astype(np.int32)
    val = rng.uniform(-2, 2, rp[-1]).astype(np.float32)
    g = custom_graph(rp, ci, val)
    H = synth.features(n, 64, 1)
    for S in (1, 2, 3, 64, 4999, 5000, 6000):
        p = problem(g, UNIT_COSTS, S)
        got, _ = run_gpu(gpu_ctx, p, H, flags=sched)
        ref32, ref64 = oracle_pair(p, g, H)
        check(got, ref32)
        check(got, ref64)


def test_all_rows_empty(gpu_ctx):
    n = 1000
    g = custom_graph(np.zeros(n + 1, np.int32), np.zeros(0, np.int32))
    H = synth.features(n, 32, 1)
    p = problem(g, UNIT_COSTS, 4)
    got, _ = run_gpu(gpu_ctx, p, H)
    assert np.array_equal(got, np.zeros((n, 32), np.float32))


def test_duplicate_columns_and_values(gpu_ctx, sched, rng):
    """Repeated columns inside a row and non-unit values."""
    n = 3000
    deg = rng.integers(0, 40, n)
    rp = np.concatenate([[0], np.cumsum(deg)]).astype(np.int32)
    ci = rng.integers(0, 50, rp[-1]).astype(np.int32)
    val = rng.normal(size=rp[-1]).astype(np.float32)
    g = custom_graph(rp, ci, val)
    H = synth.features(n, 64, 3)
    for S in (2, 5, 17):
        p = problem(g, SKEWED_COSTS, S)
        got, _ = run_gpu(gpu_ctx, p, H, flags=sched)
        ref32, ref64 = oracle_pair(p, g, H)
        check(got, ref32)
        check(got, ref64)


@pytest.mark.parametrize("K", [16, 32, 64])
@pytest.mark.parametrize("d", [1, 2, 3, 5, 8, 9, 16, 31])
def test_short_row_windows_bit_exact(gpu_ctx, sched, K, d, rng):
    """Groups of short rows whose nonzeros fit the 64-entry register window,
    the per-wave LDS window (up to 256) or neither (per-lane loads).  Every
    row is whole; rows shorter than 16 nonzeros run row-per-slot under every
    schedule, are summed in CSR order and match the oracle bit for bit
    (longer rows may take the all-slots path, whose shuffle reduction
    regroups the sum)."""
    n = 3000
    deg = rng.integers(max(d - 2, 0), d + 1, n)
    rp = np.concatenate([[0], np.cumsum(deg)]).astype(np.int32)
    ci = rng.integers(0, n, rp[-1]).astype(np.int32)
    val = rng.uniform(-2, 2, rp[-1]).astype(np.float32)
    g = custom_graph(rp, ci, val)
    H = synth.features(n, K, d)
    p = problem(g, UNIT_COSTS, 100000)
    got, _ = run_gpu(gpu_ctx, p, H, flags=sched)
    ref32 = oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H, p.tasks)
    short = deg < 16
    assert np.array_equal(got[short], ref32[short])
    check(got, ref32)


def test_unsorted_graph_custom_tasks(gpu_ctx, rng):
    """Caller-made task lists: one task per row, and whole-graph tasks."""
    g = workloads.small(2, seed=5)
    H = synth.features(g.n, 32, 3)
    origin, rp, ci, val = capi.reorder_by_degree(g.row_ptr, g.col_idx, g.val)
    base = workloads.Prepared(g.n, g.nnz, origin, rp, ci, val, None, 0, 0.0)
    per_row = np.stack([np.arange(g.n), np.arange(1, g.n + 1), np.zeros(g.n), np.zeros(g.n)],
                       1).astype(np.int32)
    whole = np.array([[0, g.n, 0, 0]], np.int32)
    for tasks in (per_row, whole):
        base.tasks = tasks
        got, _ = run_gpu(gpu_ctx, base, H)
        ref32 = oracle.spmm_mean_f32(rp, ci, val, origin, H, tasks)
        check(got, ref32)


def big_random_graph(n, max_deg, seed):
    rng = np.random.default_rng(seed)
    deg = rng.integers(0, max_deg + 1, n)
    rp = np.concatenate([[0], np.cumsum(deg)]).astype(np.int32)
    ci = rng.integers(0, n, rp[-1]).astype(np.int32)
    val = rng.uniform(-1, 1, rp[-1]).astype(np.float32)
    return custom_graph(rp, ci, val)


@pytest.mark.parametrize("order", ["shuffled", "reversed", "in_order"])
def test_many_per_row_tasks_in_any_order(gpu_ctx, order):
    """200,000 one-row tasks, in task order, reversed and shuffled: enough
    tasks that the automatic schedule runs several tasks per wave.  Runs of
    tasks that do not continue one another execute task by task, so every
    order gives the reference's result (the rows no longer neighbour each
    other, and a run taken as one range would compute other rows)."""
    g = big_random_graph(200_000, 12, 21)
    H = synth.features(g.n, 32, 3)
    origin, rp, ci, val = capi.reorder_by_degree(g.row_ptr, g.col_idx, g.val)
    base = workloads.Prepared(g.n, g.nnz, origin, rp, ci, val, None, 0, 0.0)
    per_row = np.stack([np.arange(g.n), np.arange(1, g.n + 1), np.zeros(g.n), np.zeros(g.n)],
                       1).astype(np.int32)
    if order == "shuffled":
        per_row = per_row[np.random.default_rng(5).permutation(g.n)]
    elif order == "reversed":
        per_row = per_row[::-1].copy()
    base.tasks = per_row
    got, _ = run_gpu(gpu_ctx, base, H)
    assert gpu_ctx.last_launch()["tasks_per_wave"] > 1
    check(got, oracle.spmm_mean_f32(rp, ci, val, origin, H, per_row))
    check(got, oracle.spmm_mean_f64(g.row_ptr, g.col_idx, g.val, H))


@pytest.mark.parametrize("how", ["shuffled", "swapped_pairs", "gaps"])
@pytest.mark.parametrize("m", [0, 64, 5, 130])
def test_partition_list_out_of_order(gpu_ctx, how, m):
    """The partition's task list (split rows included) shuffled, with pairs
    of neighbours swapped, or with a fifth of the tasks dropped, at the
    automatic run length and at 64, 5 and 130 tasks per wave (a run of
    three 64-task windows): with the full clear
    of CWLB_SPMM_ZERO_OUTPUT the result is the reference's for that list."""
    rng = np.random.default_rng(len(how) + m)
    g = workloads.small(4, seed=23)
    H = synth.features(g.n, 64, 8)
    p = problem(g, SKEWED_COSTS, 3)
    t = p.tasks.copy()
    if how == "shuffled":
        t = t[rng.permutation(len(t))]
    elif how == "swapped_pairs":
        idx = np.arange(len(t))
        sw = rng.choice(len(t) // 2, len(t) // 8, replace=False) * 2
        idx[sw], idx[sw + 1] = sw + 1, sw
        t = t[idx]
    else:
        t = t[rng.random(len(t)) > 0.2]
    p.tasks = np.ascontiguousarray(t)
    gpu_ctx.set_schedule(m, 0)
    try:
        got, _ = run_gpu(gpu_ctx, p, H, flags=capi.ZERO_OUTPUT)
    finally:
        gpu_ctx.set_schedule(0, 0)
    check(got, oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H, p.tasks))
    if how != "gaps":
        # Every row's first nonzero is in the list: without the full clear
        # the clearing pass alone defines every row (C starts as NaN).
        gpu_ctx.set_schedule(m, 0)
        try:
            got, _ = run_gpu(gpu_ctx, p, H)
        finally:
            gpu_ctx.set_schedule(0, 0)
        check(got, oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H, p.tasks))


@pytest.mark.parametrize("bad", ["decreasing", "beyond_nnz", "negative"])
def test_malformed_row_offsets_are_reported(gpu_ctx, bad):
    """Row offsets that decrease, pass nnz or are negative are met on the
    device without any access outside the arrays and reported as
    CWLB_INVALID_ARG; a good call afterwards clears the report."""
    g = workloads.small(1, seed=2)
    H = synth.features(g.n, 32, 3)
    p = problem(g, UNIT_COSTS, 6)
    rp = p.row_ptr.copy()
    r = len(rp) // 2
    if bad == "decreasing":
        rp[r] = rp[r + 1] + 3
    elif bad == "beyond_nnz":
        rp[-1] = p.nnz + 100
    else:
        rp[r] = -5
    good = p.row_ptr
    p.row_ptr = rp
    with pytest.raises(capi.CwlbError) as e:
        run_gpu(gpu_ctx, p, H)
    assert e.value.status == capi.INVALID_ARG
    assert b"row_ptr" in capi.lib().cwlb_last_error()
    p.row_ptr = good
    got, _ = run_gpu(gpu_ctx, p, H)
    check(got, oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H, p.tasks))


def test_zero_output_flag_with_partial_cover(gpu_ctx):
    """ZERO_OUTPUT reproduces the reference's zeroed C for rows no task touches."""
    g = workloads.small(1, seed=2)
    H = synth.features(g.n, 32, 3)
    p = problem(g, UNIT_COSTS, 6)
    p.tasks = p.tasks[: len(p.tasks) // 2].copy()
    got, _ = run_gpu(gpu_ctx, p, H, flags=capi.ZERO_OUTPUT)
    ref32 = oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H, p.tasks)
    check(got, ref32)


@pytest.mark.parametrize("phases", [0, 3])
@pytest.mark.parametrize("K", [32, 128, 1100])
def test_keep_empty_rows_flag(gpu_ctx, sched, K, phases, rng):
    """KEEP_EMPTY_ROWS leaves the rows without nonzeros as they were (the
    reference's kernel skips them, parallelMatrix.cpp:166, and its C starts
    cleared, :112); every other row gets the reference's result.  Without
    the flag they are stored as zeros; with ZERO_OUTPUT (alone or with it)
    they are the call's cleared 0.  About 60% of the rows are empty, among
    rows of degree 1 to 3 and a hub row split over many tasks."""
    n = 5000
    deg = rng.integers(1, 4, n) * (rng.random(n) < 0.4)
    deg[11] = 3000
    rp = np.concatenate([[0], np.cumsum(deg)]).astype(np.int32)
    ci = rng.integers(0, n, rp[-1]).astype(np.int32)
    val = rng.uniform(-2, 2, rp[-1]).astype(np.float32)
    g = custom_graph(rp, ci, val)
    H = synth.features(n, K, 2)
    p = problem(g, UNIT_COSTS, 8)
    ref32 = oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H, p.tasks)
    empty = p.origin[np.diff(p.row_ptr) == 0]
    assert 0 < len(empty) < n
    written = np.ones(n, bool)
    written[empty] = False
    large_k = K > 1024
    gpu_ctx.set_column_phases(phases)
    try:
        got, _ = run_gpu(gpu_ctx, p, H, flags=sched | capi.KEEP_EMPTY_ROWS, large_k=large_k)
        assert np.isnan(got[empty]).all()
        check(got[written], ref32[written])
        for f in (capi.ZERO_OUTPUT, capi.ZERO_OUTPUT | capi.KEEP_EMPTY_ROWS, 0):
            got, _ = run_gpu(gpu_ctx, p, H, flags=sched | f, large_k=large_k)
            check(got, ref32)
    finally:
        gpu_ctx.set_column_phases(0)


def test_unknown_flag_bits_are_rejected(gpu_ctx):
    """Flag bits beyond the three defined are an argument error on the
    context entry and on the allocation-free entry; nothing is written."""
    import torch
    g = workloads.small(1, seed=4)
    p = problem(g, UNIT_COSTS, 6)
    H = synth.features(g.n, 32, 2)
    d = [dev(x) for x in (p.row_ptr, p.col_idx, p.val, p.origin, H,
                          np.ascontiguousarray(p.tasks, np.int32).reshape(-1))]
    C = torch.full((g.n, 32), float("nan"), dtype=torch.float32, device="cuda")
    for bit in (0x8, 0x80000000):
        with pytest.raises(capi.CwlbError) as e:
            gpu_ctx.spmm(d[0], d[1], d[2], d[3], g.n, g.nnz, d[4], g.n, 32, d[5], len(p.tasks), C,
                         flags=bit | capi.ZERO_OUTPUT)
        assert e.value.status == capi.INVALID_ARG and "flag" in str(e.value)
        with pytest.raises(capi.CwlbError) as e:
            capi.spmm_noalloc(torch.cuda.current_stream().cuda_stream, d[0], d[1], d[2], d[3], g.n,
                              g.nnz, d[4], g.n, 32, d[5], len(p.tasks), C, flags=bit)
        assert e.value.status == capi.INVALID_ARG and "flag" in str(e.value)
    assert torch.isnan(C).all()
    got, _ = run_gpu(gpu_ctx, p, H, flags=capi.ZERO_OUTPUT | capi.PER_TASK | capi.KEEP_EMPTY_ROWS)
    check(got, oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H, p.tasks))


def test_library_loaded_before_torch():
    """A fresh process that calls the library's host functions before it
    imports torch still gets a working context.  torch's own HIP runtime
    shares ROCm's sonames; had it been loaded after this library, the
    process would hold two runtimes and the second to initialise would find
    no device.  The binding imports torch before it loads the library."""
    code = textwrap.dedent(f"""
        import sys
        sys.path[:0] = [{ROOT!r}, {PKG!r}]
        import numpy as np
        import oracle
        from cwlb_amd import capi, synth, workloads
        assert "torch" not in sys.modules
        g = workloads.small(1, seed=3)
        p = workloads.prepare(g, {UNIT_COSTS!r}, 6)  # host calls load the library
        import torch
        H = synth.features(g.n, 32, 1)
        dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
        C = torch.full((g.n, 32), float("nan"), device="cuda")
        ctx = capi.Context(0, torch.cuda.current_stream().cuda_stream)
        ctx.spmm(dev(p.row_ptr), dev(p.col_idx), dev(p.val), dev(p.origin), g.n, g.nnz,
                 dev(H), g.n, 32, dev(p.tasks.reshape(-1)), len(p.tasks), C)
        ref = oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H, p.tasks)
        np.testing.assert_allclose(C.cpu().numpy(), ref, rtol={RTOL!r}, atol={ATOL!r})
        ctx.close()
        print("OK", flush=True)
    """)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=240)
    assert r.returncode == 0 and "OK" in r.stdout, r.stdout[-2000:] + r.stderr[-2000:]


def test_launch_grid_limit(gpu_ctx):
    """70M empty tasks: one task per wave (or a fixed run length of 1) would
    need more than 2^32 work-items and is refused before any launch; the
    automatic run length fits."""
    torch = torch_mod()
    T = 70_000_000
    tasks = torch.zeros(T * 4, dtype=torch.int32, device="cuda")
    rp = dev(np.zeros(2, np.int32))
    ci, val = dev(np.zeros(1, np.int32)), dev(np.zeros(1, np.float32))
    origin = dev(np.zeros(1, np.int32))
    H = torch.ones((1, 32), dtype=torch.float32, device="cuda")
    C = torch.full((1, 32), 7.0, dtype=torch.float32, device="cuda")
    args = (rp, ci, val, origin, 1, 0, H, 1, 32, tasks, T, C)
    with pytest.raises(capi.CwlbError) as e:
        gpu_ctx.spmm(*args, flags=capi.PER_TASK)
    assert e.value.status == capi.UNSUPPORTED
    gpu_ctx.set_schedule(1, 1)
    try:
        with pytest.raises(capi.CwlbError) as e:
            gpu_ctx.spmm(*args)
        assert e.value.status == capi.UNSUPPORTED
    finally:
        gpu_ctx.set_schedule(0, 0)
    assert torch.all(C == 7.0)  # nothing ran
    gpu_ctx.spmm(*args, flags=capi.ZERO_OUTPUT)
    assert torch.all(C == 0.0)


def test_no_tasks_and_zero_k(gpu_ctx):
    g = workloads.small(1, seed=2)
    H = synth.features(g.n, 32, 3)
    p = problem(g, UNIT_COSTS, 6)
    p.tasks = np.zeros((0, 4), np.int32)
    got, t = run_gpu(gpu_ctx, p, H, flags=capi.ZERO_OUTPUT)
    assert np.array_equal(got, np.zeros_like(got))
    assert t.total_us == 0.0
    p2 = problem(g, UNIT_COSTS, 6)
    got, t = run_gpu(gpu_ctx, p2, np.zeros((g.n, 0), np.float32))
    assert got.shape == (g.n, 0) and t.total_us == 0.0


def test_empty_graph(gpu_ctx):
    g = custom_graph(np.zeros(1, np.int32), np.zeros(0, np.int32))
    p = problem(g, UNIT_COSTS, 4)
    assert len(p.tasks) == 0
    got, t = run_gpu(gpu_ctx, p, np.zeros((0, 8), np.float32))
    assert got.shape == (0, 8)


def test_bad_column_index_is_reported(gpu_ctx):
    """An out-of-range column is skipped on the device and reported."""
    g = workloads.small(1, seed=2)
    H = synth.features(g.n, 32, 3)
    p = problem(g, UNIT_COSTS, 6)
    p.col_idx = p.col_idx.copy()
    p.col_idx[len(p.col_idx) // 2] = g.n + 5
    with pytest.raises(capi.CwlbError) as e:
        run_gpu(gpu_ctx, p, H)
    assert e.value.status == capi.INVALID_ARG


def test_host_pointer_entry(gpu_ctx):
    g = workloads.small(4, seed=8)
    H = synth.features(g.n, 128, 3)
    p = problem(g, SKEWED_COSTS, 16)
    got, t = gpu_ctx.spmm_host(p.row_ptr, p.col_idx, p.val, p.origin, H, p.tasks)
    ref32, ref64 = oracle_pair(p, g, H)
    check(got, ref32)
    check(got, ref64)
    assert t.main_us > 0


def test_host_pointer_entry_overlapping_and_shuffled_tasks(gpu_ctx):
    """The host-pointer entry (the drop-in spmmKernel) takes any task list:
    the partition twice over (every nonzero covered twice: whole rows are
    stored twice, split rows receive both sets of partial sums) and the
    partition shuffled both give the reference's task-at-a-time result."""
    g = workloads.small(4, seed=8)
    H = synth.features(g.n, 64, 3)
    p = problem(g, SKEWED_COSTS, 5)
    rng = np.random.default_rng(2)
    for tasks in (np.concatenate([p.tasks, p.tasks]), p.tasks[rng.permutation(len(p.tasks))]):
        tasks = np.ascontiguousarray(tasks)
        got, _ = gpu_ctx.spmm_host(p.row_ptr, p.col_idx, p.val, p.origin, H, tasks)
        check(got, oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H, tasks))


def test_host_pointer_entry_multi_chunk(gpu_ctx):
    """Inputs and output larger than one 64 MiB staging buffer (H and C of
    about 160 MB each: several chunks through both buffers), then a small
    call on the same context."""
    g = workloads.small(2, seed=4)
    K = 2048
    H = synth.features(g.n, K, 6)
    p = problem(g, SKEWED_COSTS, 32)
    got, _ = gpu_ctx.spmm_host(p.row_ptr, p.col_idx, p.val, p.origin, H, p.tasks)
    ref32 = oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H, p.tasks)
    check(got, ref32)
    g2 = workloads.small(1, seed=4)
    H2 = synth.features(g2.n, 32, 6)
    p2 = problem(g2, UNIT_COSTS, 8)
    got2, _ = gpu_ctx.spmm_host(p2.row_ptr, p2.col_idx, p2.val, p2.origin, H2, p2.tasks)
    check(got2, oracle.spmm_mean_f32(p2.row_ptr, p2.col_idx, p2.val, p2.origin, H2, p2.tasks))


@pytest.mark.parametrize("K", [64, 128, 600])
@pytest.mark.parametrize("h_off,c_off", [(1, 0), (2, 2), (0, 1), (3, 2)])
def test_misaligned_feature_and_output_pointers(gpu_ctx, K, h_off, c_off):
    """H and C handed over as views that start 4 or 8 bytes past a 16-byte
    boundary: the kernel falls back to 8- or 4-byte lanes and still matches
    the oracle, also with the full clear of CWLB_SPMM_ZERO_OUTPUT (single
    floats up to the first 16-byte boundary); the floats around the output
    view are left untouched."""
    torch = torch_mod()
    g = workloads.small(4, seed=21)
    H = synth.features(g.n, K, 4)
    p = problem(g, SKEWED_COSTS, 24)
    d_rp, d_ci, d_v, d_o = dev(p.row_ptr), dev(p.col_idx), dev(p.val), dev(p.origin)
    d_t = dev(np.ascontiguousarray(p.tasks, np.int32).reshape(-1))
    h_buf = torch.zeros(g.n * K + 8, dtype=torch.float32, device="cuda")
    h_buf[h_off:h_off + g.n * K] = torch.from_numpy(H.reshape(-1)).cuda()
    d_H = h_buf[h_off:h_off + g.n * K].view(g.n, K)
    c_buf = torch.full((g.n * K + 8,), -5.0, dtype=torch.float32, device="cuda")
    d_C = c_buf[c_off:c_off + g.n * K].view(g.n, K)
    ref32, ref64 = oracle_pair(p, g, H)
    for flags in (0, capi.ZERO_OUTPUT):
        c_buf.fill_(-5.0)
        gpu_ctx.spmm(d_rp, d_ci, d_v, d_o, g.n, g.nnz, d_H, g.n, K, d_t, len(p.tasks), d_C,
                     flags=flags)
        got = d_C.cpu().numpy()
        check(got, ref32)
        check(got, ref64)
        rest = torch.cat([c_buf[:c_off], c_buf[c_off + g.n * K:]]).cpu().numpy()
        assert np.all(rest == -5.0)


@pytest.mark.parametrize("K", [32, 128])
def test_nan_and_inf_features_propagate(gpu_ctx, K):
    """Non-finite features propagate as in the reference's fma sums: a row
    that gathers a NaN (or both infinities) gives NaN, one that gathers
    +Inf only gives +Inf, and rows that gather neither stay finite and
    match the oracle."""
    g = workloads.small(4, seed=17)
    H = synth.features(g.n, K, 8)
    rng = np.random.default_rng(K)
    H[rng.choice(g.n, 20, replace=False), rng.integers(0, K, 20)] = np.nan
    H[rng.choice(g.n, 20, replace=False), rng.integers(0, K, 20)] = np.inf
    H[rng.choice(g.n, 20, replace=False), rng.integers(0, K, 20)] = -np.inf
    for S in (4, 1000):
        p = problem(g, UNIT_COSTS, S)
        got, _ = run_gpu(gpu_ctx, p, H)
        ref32 = oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H, p.tasks)
        assert np.array_equal(np.isnan(got), np.isnan(ref32))
        assert np.array_equal(np.isposinf(got), np.isposinf(ref32))
        assert np.array_equal(np.isneginf(got), np.isneginf(ref32))
        fin = np.isfinite(ref32)
        np.testing.assert_allclose(got[fin], ref32[fin], rtol=RTOL, atol=ATOL)
        assert np.isnan(got).any() and np.isposinf(got).any()


@pytest.mark.parametrize("K", [32, 64, 128, 256])
def test_cache_hints_change_no_value(gpu_ctx, K):
    """Hot sets from a handful of columns to all of them: every result equals
    the unhinted one (full rows bit for bit, split rows within tolerance) and
    the oracle."""
    torch = torch_mod()
    g = workloads.small(4, seed=41)
    H = synth.features(g.n, K, 12)
    p = problem(g, SKEWED_COSTS, 16)
    d_rp, d_ci, d_v, d_o = dev(p.row_ptr), dev(p.col_idx), dev(p.val), dev(p.origin)
    d_t = dev(np.ascontiguousarray(p.tasks, np.int32).reshape(-1))
    d_H = dev(H)
    C0 = torch.full((g.n, K), float("nan"), dtype=torch.float32, device="cuda")
    gpu_ctx.spmm(d_rp, d_ci, d_v, d_o, g.n, g.nnz, d_H, g.n, K, d_t, len(p.tasks), C0)
    ref32 = oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H, p.tasks)
    whole = np.ones(g.n, bool)
    whole[p.origin[split_rows(p)]] = False
    C1 = torch.full_like(C0, float("nan"))
    try:
        for hot in (4 * K, 64 * 4 * K, 1024 * 4 * K, g.n * 4 * K):
            for m, sl in ((0, 0), (4, 2), (1, 1)):
                gpu_ctx.set_schedule(m, sl)
                gpu_ctx.set_cache_hints(hot)
                C1.fill_(float("nan"))
                gpu_ctx.spmm(d_rp, d_ci, d_v, d_o, g.n, g.nnz, d_H, g.n, K, d_t, len(p.tasks), C1)
                # every hot set but the one holding all columns leaves cold ones
                assert gpu_ctx.last_launch()["cache_hints"] == int(hot < g.n * 4 * K), (hot, m, sl)
                got = C1.cpu().numpy()
                check(got, ref32)
                if (m, sl) == (0, 0):
                    assert np.array_equal(got[whole], C0.cpu().numpy()[whole]), hot
    finally:
        gpu_ctx.set_schedule(0, 0)
        gpu_ctx.set_cache_hints(0)


def test_cache_hints_left_over_from_other_columns(gpu_ctx):
    """Hints built for one column array stay in use after the caller rewrites
    that array in place (same pointer and length): only the cache policy can
    be off, the results follow the new columns.  A bad column index is still
    reported with hints on."""
    torch = torch_mod()
    g = workloads.small(4, seed=43)
    K = 64
    H = synth.features(g.n, K, 13)
    p = problem(g, UNIT_COSTS, 16)
    d_rp, d_ci, d_v, d_o = dev(p.row_ptr), dev(p.col_idx), dev(p.val), dev(p.origin)
    d_t = dev(np.ascontiguousarray(p.tasks, np.int32).reshape(-1))
    d_H = dev(H)
    C = torch.full((g.n, K), float("nan"), dtype=torch.float32, device="cuda")
    gpu_ctx.set_cache_hints(64 * 4 * K)
    try:
        gpu_ctx.spmm(d_rp, d_ci, d_v, d_o, g.n, g.nnz, d_H, g.n, K, d_t, len(p.tasks), C)
        check(C.cpu().numpy(), oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H,
                                                    p.tasks))
        perm = np.random.default_rng(3).permutation(g.n).astype(np.int32)
        ci2 = perm[p.col_idx]
        d_ci.copy_(torch.from_numpy(ci2).cuda())
        C.fill_(float("nan"))
        gpu_ctx.spmm(d_rp, d_ci, d_v, d_o, g.n, g.nnz, d_H, g.n, K, d_t, len(p.tasks), C)
        check(C.cpu().numpy(), oracle.spmm_mean_f32(p.row_ptr, ci2, p.val, p.origin, H, p.tasks))
        bad = ci2.copy()
        bad[5] = -7
        d_ci.copy_(torch.from_numpy(bad).cuda())
        with pytest.raises(capi.CwlbError) as e:
            gpu_ctx.spmm(d_rp, d_ci, d_v, d_o, g.n, g.nnz, d_H, g.n, K, d_t, len(p.tasks), C)
        assert e.value.status == capi.INVALID_ARG
    finally:
        gpu_ctx.set_cache_hints(0)


def test_cache_hints_ignored_beyond_4gib(gpu_ctx):
    """A feature matrix of 4.3 GB (32-bit offsets do not reach its end): the
    hints are not used and the result is still correct."""
    torch = torch_mod()
    g = workloads.small(4, seed=44)
    K = 128
    h_rows = (1 << 32) // (4 * K) + 4096
    p = problem(g, UNIT_COSTS, 16)
    d_H = torch.empty((h_rows, K), dtype=torch.float32, device="cuda")
    gpu_ctx.fill_features(d_H, h_rows, K, 9)
    ci = (p.col_idx.astype(np.int64) * (h_rows // g.n)).astype(np.int32)
    H_used = d_H[torch.from_numpy(np.arange(g.n) * (h_rows // g.n)).cuda()].cpu().numpy()
    d_rp, d_ci, d_v, d_o = dev(p.row_ptr), dev(ci), dev(p.val), dev(p.origin)
    d_t = dev(np.ascontiguousarray(p.tasks, np.int32).reshape(-1))
    C = torch.full((g.n, K), float("nan"), dtype=torch.float32, device="cuda")
    gpu_ctx.set_cache_hints(1 << 20)
    try:
        gpu_ctx.spmm(d_rp, d_ci, d_v, d_o, g.n, g.nnz, d_H, h_rows, K, d_t, len(p.tasks), C)
    finally:
        gpu_ctx.set_cache_hints(0)
    check(C.cpu().numpy(), oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H_used,
                                                p.tasks))


def test_cache_hints_argument(gpu_ctx):
    with pytest.raises(capi.CwlbError):
        gpu_ctx.set_cache_hints(-1)
    gpu_ctx.set_cache_hints(12345)
    assert gpu_ctx.cache_hints() == 12345
    gpu_ctx.set_cache_hints(0)


def test_two_contexts_on_two_threads(gpu_ctx):
    """Two contexts, each on its own (default-priority) stream and host
    thread, run different problems at the same time, one of them with runs
    sorted by output row and the host-pointer entry in between: each gets
    its own result, and an error on one thread does not leak into the other
    thread's last-error message."""
    import threading
    torch = torch_mod()
    probs = []
    for cfg, K, seed in ((4, 128, 31), (5, 32, 32)):
        g = workloads.small(cfg, seed=seed)
        H = synth.features(g.n, K, seed)
        p = problem(g, SKEWED_COSTS, 16)
        probs.append((g, H, p, K, oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin,
                                                         H, p.tasks)))
    errors, results = [], [None, None]

    def worker(i):
        try:
            g, H, p, K, ref = probs[i]
            stream = torch.cuda.Stream()
            ctx = capi.Context(0, stream.cuda_stream)
            if i == 1:
                ctx.set_locality(2, 2)
            with torch.cuda.stream(stream):
                d_rp, d_ci, d_v, d_o = dev(p.row_ptr), dev(p.col_idx), dev(p.val), dev(p.origin)
                d_t = dev(np.ascontiguousarray(p.tasks, np.int32).reshape(-1))
                d_H = dev(H)
                C = torch.full((g.n, K), float("nan"), dtype=torch.float32, device="cuda")
            stream.synchronize()
            for it in range(20):
                ctx.spmm(d_rp, d_ci, d_v, d_o, g.n, g.nnz, d_H, g.n, K, d_t, len(p.tasks), C)
                if it == 10:
                    got_h, _ = ctx.spmm_host(p.row_ptr, p.col_idx, p.val, p.origin, H, p.tasks)
                    np.testing.assert_allclose(got_h, ref, rtol=RTOL, atol=ATOL)
                if i == 0 and it == 5:
                    with pytest.raises(capi.CwlbError):
                        ctx.set_schedule(-1, 0)
            stream.synchronize()
            results[i] = C.cpu().numpy()
            ctx.close()
        except Exception as e:  # reported by the main thread
            errors.append((i, repr(e)))

    with pytest.raises(capi.CwlbError):
        gpu_ctx.set_locality(5, 0)  # this thread's last error: the run_order message
    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads)
    assert not errors, errors
    for i in range(2):
        check(results[i], probs[i][4])
    assert b"run_order" in capi.lib().cwlb_last_error()


def test_repeat_runs_stable(gpu_ctx):
    """Full rows are written identically on every run; split rows within tolerance."""
    g = workloads.small(4, seed=4)
    H = synth.features(g.n, 128, 3)
    p = problem(g, UNIT_COSTS, 4)
    a, _ = run_gpu(gpu_ctx, p, H)
    b, _ = run_gpu(gpu_ctx, p, H)
    check(a, b)


def test_device_features_match_host(gpu_ctx):
    torch = torch_mod()
    for rows, K in ((1000, 33), (257, 128), (1, 1)):
        H = torch.empty((rows, K), dtype=torch.float32, device="cuda")
        gpu_ctx.fill_features(H, rows, K, 42)
        assert np.array_equal(H.cpu().numpy(), synth.features(rows, K, 42))
        assert np.array_equal(features_rows(np.arange(rows), K, 42), synth.features(rows, K, 42))


def test_fresh_context_defaults_and_last_launch(gpu_ctx):
    """A new context starts with no cache hints, the standard kernel and an
    all-zero launch record; after a call the record names the launch."""
    torch = torch_mod()
    ctx = capi.Context(0, torch.cuda.current_stream().cuda_stream)
    try:
        assert ctx.cache_hints() == 0 and ctx.occupancy() == 0
        assert all(v == 0 for v in ctx.last_launch().values())
        g = workloads.small(1, seed=5)
        p = problem(g, UNIT_COSTS, 8)
        H = synth.features(g.n, 32, 1)
        got, _ = run_gpu(ctx, p, H)
        check(got, oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H, p.tasks))
        info = ctx.last_launch()
        assert info["grid_blocks"] > 0 and info["tasks_per_wave"] >= 1, info
        # 256-lane blocks: 4 to 32 waves per CU (8 per SIMD at most)
        assert 4 <= info["max_waves_per_cu"] <= 32 and info["max_waves_per_cu"] % 4 == 0, info
        assert (info["vector_width"], info["run_order"], info["cache_hints"],
                info["waves_per_simd"]) == (4, 1, 0, 0), info
    finally:
        ctx.close()


def test_schedule_and_locality_arguments(gpu_ctx):
    for bad in ((-1, 0), (0, 3), (0, 16), ((1 << 20) + 1, 0)):
        with pytest.raises(capi.CwlbError) as e:
            gpu_ctx.set_schedule(*bad)
        assert e.value.status == capi.INVALID_ARG
    gpu_ctx.set_schedule(1 << 20, 0)
    for bad in ((3, 0), (-1, 0), (0, 3), (0, -2)):
        with pytest.raises(capi.CwlbError) as e:
            gpu_ctx.set_locality(*bad)
        assert e.value.status == capi.INVALID_ARG
    for bad in (-1, 1, 5, 7, 8):
        with pytest.raises(capi.CwlbError) as e:
            gpu_ctx.set_occupancy(bad)
        assert e.value.status == capi.INVALID_ARG
    gpu_ctx.set_occupancy(6)
    assert gpu_ctx.occupancy() == 6
    gpu_ctx.set_schedule(0, 0)
    gpu_ctx.set_locality(0, 0)
    gpu_ctx.set_occupancy(0)


MB = 1 << 20
# Launch schedules checked at full size, per workload, as
# (segment-size candidate index, tasks per wave, feature slices, run order,
# XCD placement, hot-set bytes, waves per SIMD, flags[, column phases[, lane
# tiling]]);
# None = the schedule cwlb_ctx_tune_schedule picks, which is what bench.py
# times (bench.py also checks the whole C of its own timed launch).  The
# first R-MAT entries are headline launches of the benchmark (64 tasks per
# wave, 2 feature slices, 48 MB cache hints, the standard kernel) at every
# candidate S, and the launch a timed benchmark run kept at S = 125 (32 tasks
# per wave, 2 slices, 48 MB hints, automatic placement); the mesh entries
# are the launches its tuner kept
# (runs by output row, contiguous XCD stretches, the occupancy variant); the
# SBM's phased entries are its tuner's launches (12 phases, 8 slices; 16
# phases, 4 slices of packed 8 x 5 slots at S = 110) and other points of
# the phase sweep (16 phases, 4 slices, in task order; packed at S = 55),
# and its one-pass launch with packed 32 x 5 slots.
FULL_LAUNCHES = {
    4: [(0, 64, 2, 1, 1, 48 * MB, 0, 0), (2, 64, 2, 1, 1, 48 * MB, 0, 0),
        (2, 32, 2, 0, 0, 48 * MB, 0, 0), (2, None),
        (2, 64, 4, 1, 1, 0, 6, 0), (1, 64, 2, 1, 1, 48 * MB, 0, 0),
        (1, None), (1, 0, 0, 0, 0, 0, 0, 0), (1, 0, 0, 0, 0, 0, 0, capi.PER_TASK),
        (1, 4, 0, 2, 1, 0, 0, 0), (1, 8, 0, 2, 2, 0, 0, 0), (1, 32, 0, 1, 2, 0, 0, 0),
        (1, 8, 0, 2, 2, 96 * MB, 0, 0), (1, 2, 0, 2, 2, 0, 6, 0),
        (1, 64, 0, 1, 1, 48 * MB, 6, 0)],
    5: [(2, 1, 1, 2, 2, 0, 6, 0), (2, 2, 1, 2, 2, 0, 6, 0), (1, 4, 1, 2, 2, 0, 6, 0),
        (2, None), (2, 0, 0, 0, 0, 0, 0, 0), (2, 0, 0, 0, 0, 0, 0, capi.PER_TASK)],
    3: [(0, 64, 1, 2, 2, 0, 0, 0), (0, None), (0, 0, 0, 0, 0, 0, 0, 0), (2, 8, 1, 2, 2, 0, 0, 0),
        (1, 64, 8, 2, 2, 0, 0, 0, 12), (1, 16, 4, 1, 1, 0, 0, 0, 16),
        (1, 16, 4, 2, 2, 0, 0, 0, 16, 2), (0, 64, 4, 2, 2, 0, 0, 0, 16, 2),
        (0, 64, 1, 2, 2, 0, 0, 0, 0, 2)],
    2: [(1, 8, 1, 1, 1, 0, 6, 0), (1, None), (2, 0, 0, 0, 0, 0, 0, capi.PER_TASK)],
}


def _assert_close_on_device(torch, C, ref_dev, what):
    """|C - ref| <= 1e-6 + 1e-5 |ref| over the whole matrix, in row blocks."""
    worst = 0.0
    for r0 in range(0, C.shape[0], 1 << 20):
        c, r = C[r0:r0 + (1 << 20)], ref_dev[r0:r0 + (1 << 20)]
        assert not torch.isnan(c).any().item(), f"{what}: NaN in rows from {r0}"
        excess = ((c - r).abs() - (ATOL + RTOL * r.abs())).max().item()
        worst = max(worst, excess)
    assert worst <= 0.0, f"{what}: tolerance exceeded by {worst}"


@pytest.mark.parametrize("cfg", [4, 5, 3, 2])
def test_full_size_launches_vs_oracle(gpu_ctx, cfg):
    """The full-size workloads, with the committed gfx950 cost file and the
    benchmark's segment sizes, under the launches the benchmark times and
    the alternative placements: the whole of C against the reference-order
    oracle (parallelMatrix.cpp:148-236, the OpenMP restatement with atomic
    adds for split rows) at 1e-5 relative / 1e-6 absolute."""
    torch = torch_mod()
    g = workloads.graph(cfg)
    K = workloads.FEATURE_DIM[cfg]
    cands = workloads.candidate_s(g.nnz, 256)
    costs = capi.read_costs(paths.COST_FILE)
    H = torch.empty((g.n, K), dtype=torch.float32, device="cuda")
    gpu_ctx.fill_features(H, g.n, K, workloads.FEATURE_SEED)
    H_host = synth.features(g.n, K, workloads.FEATURE_SEED)
    C = torch.empty((g.n, K), dtype=torch.float32, device="cuda")
    probs = {}
    try:
        for launch in FULL_LAUNCHES[cfg]:
            si = launch[0]
            if si not in probs:
                p = problem(g, costs, cands[si])
                ref = oracle.spmm_mean_f32_omp(p.row_ptr, p.col_idx, p.val, p.origin, H_host,
                                               p.tasks)
                d = [dev(x) for x in (p.row_ptr, p.col_idx, p.val, p.origin)]
                d.append(dev(np.ascontiguousarray(p.tasks, np.int32).reshape(-1)))
                probs = {si: (p, d, torch.from_numpy(ref).cuda())}
                del ref
            p, d, ref_dev = probs[si]
            args = (d[0], d[1], d[2], d[3], g.n, g.nnz, H, g.n, K, d[4], len(p.tasks), C)
            if launch[1] is None:
                m, sl, loc = gpu_ctx.tune_schedule(*args, trials=3, locality=True)
                flags = 0
            else:
                _, m, sl, order, xcd, hot, occ, flags = launch[:8]
                gpu_ctx.set_schedule(m, sl)
                gpu_ctx.set_locality(order, xcd)
                gpu_ctx.set_cache_hints(hot)
                gpu_ctx.set_occupancy(occ)
                gpu_ctx.set_column_phases(launch[8] if len(launch) > 8 else 0)
                gpu_ctx.set_lane_tiling(launch[9] if len(launch) > 9 else 0)
            C.fill_(float("nan"))
            gpu_ctx.spmm(*args, flags=flags)
            info = gpu_ctx.last_launch()
            what = f"cfg={cfg} S={p.S} launch={launch} ran={info}"
            print(what, flush=True)
            if launch[1] is not None and flags == 0:
                assert info["tasks_per_wave"] == m or m == 0, what
                assert info["feature_slices"] == sl or sl == 0, what
                assert info["cache_hints"] == int(hot > 0), what
                assert info["column_phases"] == max(launch[8] if len(launch) > 8 else 1, 1), what
                wide = info["cache_hints"] == 0 and info["column_phases"] == 1
                packed = len(launch) > 9 and launch[9] == 2 and info["waves_per_simd"] == 0
                assert (info["slot_lanes"], info["lane_vectors"]) == expected_tiling(
                    K, info["feature_slices"], packed, wide), what
            _assert_close_on_device(torch, C, ref_dev, what)
            gpu_ctx.set_schedule(0, 0)
            gpu_ctx.set_locality(0, 0)
            gpu_ctx.set_cache_hints(0)
            gpu_ctx.set_occupancy(0)
            gpu_ctx.set_column_phases(0)
            gpu_ctx.set_lane_tiling(0)
    finally:
        gpu_ctx.set_schedule(0, 0)
        gpu_ctx.set_locality(0, 0)
        gpu_ctx.set_cache_hints(0)
        gpu_ctx.set_occupancy(0)
        gpu_ctx.set_column_phases(0)
        gpu_ctx.set_lane_tiling(0)


@pytest.mark.parametrize("K", [32, 64, 96])
def test_full_rmat_feature_widths_vs_oracle(gpu_ctx, K):
    """The full R-MAT graph at the paper's other feature widths (32, 64 and
    96; 128 is the headline above), S = 63 with the committed cost file:
    the schedule cwlb_ctx_tune_schedule keeps, and the same schedule with
    packed slots (at K = 96, 8 lanes x 3 vectors instead of 32-lane slots),
    each on the whole of C against the reference-order oracle
    (parallelMatrix.cpp:148-236) at 1e-5 relative / 1e-6 absolute."""
    torch = torch_mod()
    g = workloads.graph(4)
    costs = capi.read_costs(paths.COST_FILE)
    p = problem(g, costs, workloads.candidate_s(g.nnz, 256)[1])
    H = torch.empty((g.n, K), dtype=torch.float32, device="cuda")
    gpu_ctx.fill_features(H, g.n, K, workloads.FEATURE_SEED)
    ref_dev = torch.from_numpy(oracle.spmm_mean_f32_omp(
        p.row_ptr, p.col_idx, p.val, p.origin, synth.features(g.n, K, workloads.FEATURE_SEED),
        p.tasks)).cuda()
    d = [dev(x) for x in (p.row_ptr, p.col_idx, p.val, p.origin)]
    d_t = dev(np.ascontiguousarray(p.tasks, np.int32).reshape(-1))
    C = torch.empty((g.n, K), dtype=torch.float32, device="cuda")
    args = (d[0], d[1], d[2], d[3], g.n, g.nnz, H, g.n, K, d_t, len(p.tasks), C)
    try:
        gpu_ctx.tune_schedule(*args, trials=3, locality=True)
        for tiling in (gpu_ctx.lane_tiling(), 2):
            gpu_ctx.set_lane_tiling(tiling)
            C.fill_(float("nan"))
            gpu_ctx.spmm(*args)
            info = gpu_ctx.last_launch()
            what = f"rmat K={K} S={p.S} tiling={tiling} ran={info}"
            print(what, flush=True)
            _assert_close_on_device(torch, C, ref_dev, what)
    finally:
        gpu_ctx.set_schedule(0, 0)
        gpu_ctx.set_locality(0, 0)
        gpu_ctx.set_cache_hints(0)
        gpu_ctx.set_occupancy(0)
        gpu_ctx.set_column_phases(0)
        gpu_ctx.set_lane_tiling(0)


MESH_S_SWEEP = (32, 64, 128, 256, 512)


def test_full_mesh_segment_size_sweep_vs_oracle(gpu_ctx):
    """The full mesh (16M rows, 40M nonzeros, K = 32) at every segment size
    of the reference's range sweep (main.cpp:657-711), the S values its
    benchmark times: with the automatic schedule and with the schedule
    cwlb_ctx_tune_schedule keeps for that S (placement included), the whole
    of C against the reference-order oracle (parallelMatrix.cpp:148-236) at
    1e-5 relative / 1e-6 absolute."""
    torch = torch_mod()
    g = workloads.graph(5)
    K = workloads.FEATURE_DIM[5]
    costs = capi.read_costs(paths.COST_FILE)
    H = torch.empty((g.n, K), dtype=torch.float32, device="cuda")
    gpu_ctx.fill_features(H, g.n, K, workloads.FEATURE_SEED)
    H_host = synth.features(g.n, K, workloads.FEATURE_SEED)
    C = torch.empty((g.n, K), dtype=torch.float32, device="cuda")
    try:
        for S in MESH_S_SWEEP:
            p = problem(g, costs, S)
            ref_dev = torch.from_numpy(oracle.spmm_mean_f32_omp(
                p.row_ptr, p.col_idx, p.val, p.origin, H_host, p.tasks)).cuda()
            d = [dev(x) for x in (p.row_ptr, p.col_idx, p.val, p.origin)]
            d_t = dev(np.ascontiguousarray(p.tasks, np.int32).reshape(-1))
            args = (d[0], d[1], d[2], d[3], g.n, g.nnz, H, g.n, K, d_t, len(p.tasks), C)
            for tuned in (False, True):
                gpu_ctx.set_schedule(0, 0)
                gpu_ctx.set_locality(0, 0)
                gpu_ctx.set_cache_hints(0)
                gpu_ctx.set_occupancy(0)
                gpu_ctx.set_column_phases(0)
                if tuned:
                    gpu_ctx.tune_schedule(*args, trials=3, locality=True)
                C.fill_(float("nan"))
                gpu_ctx.spmm(*args)
                what = f"mesh S={S} tasks={len(p.tasks)} tuned={tuned} ran={gpu_ctx.last_launch()}"
                print(what, flush=True)
                _assert_close_on_device(torch, C, ref_dev, what)
            del ref_dev, d, d_t
    finally:
        gpu_ctx.set_schedule(0, 0)
        gpu_ctx.set_locality(0, 0)
        gpu_ctx.set_cache_hints(0)
        gpu_ctx.set_occupancy(0)
        gpu_ctx.set_column_phases(0)


def test_async_call_reports_bad_column_at_synchronize(gpu_ctx):
    g = workloads.small(1, seed=2)
    H = synth.features(g.n, 32, 3)
    p = problem(g, UNIT_COSTS, 6)
    ci = p.col_idx.copy()
    ci[len(ci) // 3] = -4
    torch = torch_mod()
    d = [dev(x) for x in (p.row_ptr, ci, p.val, p.origin)]
    d_t = dev(np.ascontiguousarray(p.tasks, np.int32).reshape(-1))
    C = torch.zeros((g.n, 32), dtype=torch.float32, device="cuda")
    gpu_ctx.spmm(*d, g.n, g.nnz, dev(H), g.n, 32, d_t, len(p.tasks), C, timed=False)
    with pytest.raises(capi.CwlbError) as e:
        gpu_ctx.synchronize()
    assert e.value.status == capi.INVALID_ARG
    # a good call clears the status word
    d[1] = dev(p.col_idx)
    gpu_ctx.spmm(*d, g.n, g.nnz, dev(H), g.n, 32, d_t, len(p.tasks), C, timed=False)
    gpu_ctx.synchronize()


HOT64 = 64 * 4 * 64
# (flags, (hot bytes, run order) of the eager call, the same for the captured
# call, (cache hints, run order) the captured launch uses): a captured call
# reuses the cache hints and run order an eager call built, and runs without
# them when none match.  The unbuilt hints case changes the hot set between
# the calls: the caching allocator may hand out the column array of an
# earlier case at the same address, and hints kept for it would match.
CAPTURE_CASES = {
    "default": (0, (0, 0), (0, 0), (0, 1)),
    "zero_output": (capi.ZERO_OUTPUT, (0, 0), (0, 0), (0, 1)),
    # the captured clear gives the empty rows the kernel leaves their zeros
    "zero_output_keep_empty": (capi.ZERO_OUTPUT | capi.KEEP_EMPTY_ROWS, (0, 0), (0, 0), (0, 1)),
    "cache_hints_built": (0, (HOT64, 0), (HOT64, 0), (1, 1)),
    "cache_hints_unbuilt": (0, (2 * HOT64, 0), (HOT64, 0), (0, 1)),
    "run_order_built": (0, (0, 2), (0, 2), (0, 2)),
    "run_order_unbuilt": (0, (0, 0), (0, 2), (0, 1)),
}


@pytest.mark.parametrize("case", list(CAPTURE_CASES))
def test_hip_graph_capture_and_replay(gpu_ctx, case):
    """An asynchronous call captured into a HIP graph (torch.cuda.CUDAGraph)
    and replayed several times, with eager work and synchronisations in
    between, gives the eager result on every replay."""
    torch = torch_mod()
    flags, eager_cfg, capture_cfg, used = CAPTURE_CASES[case]
    g = workloads.small(4, seed=21)
    K = 64
    p = problem(g, SKEWED_COSTS, 9)
    d_rp, d_ci, d_v, d_o = dev(p.row_ptr), dev(p.col_idx), dev(p.val), dev(p.origin)
    d_t = dev(np.ascontiguousarray(p.tasks, np.int32).reshape(-1))
    H = dev(synth.features(g.n, K, 4))
    C = torch.zeros((g.n, K), dtype=torch.float32, device="cuda")
    gpu_ctx.set_schedule(4, 0)  # runs of 4 tasks, so that a run order exists
    try:
        _capture_and_replay(gpu_ctx, torch, g, K, p, (d_rp, d_ci, d_v, d_o, d_t), H, C, flags,
                            eager_cfg, capture_cfg, used)
    finally:
        gpu_ctx.set_schedule(0, 0)
        gpu_ctx.set_cache_hints(0)
        gpu_ctx.set_locality(0, 0)


def _capture_and_replay(gpu_ctx, torch, g, K, p, d, H, C, flags, eager_cfg, capture_cfg, used):
    d_rp, d_ci, d_v, d_o, d_t = d
    gpu_ctx.set_cache_hints(eager_cfg[0])
    gpu_ctx.set_locality(eager_cfg[1], 0)
    gpu_ctx.spmm(d_rp, d_ci, d_v, d_o, g.n, g.nnz, H, g.n, K, d_t, len(p.tasks), C, flags=flags)
    info = gpu_ctx.last_launch()
    assert (info["cache_hints"], info["run_order"]) == (int(eager_cfg[0] > 0),
                                                        2 if eager_cfg[1] == 2 else 1), info
    eager = C.clone()
    gpu_ctx.set_cache_hints(capture_cfg[0])
    if capture_cfg[1] != eager_cfg[1]:
        gpu_ctx.set_locality(capture_cfg[1], 0)
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        gpu_ctx.set_stream(side.cuda_stream)
        with torch.cuda.graph(graph, stream=side):
            gpu_ctx.spmm(d_rp, d_ci, d_v, d_o, g.n, g.nnz, H, g.n, K, d_t, len(p.tasks), C,
                         flags=flags, timed=False)
    gpu_ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    info = gpu_ctx.last_launch()
    assert (info["cache_hints"], info["run_order"]) == used, info
    torch.cuda.synchronize()
    for i in range(4):
        C.fill_(float("nan") if flags else float(i))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        np.testing.assert_allclose(C.cpu().numpy(), eager.cpu().numpy(), rtol=RTOL, atol=ATOL)
        _ = (H * 2.0).sum().item()  # eager work between replays
    ref32 = oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H.cpu().numpy(), p.tasks)
    np.testing.assert_allclose(C.cpu().numpy(), ref32, rtol=RTOL, atol=ATOL)


def test_graph_replay_after_rebuild_on_other_arrays(gpu_ctx):
    """A graph captured with a run order and cache hints built by an eager
    call keeps working after eager calls on the same context rebuild both
    for another problem (fewer runs, another column array): the rebuild
    goes into new buffers, and every replay still gives the first problem's
    result, interleaved with the second problem's eager calls."""
    torch = torch_mod()
    K = 64
    g1 = workloads.small(4, seed=21)
    p1 = problem(g1, SKEWED_COSTS, 9)
    g2 = workloads.small(4, seed=22)
    p2 = problem(g2, SKEWED_COSTS, 40)
    d1 = [dev(x) for x in (p1.row_ptr, p1.col_idx, p1.val, p1.origin)]
    d1.append(dev(np.ascontiguousarray(p1.tasks, np.int32).reshape(-1)))
    d2 = [dev(x) for x in (p2.row_ptr, p2.col_idx, p2.val, p2.origin)]
    d2.append(dev(np.ascontiguousarray(p2.tasks, np.int32).reshape(-1)))
    H1, H2 = synth.features(g1.n, K, 4), synth.features(g2.n, K, 5)
    dH1, dH2 = dev(H1), dev(H2)
    C1 = torch.zeros((g1.n, K), dtype=torch.float32, device="cuda")
    C2 = torch.zeros((g2.n, K), dtype=torch.float32, device="cuda")
    ref1 = oracle.spmm_mean_f32(p1.row_ptr, p1.col_idx, p1.val, p1.origin, H1, p1.tasks)
    ref2 = oracle.spmm_mean_f32(p2.row_ptr, p2.col_idx, p2.val, p2.origin, H2, p2.tasks)

    def call(d, g, p, dH, C, **kw):
        gpu_ctx.spmm(d[0], d[1], d[2], d[3], g.n, g.nnz, dH, g.n, K, d[4], len(p.tasks), C,
                     **kw)

    gpu_ctx.set_schedule(4, 0)
    gpu_ctx.set_locality(2, 0)
    gpu_ctx.set_cache_hints(HOT64)
    try:
        call(d1, g1, p1, dH1, C1)  # builds the run order and the hints for problem 1
        info = gpu_ctx.last_launch()
        assert (info["run_order"], info["cache_hints"]) == (2, 1), info
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            gpu_ctx.set_stream(side.cuda_stream)
            with torch.cuda.graph(graph, stream=side):
                call(d1, g1, p1, dH1, C1, timed=False)
        gpu_ctx.set_stream(torch.cuda.current_stream().cuda_stream)
        info = gpu_ctx.last_launch()
        assert (info["run_order"], info["cache_hints"]) == (2, 1), info
        torch.cuda.synchronize()
        for i in range(3):
            C2.fill_(float("nan"))
            call(d2, g2, p2, dH2, C2)  # rebuilds order and hints for problem 2
            info = gpu_ctx.last_launch()
            assert (info["run_order"], info["cache_hints"]) == (2, 1), info
            check(C2.cpu().numpy(), ref2)
            C1.fill_(float("nan"))
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            check(C1.cpu().numpy(), ref1)
            gpu_ctx.set_locality(2, 0)  # forget the order: the next call sorts again
    finally:
        gpu_ctx.set_schedule(0, 0)
        gpu_ctx.set_locality(0, 0)
        gpu_ctx.set_cache_hints(0)


def test_allocating_entries_refused_under_capture(gpu_ctx):
    """The entry points that allocate, read back or synchronise -- the GPU
    reorder and partition, the host-pointer call, the calibration and the
    schedule tuner -- return CWLB_UNSUPPORTED on a stream under graph
    capture before enqueueing anything: the capture stays valid, and an
    aggregation call captured after them replays to the oracle's result
    (with eager work between replays)."""
    torch = torch_mod()
    g = workloads.small(4, seed=41)
    K = 64
    p = problem(g, SKEWED_COSTS, 8)
    H_host = synth.features(g.n, K, 6)
    d_rp0, d_ci0, d_v0 = dev(g.row_ptr), dev(g.col_idx), dev(g.val)
    d_rp, d_ci, d_v, d_o = dev(p.row_ptr), dev(p.col_idx), dev(p.val), dev(p.origin)
    d_t = dev(np.ascontiguousarray(p.tasks, np.int32).reshape(-1))
    H = dev(H_host)
    C = torch.zeros((g.n, K), dtype=torch.float32, device="cuda")
    outs = [torch.zeros(g.n, dtype=torch.int32, device="cuda"),
            torch.zeros(g.n + 1, dtype=torch.int32, device="cuda"),
            torch.zeros(g.nnz, dtype=torch.int32, device="cuda"),
            torch.zeros(g.nnz, dtype=torch.float32, device="cuda")]
    t_out = torch.zeros((len(p.tasks), 4), dtype=torch.int32, device="cuda")
    args = (d_rp, d_ci, d_v, d_o, g.n, g.nnz, H, g.n, K, d_t, len(p.tasks), C)
    refused = {
        "reorder": lambda: gpu_ctx.reorder_device(g.n, g.nnz, d_rp0, d_ci0, d_v0, *outs),
        "partition": lambda: gpu_ctx.partition_device(d_rp, g.n, SKEWED_COSTS, p.capacity, t_out,
                                                      len(p.tasks)),
        "host_call": lambda: gpu_ctx.spmm_host(p.row_ptr, p.col_idx, p.val, p.origin, H_host,
                                               p.tasks),
        "calibrate": lambda: gpu_ctx.calibrate(K=32, repeat=2, WI=4096, load_MB=8),
        "tune": lambda: gpu_ctx.tune_schedule(*args, trials=1),
    }
    statuses = {}
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    try:
        with torch.cuda.stream(side):
            gpu_ctx.set_stream(side.cuda_stream)
            with torch.cuda.graph(graph, stream=side):
                for name, fn in refused.items():
                    try:
                        fn()
                        statuses[name] = (capi.OK, "")
                    except capi.CwlbError as e:
                        statuses[name] = (e.status, str(e))
                gpu_ctx.spmm(*args, timed=False)
    finally:
        gpu_ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    for name, (status, msg) in statuses.items():
        assert status == capi.UNSUPPORTED and "graph capture" in msg, (name, status, msg)
    torch.cuda.synchronize()
    ref = oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H_host, p.tasks)
    for i in range(3):
        C.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        check(C.cpu().numpy(), ref)
        _ = (H * 2.0).sum().item()  # eager work between replays
    # Outside capture the same entries run: the reorder and partition match
    # the host's.
    gpu_ctx.reorder_device(g.n, g.nnz, d_rp0, d_ci0, d_v0, *outs)
    assert np.array_equal(outs[1].cpu().numpy(), p.row_ptr)
    n_t = gpu_ctx.partition_device(d_rp, g.n, SKEWED_COSTS, p.capacity, t_out, len(p.tasks))
    assert n_t == len(p.tasks) and np.array_equal(t_out.cpu().numpy(), p.tasks)


def test_tune_schedule(gpu_ctx):
    """cwlb_ctx_tune_schedule picks one of its candidates, leaves it on the
    context, and every schedule it tried computes the same result.  A hot
    set the context held before is replaced by one of the tuner's sizes."""
    g = workloads.small(4, seed=13)
    K = 128
    p = problem(g, SKEWED_COSTS, 16)
    H = synth.features(g.n, K, 2)
    torch = torch_mod()
    d_rp, d_ci, d_v, d_o = dev(p.row_ptr), dev(p.col_idx), dev(p.val), dev(p.origin)
    d_t = dev(np.ascontiguousarray(p.tasks, np.int32).reshape(-1))
    d_H = dev(H)
    C = torch.full((g.n, K), float("nan"), dtype=torch.float32, device="cuda")
    gpu_ctx.set_cache_hints(7 << 20)
    try:
        m, sl, loc = gpu_ctx.tune_schedule(d_rp, d_ci, d_v, d_o, g.n, g.nnz, d_H, g.n, K, d_t,
                                           len(p.tasks), C, trials=2, locality=True)
        assert (m, sl) == (0, 0) or (m in (1, 2, 4, 8, 16, 32, 64) and sl in (1, 2, 4))
        assert loc in ((0, 0), (2, 1), (2, 2))
        assert gpu_ctx.cache_hints() in (0, 24 << 20, 48 << 20, 96 << 20)
        assert gpu_ctx.occupancy() in (0, 6)
        assert gpu_ctx.lane_tiling() in (0, 2)
        ref32, ref64 = oracle_pair(p, g, H)
        check(C.cpu().numpy(), ref32)
        C.fill_(float("nan"))
        gpu_ctx.spmm(d_rp, d_ci, d_v, d_o, g.n, g.nnz, d_H, g.n, K, d_t, len(p.tasks), C)
        check(C.cpu().numpy(), ref32)
        check(C.cpu().numpy(), ref64)
        info = gpu_ctx.last_launch()
        assert info["cache_hints"] == int(gpu_ctx.cache_hints() > 0), info
        assert (info["feature_slices"] == sl) if sl else True, info
        assert (info["tasks_per_wave"] == m) if m else True, info
        assert info["run_order"] == (2 if loc[0] == 2 else 1), info
        assert info["waves_per_simd"] == gpu_ctx.occupancy(), info
        wide = info["cache_hints"] == 0 and info["column_phases"] == 1
        packed = gpu_ctx.lane_tiling() == 2 and info["waves_per_simd"] == 0
        assert (info["slot_lanes"], info["lane_vectors"]) == expected_tiling(
            K, info["feature_slices"], packed, wide), info
        with pytest.raises(capi.CwlbError) as e:
            gpu_ctx.tune_schedule(d_rp, d_ci, d_v, d_o, g.n, g.nnz, d_H, g.n, K, d_t,
                                  len(p.tasks), C, trials=0)
        assert e.value.status == capi.INVALID_ARG
    finally:
        gpu_ctx.set_schedule(0, 0)
        gpu_ctx.set_locality(0, 0)
        gpu_ctx.set_cache_hints(0)
        gpu_ctx.set_occupancy(0)
        gpu_ctx.set_column_phases(0)
        gpu_ctx.set_lane_tiling(0)


def test_run_order_reused_across_task_lists(gpu_ctx):
    """With runs sorted by output row, the order is kept between calls and
    rebuilt when the task array changes; each list's result is right."""
    g = workloads.small(5, seed=4)
    K = 32
    H = synth.features(g.n, K, 6)
    torch = torch_mod()
    gpu_ctx.set_schedule(2, 1)
    gpu_ctx.set_locality(2, 2)
    try:
        for S in (3, 7, 3):
            p = problem(g, SKEWED_COSTS, S)
            for _ in range(2):
                got, _ = run_gpu(gpu_ctx, p, H)
                ref32, ref64 = oracle_pair(p, g, H)
                check(got, ref32)
                check(got, ref64)
    finally:
        gpu_ctx.set_schedule(0, 0)
        gpu_ctx.set_locality(0, 0)
