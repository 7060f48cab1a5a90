"""GPU parity of the column-phased aggregation (cwlb_ctx_set_column_phases).

The phased path runs a chain of tasks P times, phase p gathering the
nonzeros whose column c has c mod P = p from a band-sorted copy of the
column and value arrays, each row owned by one wave (stored in the first
phase, added to in the others).  Its results must be the reference's (the
oracle, src/parallelMatrix.cpp:148-236) within the parity tolerance
|gpu - ref| <= 1e-6 + 1e-5 |ref|, for every run length, slice count and
phase count, for chains that start and end inside rows, and lists that are
not chains must run in one pass with the one-pass results.  The device's
band sort (bounds and copy) must equal its host restatement exactly.
"""
import numpy as np
import pytest

import oracle
from conftest import SKEWED_COSTS, UNIT_COSTS
from cwlb_amd import capi, synth, workloads
from test_column_phases import band_copy, phase_bounds
from test_gpu_spmm import check, custom_graph, dev, oracle_pair, problem, run_gpu, torch_mod

pytestmark = pytest.mark.gpu


def set_phased(ctx, P, M, SL, order=1, xcd=1):
    ctx.set_schedule(M, SL)
    ctx.set_locality(order, xcd)
    ctx.set_column_phases(P)


@pytest.fixture
def reset(gpu_ctx):
    yield
    gpu_ctx.set_column_phases(0)
    gpu_ctx.set_schedule(0, 0)
    gpu_ctx.set_locality(0, 0)
    gpu_ctx.set_lane_tiling(0)


def expected_phases(K, SL, P):
    """Phases the launch runs: 16-byte lanes and at most 64 vectors per slice."""
    if P < 2 or K % 4 or K < 4:
        return 1
    sl = SL if (SL > 0 and K // 4 >= SL) else 1
    return P if -(-(K // 4) // sl) <= 64 else 1


def device_band_sort(ctx, rp, ci, val, h_rows, P):
    """(bounds, col copy, val copy) from cwlb_column_phase_sort."""
    torch = torch_mod()
    n, nnz = len(rp) - 1, len(ci)
    out = torch.full(((P - 1) * max(n, 1),), -7, dtype=torch.int32, device="cuda")
    col = torch.full((max(nnz, 1),), -9, dtype=torch.int32, device="cuda")
    vals = torch.full((max(nnz, 1),), -9.0, dtype=torch.float32, device="cuda")
    ctx.column_phase_sort(dev(rp), dev(ci), dev(val), n, nnz, h_rows, P, out, col, vals)
    torch.cuda.synchronize()
    return (out.cpu().numpy()[:(P - 1) * n].reshape(P - 1, n), col.cpu().numpy()[:nnz],
            vals.cpu().numpy()[:nnz])


@pytest.mark.parametrize("P", [2, 3, 5, 12, 16, 33, 63, 64])
def test_band_sort_matches_host(gpu_ctx, P):
    """Sorted and unsorted rows, columns below 0 and at or past h_rows,
    rows of 512, 513, 700 and 3000 nonzeros (one batch of loads exactly,
    and more: those are scattered straight to memory), empty rows, and band
    counts at each width of the band number (P = 3, 5, 12, 33, 63, 64:
    2 to 7 bits with the past-the-row marker): the device
    bounds and band-sorted copy equal the host restatement exactly (the
    copy is stable within each band).  Rows whose offsets leave [0, nnz] or
    decrease get bounds 0."""
    rng = np.random.default_rng(P)
    n, h = 2000, 777
    deg = rng.integers(0, 90, n)
    deg[5] = 3000
    deg[6:9] = (512, 513, 700)
    deg[rng.integers(10, n, 200)] = 0
    rp = np.concatenate([[0], np.cumsum(deg)]).astype(np.int32)
    ci = rng.integers(-3, h + 4, rp[-1]).astype(np.int32)
    val = rng.normal(size=rp[-1]).astype(np.float32)
    for r in range(0, n, 2):
        ci[rp[r]:rp[r + 1]].sort()
    bounds, col, vals = device_band_sort(gpu_ctx, rp, ci, val, h, P)
    assert np.array_equal(bounds, phase_bounds(rp, ci, h, P))
    want_c, want_v = band_copy(rp, ci, val, h, P)
    assert np.array_equal(col, want_c) and np.array_equal(vals, want_v)
    bad = rp.copy()
    bad[100] = bad[101] + 5       # row 100 decreases
    bad[-1] = rp[-1] + 50         # the last row passes nnz
    got, _, _ = device_band_sort(gpu_ctx, bad, ci, val, h, P)
    assert np.array_equal(got, phase_bounds(bad, ci, h, P))
    assert (got[:, 100] == 0).all() and (got[:, n - 1] == 0).all()


def test_band_sort_arguments(gpu_ctx):
    torch = torch_mod()
    rp, ci = dev(np.array([0, 1], np.int32)), dev(np.array([0], np.int32))
    val = dev(np.array([1.0], np.float32))
    out = torch.zeros(64, dtype=torch.int32, device="cuda")
    col = torch.zeros(64, dtype=torch.int32, device="cuda")
    vals = torch.zeros(64, dtype=torch.float32, device="cuda")
    for P, h in ((1, 1), (65, 1), (2, 0)):
        with pytest.raises(capi.CwlbError) as e:
            gpu_ctx.column_phase_sort(rp, ci, val, 1, 1, h, P, out)
        assert e.value.status == capi.INVALID_ARG
    with pytest.raises(capi.CwlbError) as e:  # the two copies go together
        gpu_ctx.column_phase_sort(rp, ci, val, 1, 1, 1, 2, out, col, None)
    assert e.value.status == capi.INVALID_ARG
    with pytest.raises(capi.CwlbError) as e:  # a copy needs the values
        gpu_ctx.column_phase_sort(rp, ci, None, 1, 1, 1, 2, out, col, vals)
    assert e.value.status == capi.INVALID_ARG
    gpu_ctx.column_phase_sort(rp, ci, val, 0, 0, 1, 2, out)  # nothing to do
    gpu_ctx.column_phase_sort(rp, ci, None, 1, 1, 1, 2, out)  # bounds only


# (P, tasks per wave, slices)
PHASED = [(2, 1, 1), (4, 3, 2), (16, 16, 4), (8, 64, 8), (64, 5, 1), (3, 200, 2), (12, 16, 0)]
PHASED_IDS = [f"p{p}m{m}s{s}" for p, m, s in PHASED]


@pytest.mark.parametrize("P,M,SL", PHASED, ids=PHASED_IDS)
@pytest.mark.parametrize("cfg", [1, 2, 3, 4, 5])
def test_small_configs(gpu_ctx, reset, cfg, P, M, SL):
    """Each configuration family at reduced size (K = 64, or 600 for the
    block model, where slices of at most 64 vectors need 4 or 8 of them)."""
    g = workloads.small(cfg)
    K = 600 if cfg == 3 else 64
    S = workloads.candidate_s(g.nnz, 256)[1]
    p = problem(g, SKEWED_COSTS, S)
    H = synth.features(g.n, K, workloads.FEATURE_SEED)
    set_phased(gpu_ctx, P, M, SL)
    print(f"cfg={cfg} P={P} M={M} SL={SL} n={g.n} tasks={len(p.tasks)}", flush=True)
    got, _ = run_gpu(gpu_ctx, p, H)
    assert gpu_ctx.last_launch()["column_phases"] == expected_phases(K, SL, P)
    ref32, ref64 = oracle_pair(p, g, H)
    check(got, ref32)
    check(got, ref64)


@pytest.mark.parametrize("K", [4, 8, 12, 64, 100, 128, 256, 260, 512])
def test_feature_widths(gpu_ctx, reset, K):
    """Phases apply with at most 64 vectors per slice; other widths run in
    one pass; every width gives the reference's result."""
    g = workloads.small(4, seed=3)
    p = problem(g, UNIT_COSTS, 5)
    H = synth.features(g.n, K, 2)
    for SL in (1, 4):
        set_phased(gpu_ctx, 6, 8, SL)
        got, _ = run_gpu(gpu_ctx, p, H)
        assert gpu_ctx.last_launch()["column_phases"] == expected_phases(K, SL, 6), (K, SL)
        check(got, oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H, p.tasks))


@pytest.mark.parametrize("K", [1028, 2048, 2052])
def test_large_k_entry(gpu_ctx, reset, K):
    """The large-K entry takes phases when its slices are narrow enough (8
    slices of at most 64 float4 up to K = 2,048), else runs in one pass."""
    g = workloads.small(2, seed=7)
    p = problem(g, SKEWED_COSTS, 6)
    H = synth.features(g.n, K, 4)
    ref = oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H, p.tasks)
    for SL in (8, 4):
        set_phased(gpu_ctx, 5, 16, SL)
        got, _ = run_gpu(gpu_ctx, p, H, large_k=True)
        assert gpu_ctx.last_launch()["column_phases"] == expected_phases(K, SL, 5), (K, SL)
        check(got, ref)


@pytest.mark.parametrize("M", [1, 4, 64])
def test_chains_inside_rows(gpu_ctx, reset, M):
    """Sub-lists of a partition start and end inside split rows.  With C
    holding earlier values, rows outside keep them, the first row (partial,
    not cleared) is added onto them, the last is cleared and added: the
    phased result equals the one-pass result; with ZERO_OUTPUT it equals
    the oracle."""
    torch = torch_mod()
    rng = np.random.default_rng(M)
    g = workloads.small(4, seed=5)
    K = 32
    p = problem(g, UNIT_COSTS, 3)
    H = synth.features(g.n, K, 1)
    split = np.nonzero(p.tasks[:, 2] > 0)[0]
    d_rp, d_ci, d_v, d_o = dev(p.row_ptr), dev(p.col_idx), dev(p.val), dev(p.origin)
    d_H = dev(H)
    prior = torch.from_numpy(synth.features(g.n, K, 9)).cuda()
    for _ in range(4):
        k, j = np.sort(rng.choice(split, 2, replace=False))
        sub = p.tasks[k:j + 1]
        d_t = dev(np.ascontiguousarray(sub).reshape(-1))
        outs = []
        for P in (0, 5):
            set_phased(gpu_ctx, P, M, 2)
            C = prior.clone()
            gpu_ctx.spmm(d_rp, d_ci, d_v, d_o, g.n, g.nnz, d_H, g.n, K, d_t, len(sub), C)
            outs.append(C.cpu().numpy())
            assert gpu_ctx.last_launch()["column_phases"] == max(P, 1)
        np.testing.assert_allclose(outs[1], outs[0], rtol=1e-5, atol=1e-6)
        C = torch.full((g.n, K), float("nan"), dtype=torch.float32, device="cuda")
        gpu_ctx.spmm(d_rp, d_ci, d_v, d_o, g.n, g.nnz, d_H, g.n, K, d_t, len(sub), C,
                     flags=capi.ZERO_OUTPUT)
        check(C.cpu().numpy(), oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H,
                                                    sub))


@pytest.mark.parametrize("how", ["shuffled", "gaps", "malformed_task"])
def test_lists_that_are_not_chains(gpu_ctx, reset, how):
    """Lists that break the chain run in one pass inside the phased launch
    sequence: the reference's result (with ZERO_OUTPUT for gapped lists),
    then a chain on the same context runs phased again."""
    rng = np.random.default_rng(len(how))
    g = workloads.small(4, seed=8)
    K = 64
    p = problem(g, SKEWED_COSTS, 4)
    H = synth.features(g.n, K, 3)
    t = p.tasks.copy()
    if how == "shuffled":
        t = t[rng.permutation(len(t))]
    elif how == "gaps":
        t = t[rng.random(len(t)) > 0.1]
    else:
        t = np.concatenate([t[:50], [[3, 3, 0, 0]], t[50:]]).astype(np.int32)
    q = workloads.Prepared(p.n, p.nnz, p.origin, p.row_ptr, p.col_idx, p.val, t, 0, 0.0)
    set_phased(gpu_ctx, 7, 16, 2)
    got, _ = run_gpu(gpu_ctx, q, H, flags=capi.ZERO_OUTPUT)
    check(got, oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H, t))
    got, _ = run_gpu(gpu_ctx, p, H)
    check(got, oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H, p.tasks))


def test_hub_row_degree_zero_rows_and_zero_output(gpu_ctx, reset, rng):
    """A row of 5,000 nonzeros split into many tasks among empty rows and
    rows whose nonzeros all lie in one band; with and without ZERO_OUTPUT."""
    n = 6000
    deg = np.zeros(n, np.int64)
    deg[17] = 5000
    deg[rng.integers(0, n, 400)] = rng.integers(1, 9, 400)
    rp = np.concatenate([[0], np.cumsum(deg)]).astype(np.int32)
    ci = rng.integers(0, n, rp[-1]).astype(np.int32)
    ci[rp[100]:rp[101]] = n - 1  # (row 100 may be empty) the last band only
    val = rng.uniform(-2, 2, rp[-1]).astype(np.float32)
    g = custom_graph(rp, ci, val)
    H = synth.features(n, 64, 1)
    for S in (1, 3, 64, 5000):
        p = problem(g, UNIT_COSTS, S)
        ref32, ref64 = oracle_pair(p, g, H)
        for P, M, flags in ((4, 1, 0), (16, 64, capi.ZERO_OUTPUT), (64, 7, 0)):
            set_phased(gpu_ctx, P, M, 1)
            got, _ = run_gpu(gpu_ctx, p, H, flags=flags)
            check(got, ref32)
            check(got, ref64)


def test_rewritten_columns_keep_results_right(gpu_ctx, reset):
    """Columns rewritten in place between two phased calls (same pointer and
    sizes): every call sorts the arrays as they are."""
    torch = torch_mod()
    g = workloads.small(2, seed=4)
    K = 64
    p = problem(g, SKEWED_COSTS, 5)
    H = synth.features(g.n, K, 5)
    d_rp, d_ci, d_v, d_o = dev(p.row_ptr), dev(p.col_idx), dev(p.val), dev(p.origin)
    d_t = dev(np.ascontiguousarray(p.tasks).reshape(-1))
    d_H = dev(H)
    C = torch.zeros((g.n, K), dtype=torch.float32, device="cuda")
    set_phased(gpu_ctx, 8, 16, 1)
    gpu_ctx.spmm(d_rp, d_ci, d_v, d_o, g.n, g.nnz, d_H, g.n, K, d_t, len(p.tasks), C)
    other = np.random.default_rng(2).integers(0, g.n, g.nnz).astype(np.int32)
    d_ci.copy_(torch.from_numpy(other))
    gpu_ctx.spmm(d_rp, d_ci, d_v, d_o, g.n, g.nnz, d_H, g.n, K, d_t, len(p.tasks), C)
    check(C.cpu().numpy(), oracle.spmm_mean_f32(p.row_ptr, other, p.val, p.origin, H, p.tasks))


@pytest.mark.parametrize("bad", ["decreasing", "beyond_nnz", "column"])
def test_bad_entries_are_reported(gpu_ctx, reset, bad):
    """Bad row offsets and column indices are reported as with one pass; a
    good call afterwards clears the report."""
    g = workloads.small(1, seed=2)
    H = synth.features(g.n, 32, 3)
    p = problem(g, UNIT_COSTS, 6)
    good_rp, good_ci = p.row_ptr, p.col_idx
    if bad == "column":
        ci = p.col_idx.copy()
        ci[len(ci) // 3] = g.n + 5
        p.col_idx = ci
    else:
        rp = p.row_ptr.copy()
        r = len(rp) // 2
        if bad == "decreasing":
            rp[r] = rp[r + 1] + 3
        else:
            rp[-1] = p.nnz + 100
        p.row_ptr = rp
    set_phased(gpu_ctx, 5, 8, 1)
    with pytest.raises(capi.CwlbError) as e:
        run_gpu(gpu_ctx, p, H)
    assert e.value.status == capi.INVALID_ARG
    p.row_ptr, p.col_idx = good_rp, good_ci
    got, _ = run_gpu(gpu_ctx, p, H)
    check(got, oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H, p.tasks))


@pytest.mark.parametrize("built", [True, False], ids=["buffers_sized", "buffers_small"])
def test_graph_capture_and_replay(gpu_ctx, built):
    """A phased call captured into a HIP graph after an eager call sized the
    context's phase buffers replays the band sort and the phases; with
    buffers too small for its phase count the captured call runs in one
    pass.  Every replay, between eager phased calls that rewrite the same
    buffers, gives the eager result.  (A context of its own: the buffers'
    sizes are the point.)"""
    torch = torch_mod()
    g = workloads.small(4, seed=21)
    K = 64
    p = problem(g, SKEWED_COSTS, 9)
    d_rp, d_ci, d_v, d_o = dev(p.row_ptr), dev(p.col_idx), dev(p.val), dev(p.origin)
    d_t = dev(np.ascontiguousarray(p.tasks, np.int32).reshape(-1))
    H = dev(synth.features(g.n, K, 4))
    C = torch.zeros((g.n, K), dtype=torch.float32, device="cuda")
    ctx = capi.Context(0, torch.cuda.current_stream().cuda_stream)
    try:
        # The phased calls of the test have 6 phases; the buffers come from
        # an eager call with 6 phases, or with 3 (2 bounds per row: too
        # small for 6 phases under capture).
        set_phased(ctx, 6 if built else 3, 8, 2)
        ctx.spmm(d_rp, d_ci, d_v, d_o, g.n, g.nnz, H, g.n, K, d_t, len(p.tasks), C)
        ctx.set_column_phases(6)
        eager = C.clone()
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            ctx.set_stream(side.cuda_stream)
            with torch.cuda.graph(graph, stream=side):
                ctx.spmm(d_rp, d_ci, d_v, d_o, g.n, g.nnz, H, g.n, K, d_t, len(p.tasks), C,
                         timed=False)
        ctx.set_stream(torch.cuda.current_stream().cuda_stream)
        assert ctx.last_launch()["column_phases"] == (6 if built else 1)
        torch.cuda.synchronize()
        for i in range(4):
            C.fill_(float(i))
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            np.testing.assert_allclose(C.cpu().numpy(), eager.cpu().numpy(), rtol=1e-5,
                                       atol=1e-6)
            # eager phased calls on another list between replays
            ctx.spmm(d_rp, d_ci, d_v, d_o, g.n, g.nnz, H, g.n, K, d_t, len(p.tasks) // 2,
                     torch.zeros_like(C))
        torch.cuda.synchronize()
        del graph
    finally:
        ctx.close()
    ref32 = oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H.cpu().numpy(), p.tasks)
    np.testing.assert_allclose(C.cpu().numpy(), ref32, rtol=1e-5, atol=1e-6)


def test_phase_arguments(gpu_ctx, reset):
    for bad in (-1, 65):
        with pytest.raises(capi.CwlbError) as e:
            gpu_ctx.set_column_phases(bad)
        assert e.value.status == capi.INVALID_ARG
    gpu_ctx.set_column_phases(64)
    assert gpu_ctx.column_phases() == 64
    gpu_ctx.set_column_phases(0)
    assert gpu_ctx.column_phases() == 0


def test_per_task_flag_runs_one_pass(gpu_ctx, reset):
    g = workloads.small(2, seed=3)
    p = problem(g, SKEWED_COSTS, 5)
    H = synth.features(g.n, 32, 1)
    set_phased(gpu_ctx, 8, 8, 1)
    got, _ = run_gpu(gpu_ctx, p, H, flags=capi.PER_TASK)
    assert gpu_ctx.last_launch()["column_phases"] == 1
    check(got, oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H, p.tasks))


def test_tuner_tries_phases(gpu_ctx, reset):
    """A graph where phases may pay (H of 512 MB, 64 nonzeros per row): the
    tuner's choice, phases or not, leaves a context whose calls give the
    reference's result on sampled rows (the full oracle is too slow here)."""
    torch = torch_mod()
    n, deg, K = 131072, 64, 1024
    gen = torch.Generator(device="cuda").manual_seed(5)
    rp = torch.arange(0, (n + 1) * deg, deg, dtype=torch.int32, device="cuda")
    ci = torch.randint(0, n, (n * deg,), generator=gen, dtype=torch.int32, device="cuda")
    ci = ci.view(n, deg).sort(dim=1).values.reshape(-1).contiguous()
    val = torch.ones(n * deg, dtype=torch.float32, device="cuda")
    origin = torch.arange(n, dtype=torch.int32, device="cuda")
    tasks_np = capi.partition(rp.cpu().numpy(), SKEWED_COSTS,
                              capi.capacity_from_s(40, SKEWED_COSTS))
    tasks = dev(np.ascontiguousarray(tasks_np).reshape(-1))
    H = torch.empty((n, K), dtype=torch.float32, device="cuda")
    gpu_ctx.fill_features(H, n, K, 3)
    C = torch.full((n, K), float("nan"), dtype=torch.float32, device="cuda")
    m, sl, loc = gpu_ctx.tune_schedule(rp, ci, val, origin, n, n * deg, H, n, K, tasks,
                                       len(tasks_np), C, trials=1, locality=True)
    P = gpu_ctx.column_phases()
    print(f"tuned m={m} sl={sl} loc={loc} phases={P} tiling={gpu_ctx.lane_tiling()}", flush=True)
    assert P in (0, 8, 12, 16)
    assert gpu_ctx.lane_tiling() in (0, 2)
    C.fill_(float("nan"))
    gpu_ctx.spmm(rp, ci, val, origin, n, n * deg, H, n, K, tasks, len(tasks_np), C)
    assert gpu_ctx.last_launch()["column_phases"] == max(P, 1)
    rows = np.random.default_rng(1).choice(n, 64, replace=False)
    ci_h = ci.view(n, deg)[torch.from_numpy(rows).cuda().long()].long()
    want = H[ci_h].double().mean(dim=1).cpu().numpy()
    got = C[torch.from_numpy(rows).cuda().long()].double().cpu().numpy()
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)
    del H, C
    torch.cuda.empty_cache()


def test_stream_switch_orders_the_streams(gpu_ctx, reset):
    """An asynchronous phased call on stream A, then cwlb_ctx_set_stream(B)
    and a phased call on other arrays (another graph, task list and feature
    width): B's band sort rewrites the context's band-sorted copy and row
    bounds that A's phases read, so B must start after A's work.  Both
    results match the oracle; then back on A, a third call on A's arrays
    (after B's) does too.  Run order and XCD placement as built by the
    calls."""
    torch = torch_mod()
    probs = []
    for cfg, seed, K, S in ((4, 12, 256, 7), (1, 13, 64, 5)):
        g = workloads.small(cfg, seed=seed)
        p = problem(g, SKEWED_COSTS, S)
        H = synth.features(g.n, K, seed)
        d = [dev(x) for x in (p.row_ptr, p.col_idx, p.val, p.origin)]
        d_t = dev(np.ascontiguousarray(p.tasks).reshape(-1))
        ref = oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H, p.tasks)
        probs.append((g, p, K, d, d_t, dev(H), ref))
    a, b = torch.cuda.Stream(), torch.cuda.Stream()
    Cs = [torch.full((pr[0].n, pr[2]), float("nan"), dtype=torch.float32, device="cuda")
          for pr in probs]
    torch.cuda.synchronize()
    set_phased(gpu_ctx, 7, 4, 2, order=2, xcd=2)

    def call(i):
        g, p, K, d, d_t, d_H, _ = probs[i]
        gpu_ctx.spmm(d[0], d[1], d[2], d[3], g.n, g.nnz, d_H, g.n, K, d_t, len(p.tasks), Cs[i],
                     timed=False)
        return gpu_ctx.last_launch()

    try:
        gpu_ctx.set_stream(a.cuda_stream)
        info_a = call(0)
        gpu_ctx.set_stream(b.cuda_stream)
        info_b = call(1)
        torch.cuda.synchronize()
        got = [C.cpu().numpy() for C in Cs]
        Cs[0].fill_(float("nan"))
        torch.cuda.synchronize()
        gpu_ctx.set_stream(a.cuda_stream)
        call(0)
        torch.cuda.synchronize()
        again = Cs[0].cpu().numpy()
    finally:
        gpu_ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    assert info_a["column_phases"] == 7 and info_b["column_phases"] == 7, (info_a, info_b)
    check(got[0], probs[0][6])
    check(got[1], probs[1][6])
    check(again, probs[0][6])


def test_chain_check_resets_between_graph_replays(gpu_ctx):
    """A phased call captured into a graph, replayed over a chain, then over
    a list that is not a chain (the same tasks shuffled, written into the
    captured task array), then over the chain again: the last replay runs
    phased again (its C is bit-identical to the first replay's, and differs
    from the one-pass result, which rounds differently), and every replay
    matches the oracle.  One run of all tasks per wave (tasks_per_wave
    2^20) keeps every result deterministic."""
    torch = torch_mod()
    g = workloads.small(1, seed=17)
    K = 64
    p = problem(g, SKEWED_COSTS, 6)
    H_host = synth.features(g.n, K, 17)
    d_rp, d_ci, d_v, d_o = dev(p.row_ptr), dev(p.col_idx), dev(p.val), dev(p.origin)
    chain = np.ascontiguousarray(p.tasks, np.int32)
    shuffled = np.ascontiguousarray(chain[np.random.default_rng(3).permutation(len(chain))])
    d_t = dev(chain.reshape(-1))
    H = dev(H_host)
    C = torch.zeros((g.n, K), dtype=torch.float32, device="cuda")
    args = (d_rp, d_ci, d_v, d_o, g.n, g.nnz, H, g.n, K, d_t, len(chain), C)
    ctx = capi.Context(0, torch.cuda.current_stream().cuda_stream)
    try:
        set_phased(ctx, 4, 1 << 20, 1)
        ctx.spmm(*args, flags=capi.ZERO_OUTPUT)  # sizes the phase buffers
        phased_eager = C.cpu().numpy()
        ctx.set_column_phases(0)
        ctx.spmm(*args, flags=capi.ZERO_OUTPUT)
        one_pass = C.cpu().numpy()
        ctx.set_column_phases(4)
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            ctx.set_stream(side.cuda_stream)
            with torch.cuda.graph(graph, stream=side):
                ctx.spmm(*args, flags=capi.ZERO_OUTPUT, timed=False)
        ctx.set_stream(torch.cuda.current_stream().cuda_stream)
        assert ctx.last_launch()["column_phases"] == 4
        torch.cuda.synchronize()
        got = []
        for tasks in (chain, shuffled, chain):
            d_t.copy_(torch.from_numpy(tasks.reshape(-1)))
            C.fill_(float("nan"))
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            got.append(C.cpu().numpy())
        del graph
    finally:
        ctx.close()
    ref = oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H_host, chain)
    for c in got:
        check(c, ref)
    assert not np.array_equal(phased_eager, one_pass)  # the two paths are told apart
    assert np.array_equal(got[0], phased_eager)
    assert np.array_equal(got[2], got[0])


@pytest.mark.parametrize("P", [3, 16])
def test_duplicate_and_unsorted_columns(gpu_ctx, reset, rng, P):
    """Rows that repeat columns in any order, with non-unit values: the band
    sort keeps every copy (stable within a band) and the phased result is
    the reference's."""
    n = 3000
    deg = rng.integers(0, 60, n)
    rp = np.concatenate([[0], np.cumsum(deg)]).astype(np.int32)
    ci = rng.integers(0, 50, rp[-1]).astype(np.int32)  # many repeats per row
    val = rng.normal(size=rp[-1]).astype(np.float32)
    g = custom_graph(rp, ci, val)
    H = synth.features(n, 64, 3)
    for S in (2, 17):
        p = problem(g, SKEWED_COSTS, S)
        set_phased(gpu_ctx, P, 8, 2)
        got, _ = run_gpu(gpu_ctx, p, H)
        assert gpu_ctx.last_launch()["column_phases"] == P
        ref32, ref64 = oracle_pair(p, g, H)
        check(got, ref32)
        check(got, ref64)
