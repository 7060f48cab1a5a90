"""Pins the oracle (oracle/oracle.c) before the other tests rely on it.

Checks, per function:
  partition   the reference's own costWeightedTaskPartitioning compiled from
              /root/reference (oracle/_ref), hand-derived known answers and
              tiling invariants;
  reorder     numpy's stable argsort of the degrees (closed form);
  aggregation the fp64 closed form, scipy, dense brute force on tiny graphs,
              exact special cases (degree-1 rows, all-ones features, K = 1);
  S selection the reference extract and the README's worked examples;
  cost file   byte-identical output with the reference's writer.
Planted mistakes (oracle_set_mutation) must each fail one of these checks.
"""
import numpy as np
import pytest
import scipy.sparse as sp

import oracle
from conftest import SKEWED_COSTS, UNIT_COSTS
from cwlb_amd import synth, workloads

need_ref = pytest.mark.skipif(not oracle.ref_built(), reason="oracle/_ref not built (no /root/reference)")


def rp_of(degs):
    return np.concatenate([[0], np.cumsum(degs)]).astype(np.int32)


# Appendix-style known answers derived by hand from utils.cpp:832-1021 with
# Cc=0.25 Cl=0.75 Cs=0.5 Ca=0.5 (wCL=1), capacity_from_s(4)=4.5, S=4.
KATS = [
    ([1, 1, 2, 10], [(0, 2, 0, 0), (2, 3, 0, 0), (3, 4, 0, 4), (3, 4, 4, 8), (3, 4, 8, 0)]),
    ([1, 10], [(0, 2, 0, 2), (1, 2, 2, 6), (1, 2, 6, 0)]),
    ([6, 9], [(0, 1, 0, 4), (0, 2, 4, 1), (1, 2, 1, 5), (1, 2, 5, 0)]),
    ([1, 8], [(0, 1, 0, 0), (1, 2, 0, 4), (1, 2, 4, 0)]),
    ([0, 0, 3], [(0, 3, 0, 0)]),
    ([], []),
    ([4], [(0, 1, 0, 0)]),
    ([5], [(0, 1, 0, 4), (0, 1, 4, 0)]),
]


def tasks_list(t):
    return [tuple(int(x) for x in row) for row in t]


@pytest.mark.parametrize("degs,expected", KATS)
def test_partition_known_answers(degs, expected):
    cap = oracle.capacity_from_s(4, UNIT_COSTS)
    assert cap == 4.5
    assert tasks_list(oracle.partition(rp_of(degs), UNIT_COSTS, cap)) == expected
    if oracle.ref() is not None:
        assert tasks_list(oracle.ref_partition(rp_of(degs), UNIT_COSTS, cap)) == expected


def chunks_of(rp, tasks):
    """Expands tasks into (row, begin, end) chunks with the kernel's clamps."""
    out = []
    for rs, re, fo, ln in tasks:
        for r in range(rs, re):
            d = rp[r + 1] - rp[r]
            b = fo if r == rs else 0
            e = ln if (r == re - 1 and ln > 0) else d
            b = min(max(b, 0), d)
            e = min(max(e, b), d)
            out.append((r, b, e))
    return out


def assert_tiling(rp, tasks, S):
    """Tasks cover every nonzero exactly once, in order; segments of split rows <= S."""
    n = len(rp) - 1
    assert all(s < e for s, e, _, _ in tasks), "empty task"
    pos = {r: 0 for r in range(n)}
    seen = set()
    for r, b, e in chunks_of(rp, tasks):
        d = rp[r + 1] - rp[r]
        if d == 0:
            assert r not in seen
            seen.add(r)
            continue
        if b == e:
            continue
        assert b == pos[r], f"row {r}: chunk starts at {b}, expected {pos[r]}"
        pos[r] = e
        if not (b == 0 and e == d):
            assert e - b <= S or b == 0, f"row {r}: segment {b}:{e} longer than S={S}"
    for r in range(n):
        d = rp[r + 1] - rp[r]
        assert pos[r] == d or (d == 0 and r in seen), f"row {r} not fully covered"


def random_degrees(rng):
    n = int(rng.integers(0, 80))
    kind = rng.integers(0, 4)
    if kind == 0:
        return np.sort(rng.integers(0, rng.integers(1, 100), n))
    if kind == 1:
        return np.sort(rng.zipf(1.6, n).clip(0, 5000) - 1)
    if kind == 2:
        return rng.integers(0, 40, n)
    return np.sort(np.concatenate([np.zeros(n // 2, int), rng.integers(20, 300, n - n // 2)]))


COST_CHOICES = [0.0, 0.01, 0.125, 0.25, 0.5, 1.0, 1.7, 3.3, 12.5]


@need_ref
def test_partition_matches_reference_random(rng):
    for _ in range(4000):
        degs = random_degrees(rng)
        rp = rp_of(degs)
        costs = tuple(float(rng.choice(COST_CHOICES)) for _ in range(4))
        if rng.random() < 0.8:
            cap = oracle.capacity_from_s(int(rng.integers(1, 60)), costs)
        else:
            cap = float(rng.random() * 60)
        a = oracle.partition(rp, costs, cap)
        b = oracle.ref_partition(rp, costs, cap)
        assert np.array_equal(a, b), (degs.tolist(), costs, cap)


@need_ref
@pytest.mark.parametrize("cfg", [1, 2, 3, 4, 5])
def test_partition_matches_reference_on_workloads(cfg):
    g = workloads.small(cfg)
    origin, rp, _, _ = oracle.reorder_by_degree(g.row_ptr, g.col_idx, g.val)
    for costs in (UNIT_COSTS, SKEWED_COSTS, (0.0171, 0.4126, 0.0532, 2.2409)):
        for S in workloads.candidate_s(g.nnz, 256) + [1, 3, 64]:
            cap = oracle.capacity_from_s(S, costs)
            a = oracle.partition(rp, costs, cap)
            b = oracle.ref_partition(rp, costs, cap)
            assert np.array_equal(a, b)
            assert_tiling(rp, a, S)


def test_partition_invariants_random(rng):
    for _ in range(1500):
        degs = random_degrees(rng)
        rp = rp_of(degs)
        costs = tuple(float(rng.choice([0.125, 0.25, 0.5, 1.0, 1.7])) for _ in range(4))
        S = int(rng.integers(1, 40))
        cap = oracle.capacity_from_s(S, costs)
        tasks = oracle.partition(rp, costs, cap)
        wcl = costs[0] + costs[1]
        S_eff = max(1, int(np.floor((cap - costs[3]) / wcl)))
        assert_tiling(rp, tasks, S_eff)


# ------------------------------------------------------------------ reorder
@pytest.mark.parametrize("cfg", [1, 2, 4, 5])
def test_reorder_is_stable_degree_argsort(cfg):
    g = workloads.small(cfg)
    origin, rp, ci, val = oracle.reorder_by_degree(g.row_ptr, g.col_idx, g.val)
    deg = np.diff(g.row_ptr)
    assert np.array_equal(origin, np.argsort(deg, kind="stable"))
    assert np.array_equal(np.diff(rp), deg[origin])
    for r in range(0, g.n, max(1, g.n // 500)):
        o = origin[r]
        assert np.array_equal(ci[rp[r]:rp[r + 1]], g.col_idx[g.row_ptr[o]:g.row_ptr[o + 1]])


def test_reorder_edge_cases():
    origin, rp, ci, val = oracle.reorder_by_degree(np.zeros(1, np.int32), np.zeros(0, np.int32),
                                                   np.zeros(0, np.float32))
    assert len(origin) == 0 and rp.tolist() == [0]
    origin, rp, _, _ = oracle.reorder_by_degree(rp_of([3, 0, 3, 1, 0]), np.arange(7, dtype=np.int32),
                                                np.ones(7, np.float32))
    assert origin.tolist() == [1, 4, 3, 0, 2]
    assert rp.tolist() == [0, 0, 0, 1, 4, 7]


# -------------------------------------------------------------- aggregation
def random_graph(rng, n, max_deg, K, vals=False):
    deg = rng.integers(0, max_deg + 1, n)
    rp = rp_of(deg)
    ci = rng.integers(0, n, rp[-1]).astype(np.int32)
    val = (rng.normal(size=rp[-1]) if vals else np.ones(rp[-1])).astype(np.float32)
    H = rng.uniform(-1, 1, (n, K)).astype(np.float32)
    return synth.Graph(n, rp, ci, val), H


def run_oracle(g, H, costs, S):
    origin, rp, ci, val = oracle.reorder_by_degree(g.row_ptr, g.col_idx, g.val)
    tasks = oracle.partition(rp, costs, oracle.capacity_from_s(S, costs))
    return oracle.spmm_mean_f32(rp, ci, val, origin, H, tasks), (origin, rp, ci, val, tasks)


def test_aggregation_brute_force_dense(rng):
    for _ in range(30):
        n = int(rng.integers(1, 40))
        g, H = random_graph(rng, n, 12, int(rng.integers(1, 9)), vals=True)
        A = np.zeros((n, n), np.float64)
        for i in range(n):
            for j in range(g.row_ptr[i], g.row_ptr[i + 1]):
                A[i, g.col_idx[j]] += g.val[j]
        deg = np.diff(g.row_ptr).astype(np.float64)
        exp = (A @ H.astype(np.float64)) / np.where(deg > 0, deg, 1)[:, None]
        got, _ = run_oracle(g, H, UNIT_COSTS, int(rng.integers(1, 6)))
        np.testing.assert_allclose(got, exp, rtol=1e-5, atol=1e-6)


def test_aggregation_matches_closed_form_and_scipy(rng):
    g, H = random_graph(rng, 3000, 60, 16, vals=True)
    got, _ = run_oracle(g, H, SKEWED_COSTS, 5)
    exp64 = oracle.spmm_mean_f64(g.row_ptr, g.col_idx, g.val, H)
    A = sp.csr_matrix((g.val.astype(np.float64), g.col_idx, g.row_ptr), shape=(g.n, g.n))
    deg = np.diff(g.row_ptr)
    exp_sp = (A @ H.astype(np.float64)) / np.where(deg > 0, deg, 1)[:, None]
    np.testing.assert_allclose(exp64, exp_sp, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(got, exp64, rtol=1e-5, atol=1e-6)


def test_aggregation_exact_special_cases(rng):
    # Degree-1 rows: C = fl(v * H[c]) exactly; all-ones H: 1 exactly; deg 0: 0.
    n = 500
    deg = rng.integers(0, 2, n)
    deg[::7] = 0
    rp = rp_of(deg)
    ci = rng.integers(0, n, rp[-1]).astype(np.int32)
    val = rng.normal(size=rp[-1]).astype(np.float32)
    g = synth.Graph(n, rp, ci, val)
    H = rng.uniform(-1, 1, (n, 8)).astype(np.float32)
    got, _ = run_oracle(g, H, UNIT_COSTS, 2)
    for i in range(n):
        if deg[i] == 0:
            assert not got[i].any()
        else:
            j = rp[i]
            assert np.array_equal(got[i], (val[j] * H[ci[j]]).astype(np.float32))
    g2, _ = random_graph(rng, 800, 50, 4)
    got1, _ = run_oracle(g2, np.ones((800, 4), np.float32), UNIT_COSTS, 1000)
    d2 = np.diff(g2.row_ptr)
    assert np.array_equal(got1, np.where(d2 > 0, 1.0, 0.0).astype(np.float32)[:, None] *
                          np.ones((1, 4), np.float32))


def test_aggregation_k1_is_spmv(rng):
    g, H = random_graph(rng, 2000, 30, 1, vals=True)
    got, _ = run_oracle(g, H, SKEWED_COSTS, 3)
    A = sp.csr_matrix((g.val.astype(np.float64), g.col_idx, g.row_ptr), shape=(g.n, g.n))
    deg = np.diff(g.row_ptr)
    exp = (A @ H[:, 0].astype(np.float64)) / np.where(deg > 0, deg, 1)
    np.testing.assert_allclose(got[:, 0], exp, rtol=1e-5, atol=1e-6)


def test_aggregation_full_rows_independent_of_partition(rng):
    # Rows never split (S >= max degree) give bit-identical results for any costs.
    g, H = random_graph(rng, 1500, 40, 8, vals=True)
    a, _ = run_oracle(g, H, UNIT_COSTS, 100)
    b, _ = run_oracle(g, H, SKEWED_COSTS, 100)
    assert np.array_equal(a, b)


def test_cpu_baseline_matches_oracle(rng):
    g = workloads.small(4, seed=2)
    H = synth.features(g.n, 32, 3)
    got, (origin, rp, ci, val, tasks) = run_oracle(g, H, SKEWED_COSTS, 8)
    omp = oracle.spmm_mean_f32_omp(rp, ci, val, origin, H, tasks, threads=4)
    np.testing.assert_allclose(omp, got, rtol=1e-5, atol=1e-6)


# ----------------------------------------------------------- S selection
def test_s_selection_readme_examples():
    # README.md:289  S = max(1, ceil(NNZ / (CU * w)))
    assert oracle.wave_based_s(65_245_138, 2, 256, 8192) == 32
    assert oracle.wave_based_s(65_245_138, 2, 256, 4096) == 63
    assert oracle.wave_based_s(65_245_138, 2, 256, 2048) == 125
    assert oracle.wave_based_s(0, 2, 256, 64) == 1
    assert oracle.wave_based_s(5, 0, 256, 64) == 1
    assert oracle.wave_based_s(5, 2, 0, 64) == -1
    assert oracle.recommended_candidate_w(65_245_138) == [8192, 4096, 2048]
    assert oracle.recommended_candidate_w(10_556) == [64, 32, 16]
    assert oracle.recommended_candidate_w(49_999_999) == [4096, 2048, 1024]
    # README.md:306-310 search intervals for S1 <= S2 <= S3.
    assert oracle.candidate_search_bounds([10, 20, 40], 0) == (1, 20)
    assert oracle.candidate_search_bounds([10, 20, 40], 1) == (10, 40)
    assert oracle.candidate_search_bounds([10, 20, 40], 2) == (20, 60)
    assert oracle.candidate_search_bounds([5, 20, 40], 0) == (1, 20)
    # README.md:342-345 step grid keeps the upper endpoint.
    assert oracle.candidate_search_by_step(20, 60, 15) == [20, 35, 50, 60]
    assert oracle.candidate_search_by_step(20, 60, 20) == [20, 40, 60]
    # Six near-uniform points including both endpoints; count 1 is the midpoint.
    assert oracle.candidate_search_by_count(10, 40, 6) == [10, 16, 22, 28, 34, 40]
    assert oracle.candidate_search_by_count(10, 40, 1) == [25]
    assert oracle.candidate_search_by_count(3, 5, 6) == [3, 4, 5]
    with pytest.raises(ValueError):
        oracle.candidate_search_by_step(1, 20000, 1)


@need_ref
def test_s_selection_matches_reference(rng):
    import ctypes as C
    R = oracle.ref()
    for _ in range(3000):
        nnz = int(rng.integers(0, 2**40))
        out_a, out_b = np.zeros(3, np.int32), np.zeros(3, np.int32)
        R.cwlbref_recommended_candidate_w(nnz, out_b)
        assert oracle.recommended_candidate_w(nnz) == out_b.tolist()
        s = int(rng.integers(-3, 300))
        costs = tuple(float(rng.choice(COST_CHOICES + [-1.0])) for _ in range(4))
        assert oracle.capacity_from_s(s, costs) == R.cwlbref_capacity_from_s(s, *costs)
        cu, w = int(rng.integers(-1, 300)), int(rng.integers(-1, 9000))
        rp = np.array([0, min(nnz, 2**31 - 1)], np.int32)
        err = C.c_int()
        sref = R.cwlbref_wave_based_s(rp, 2, cu, w, C.byref(err))
        so = oracle.wave_based_s(int(rp[-1]), 2, cu, w)
        assert (so == -1) == (err.value == 1)
        if err.value == 0:
            assert so == sref
        v = np.sort(rng.integers(0, 50, 3)).astype(np.int32)
        best = int(rng.integers(-1, 4))
        lo, hi = C.c_int(), C.c_int()
        rc = R.cwlbref_candidate_search_bounds(v, best, C.byref(lo), C.byref(hi))
        if rc:
            with pytest.raises(ValueError):
                oracle.candidate_search_bounds(v, best)
        else:
            assert oracle.candidate_search_bounds(v, best) == (lo.value, hi.value)
        a, b, c = (int(x) for x in rng.integers(-2, 200, 3))
        for ofn, rfn in ((oracle.candidate_search_by_count, R.cwlbref_candidate_search_by_count),
                         (oracle.candidate_search_by_step, R.cwlbref_candidate_search_by_step)):
            buf = np.zeros(20000, np.int32)
            n = rfn(a, b, c, buf, len(buf), C.byref(err))
            if err.value:
                with pytest.raises(ValueError):
                    ofn(a, b, c)
            else:
                assert ofn(a, b, c) == buf[:n].tolist()


# --------------------------------------------------------------- cost file
@need_ref
@pytest.mark.parametrize("c4", [(0.25, 0.75, 0.5, 0.5), (0.0123456789, 12.3456789, 1e-9, 123456.7),
                                (1.0000005, 2.4999995, 0.0, 3.0)])
def test_cost_file_format_matches_reference(c4):
    for prec in (6, 3, 10):
        assert oracle.format_costs(c4, prec) == oracle.ref_format_costs(c4, prec)
    txt = oracle.format_costs(c4)
    assert oracle.parse_costs(txt) == [float(f"{x:.6f}") for x in c4]


# ------------------------------------------------------ planted mistakes
@pytest.mark.parametrize("m", [1, 2, 3])
def test_planted_partition_mistakes_are_caught(m):
    """Each partition mutation fails a known answer or the reference comparison."""
    cap = oracle.capacity_from_s(4, UNIT_COSTS)
    caught = False
    try:
        oracle.set_mutation(m)
        for degs, expected in KATS:
            if tasks_list(oracle.partition(rp_of(degs), UNIT_COSTS, cap)) != expected:
                caught = True
        if oracle.ref() is not None and not caught:
            rng = np.random.default_rng(0)
            for _ in range(500):
                rp = rp_of(random_degrees(rng))
                if not np.array_equal(oracle.partition(rp, UNIT_COSTS, cap),
                                      oracle.ref_partition(rp, UNIT_COSTS, cap)):
                    caught = True
                    break
    finally:
        oracle.set_mutation(0)
    assert caught


def test_planted_aggregation_mistake_is_caught(rng):
    g, H = random_graph(rng, 400, 30, 4)
    exp64 = oracle.spmm_mean_f64(g.row_ptr, g.col_idx, g.val, H)
    try:
        oracle.set_mutation(4)
        got, _ = run_oracle(g, H, UNIT_COSTS, 3)
    finally:
        oracle.set_mutation(0)
    assert not np.allclose(got, exp64, rtol=1e-5, atol=1e-6)


def test_planted_reorder_mistake_is_caught():
    g = workloads.small(4, seed=2)
    try:
        oracle.set_mutation(5)
        origin, _, _, _ = oracle.reorder_by_degree(g.row_ptr, g.col_idx, g.val)
    finally:
        oracle.set_mutation(0)
    assert not np.array_equal(origin, np.argsort(np.diff(g.row_ptr), kind="stable"))


# ------------------------------------------------- calibration normalisation
# Hand-derived from utils.cpp:419-421, 522-524, 583-585 (ns per op per
# work-item x 10) and 597-640, 791-806 (atomic: writer groups rounded up to a
# multiple of the writers per address, ops = groups x K_block).  The inputs
# are chosen so that every coefficient is an exact binary fraction.
CAL_KATS = [
    # ms (compute, load, store, atomic), K, WI, writers -> ops, coefficients
    ((1.0, 2.0, 0.5, 4.0), 128, 131072, 8,
     (16777216, 16777216, 16777216, 131072),   # 1024 groups x K_block 128
     (78125 / 2**17, 2 * 78125 / 2**17, 78125 / 2**18, 305.17578125)),
    # K = 40: K_block 32; ceil(1000 / 128) = 8 groups wanted, 8 // 3 = 2
    # rows give 6 < 8, so 3 rows of 3 writers: 9 groups, 288 atomics.
    ((0.25, 0.25, 0.25, 0.0288), 40, 1000, 3,
     (40000, 40000, 40000, 288),
     (0.25e6 / 1000 / 40 * 10,) * 3 + (1000.0,)),
    # K = 20 rounds K_block down to 0, which becomes 32; 1 writer.
    ((0.5, 0.5, 0.5, 0.5), 20, 64, 1,
     (1280, 1280, 1280, 32), (0.5e6 / 64 / 20 * 10,) * 3 + (0.5e6 / 32 * 10,)),
]


@pytest.mark.parametrize("case", range(len(CAL_KATS)))
def test_calibration_normalisation_known_answers(case):
    ms, K, WI, writers, ops, coef = CAL_KATS[case]
    got, got_ops = oracle.cost_coefficients(ms, K, WI, writers)
    assert got_ops == list(ops)
    assert got == pytest.approx(list(coef), rel=1e-15)
    if case == 0:
        assert got == list(coef)  # exact binary fractions


def test_planted_calibration_mistake_is_caught():
    ms, K, WI, writers, ops, coef = CAL_KATS[1]
    try:
        oracle.set_mutation(7)
        got, got_ops = oracle.cost_coefficients(ms, K, WI, writers)
    finally:
        oracle.set_mutation(0)
    assert got_ops[3] != ops[3] and got[3] != pytest.approx(coef[3])
