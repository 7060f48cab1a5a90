"""Host emulation of the column-phased aggregation.

With column phases (cwlb_ctx_set_column_phases, csrc/col_phases.hip and
the PH branch of csrc/spmm_mean.hip) a task list that is a chain -- every
task well formed and starting where its predecessor ended -- is executed
P times.  Phase p gathers only the nonzeros of each row between the row's
bounds B_p and B_{p+1}, where B_p(r) = row_ptr[r] + #{j in row r :
floor(col[j] * P / h_rows) < p}.  A run of M tasks takes, whole, every row
whose first nonzero lies in its tasks (the chain's first and last task keep
their offsets), so each row has one owner: it is stored in the first phase
and added to in the others.  Rows the chain covers only in part (its ends)
are added to in every phase, after the clearing pass of the one-pass
kernel.

This file restates those rules in Python and checks, against the oracle
(the reference's task-at-a-time semantics, src/parallelMatrix.cpp:148-236):
the partition's lists at many run lengths and phase counts, chains that
start and end inside rows, unsorted rows and columns outside the feature
matrix.  The bounds are checked against what they mean (every nonzero of
phase p's range lies in band p when the row is sorted), and planted
mistakes in the restated rules make the comparison fail.
"""
import numpy as np
import pytest

import oracle
from conftest import SKEWED_COSTS
from cwlb_amd import synth, workloads
from test_segments import cleared_rows, continues, row_chunk, well_formed


def is_chain(tasks, n_rows):
    """zero_split_rows' chain check."""
    return all(well_formed(t, n_rows) for t in tasks) and all(
        continues(tasks[i - 1], tasks[i]) for i in range(1, len(tasks)))


def bands(ci, h_rows, P):
    c = ci.astype(np.int64)
    return np.where(c < 0, 0, np.where(c >= h_rows, P - 1, c * P // max(h_rows, 1)))


def phase_bounds(rp, ci, h_rows, P):
    """cwlb_column_phase_bounds: out[p - 1][r] = B_p(r), p in [1, P)."""
    n, nnz = len(rp) - 1, len(ci)
    out = np.zeros((P - 1, n), np.int64)
    b = bands(ci, h_rows, P)
    p0, p1 = rp[:-1].astype(np.int64), rp[1:].astype(np.int64)
    ok = (p0 >= 0) & (p1 >= p0) & (p1 <= nnz)
    s0, s1 = np.where(ok, p0, 0), np.where(ok, p1, 0)
    for q in range(1, P):
        cs = np.concatenate([[0], np.cumsum(b < q)])
        out[q - 1] = np.where(ok, p0 + cs[s1] - cs[s0], 0)
    return out


def run_segments(tasks, M):
    """The (rs, re, fo, ln) of every run: rows whose first nonzero lies in
    the run, the chain's ends keeping their offsets (spmm_mean.hip, PH)."""
    T = len(tasks)
    zl = tasks[T - 1]
    out = []
    for t0 in range(0, T, M):
        a = tasks[t0]
        z = tasks[min(t0 + M, T) - 1]
        head = t0 == 0
        rs = int(a[0]) if (head or a[2] == 0) else int(a[0]) + 1
        fo = int(a[2]) if head else 0
        ln = int(zl[3]) if z[1] == zl[1] else 0
        if rs < z[1]:
            out.append((rs, int(z[1]), fo, ln))
    return out


def emulate_phased(rp, ci, val, origin, H, tasks, M, P, C0, rng, bounds=None,
                   segments_of=run_segments, later_phase_adds=True):
    """C after the clearing pass and the P phase launches (float64)."""
    n_rows, nnz = len(rp) - 1, len(ci)
    C = C0.astype(np.float64)
    for o in cleared_rows(rp, origin, tasks, M, n_rows, nnz):
        C[o] = 0.0
    B = phase_bounds(rp, ci, H.shape[0], P) if bounds is None else bounds
    segs = segments_of(tasks, M)
    for p in range(P):
        first = p == 0
        for k in rng.permutation(len(segs)):
            seg = segs[k]
            for r in range(max(seg[0], 0), min(seg[1], n_rows)):
                base, b, e, d = row_chunk(rp, r, seg, nnz)
                o = origin[r]
                if d < 0:
                    continue
                if d == 0:
                    if first:
                        C[o] = 0.0
                    continue
                own = b == 0 and e == d
                lo = 0 if p == 0 else min(max(int(B[p - 1, r]) - base, 0), d)
                hi = d if p == P - 1 else min(max(int(B[p, r]) - base, lo), d)
                b, e = max(b, lo), max(min(e, hi), max(b, lo))
                cols = ci[base + b:base + e]
                acc = (val[base + b:base + e, None].astype(np.float64) * H[cols]).sum(0) / d
                if own and first:
                    C[o] = acc
                elif own and not later_phase_adds:
                    C[o] = acc
                elif e > b:
                    C[o] += acc
    return C


def check(p, H, tasks, M, P, zero_output, rng, **kw):
    ref = oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H, tasks)
    C0 = np.zeros((p.n, H.shape[1])) if zero_output else np.full((p.n, H.shape[1]), np.nan)
    got = emulate_phased(p.row_ptr, p.col_idx, p.val, p.origin, H.astype(np.float64), tasks, M,
                         P, C0, rng, **kw)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-6)


def small_problem(cfg, S, seed):
    g = workloads.small(cfg, seed=seed)
    p = workloads.prepare(g, SKEWED_COSTS, S)
    H = synth.features(g.n, 3, seed)
    return p, H


@pytest.mark.parametrize(
    "cfg,S,P,M", [(3, 6, P, M) for P in (2, 5, 16) for M in (1, 3, 16, 64, 200)]
    + [(4, 3, 2, 3), (4, 3, 5, 64), (4, 3, 16, 1), (4, 3, 3, 200)])
def test_partition_lists(cfg, S, P, M):
    """The partition's lists are chains; every row has one owner run; the
    phases give the reference's result with C not cleared beforehand."""
    p, H = small_problem(cfg, S, 2)
    assert is_chain(p.tasks, p.n)
    segs = run_segments(p.tasks, M)
    owners = np.zeros(p.n, np.int64)
    for rs, re, _, _ in segs:
        owners[rs:re] += 1
    assert (owners == 1).all()
    check(p, H, p.tasks, M, P, zero_output=False, rng=np.random.default_rng(P * M))


@pytest.mark.parametrize("M", [1, 4, 64])
def test_chains_that_start_and_end_inside_rows(M):
    """Sub-lists of the partition's list start and end inside split rows:
    the chain's first and last rows are partial and added to; rows outside
    keep C's contents (the reference's zeroed C here)."""
    rng = np.random.default_rng(M)
    p, H = small_problem(4, 3, 5)
    split = np.nonzero(p.tasks[:, 2] > 0)[0]
    assert len(split) > 10
    for _ in range(6):
        k, j = np.sort(rng.choice(split, 2, replace=False))
        sub = p.tasks[k:j + 1]
        assert sub[0, 2] > 0
        check(p, H, sub, M, 4, zero_output=True, rng=rng)


def test_bounds_split_rows_into_bands():
    """Sorted rows: every nonzero of phase p's range has band p, the bounds
    are non-decreasing and within the row; unsorted rows are still split
    exactly (the phases partition each row)."""
    rng = np.random.default_rng(0)
    n, h = 300, 1000
    deg = rng.integers(0, 40, n)
    rp = np.concatenate([[0], np.cumsum(deg)]).astype(np.int64)
    ci = rng.integers(0, h, rp[-1])
    ci_sorted = ci.copy()
    for r in range(n):
        ci_sorted[rp[r]:rp[r + 1]].sort()
    for P in (2, 7, 64):
        B = phase_bounds(rp, ci_sorted, h, P)
        full = np.concatenate([rp[None, :-1], B, rp[None, 1:]])
        assert (np.diff(full, axis=0) >= 0).all()
        bnd = bands(ci_sorted, h, P)
        for q in range(P):
            for r in range(0, n, 17):
                assert (bnd[full[q, r]:full[q + 1, r]] == q).all()
        # unsorted: the counts per phase are still the band sizes
        Bu = phase_bounds(rp, ci, h, P)
        fu = np.concatenate([rp[None, :-1], Bu, rp[None, 1:]])
        bu = bands(ci, h, P)
        for r in range(0, n, 13):
            for q in range(P):
                assert fu[q + 1, r] - fu[q, r] == (bu[rp[r]:rp[r + 1]] == q).sum()


def test_unsorted_rows_and_foreign_bounds():
    """Unsorted rows and bounds built for other contents of col_idx only
    move nonzeros between phases: the result is the reference's."""
    rng = np.random.default_rng(3)
    p, H = small_problem(3, 6, 4)
    ci = p.col_idx.copy()
    for r in range(p.n):
        seg = ci[p.row_ptr[r]:p.row_ptr[r + 1]]
        rng.shuffle(seg)
    p.col_idx = ci
    check(p, H, p.tasks, 16, 6, zero_output=False, rng=rng)
    other = rng.integers(0, p.n, len(ci)).astype(np.int32)
    check(p, H, p.tasks, 16, 6, zero_output=False, rng=rng,
          bounds=phase_bounds(p.row_ptr, other, p.n, 6))


def test_planted_mistakes_fail():
    """Each plausible mistake in the run rule or the phase writes breaks
    the comparison: no +1 for a run that starts inside a row begun
    earlier, the chain's last offset or first offset dropped, a later
    phase storing instead of adding."""
    rng = np.random.default_rng(7)
    p, H = small_problem(4, 3, 5)
    split = np.nonzero(p.tasks[:, 2] > 0)[0]
    k, j = split[len(split) // 3], split[2 * len(split) // 3]
    sub = p.tasks[k:j + 1]
    ref = oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H, sub)
    zeros = np.zeros((p.n, H.shape[1]))

    def differs(tasks, **kw):
        got = emulate_phased(p.row_ptr, p.col_idx, p.val, p.origin, H.astype(np.float64), tasks,
                             8, 4, zeros, rng, **kw)
        return not np.allclose(got, oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin,
                                                         H, tasks), rtol=1e-5, atol=1e-6)

    assert not differs(sub)
    assert np.isfinite(ref).all()

    def no_plus_one(tasks, M):
        segs = []
        for t0 in range(0, len(tasks), M):
            a, z = tasks[t0], tasks[min(t0 + M, len(tasks)) - 1]
            segs.append((int(a[0]), int(z[1]), int(a[2]) if t0 == 0 else 0,
                         int(tasks[-1][3]) if z[1] == tasks[-1][1] else 0))
        return segs

    def no_tail(tasks, M):
        return [(rs, re, fo, 0) for rs, re, fo, _ in run_segments(tasks, M)]

    def no_head(tasks, M):
        return [(rs, re, 0, ln) for rs, re, _, ln in run_segments(tasks, M)]

    assert differs(sub, segments_of=no_plus_one)
    assert differs(sub, segments_of=no_tail)
    assert differs(sub, segments_of=no_head)
    assert differs(sub, later_phase_adds=False)


def test_broken_lists_are_not_chains():
    """Shuffled, gapped or malformed lists fail the chain check (they run
    in one pass)."""
    p, _ = small_problem(4, 3, 5)
    rng = np.random.default_rng(1)
    assert not is_chain(p.tasks[rng.permutation(len(p.tasks))], p.n)
    assert not is_chain(np.delete(p.tasks, len(p.tasks) // 2, 0), p.n)
    bad = p.tasks.copy()
    bad[5] = [3, 3, 0, 0]
    assert not is_chain(bad, p.n)
