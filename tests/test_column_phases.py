"""Host emulation of the column-phased aggregation.

With column phases (cwlb_ctx_set_column_phases, csrc/col_phases.hip and
the PH branch of csrc/spmm_mean.hip) a task list that is a chain -- every
task well formed and starting where its predecessor ended -- is executed
P times.  The bands interleave the columns: band(c) = c mod P.  Each call
first writes a copy of the column and value arrays with every row's
nonzeros stably sorted by band, and the bounds B_p(r) = row_ptr[r] +
#{j in row r : band(col[j]) < p}; phase p gathers the copy's range
[B_p(r), B_{p+1}(r)) of each row.  A run of M tasks takes, whole, every row
whose first nonzero lies in its tasks, so each row has one owner: it is
stored in the first phase and added to in the others.  Task offsets index
the caller's order of a row's nonzeros, so the rows the chain covers only
in part (its first row when it starts inside it, its last when it ends at
an offset) are summed whole from the caller's arrays in the first phase,
with the one-pass rules (after the one-pass clearing pass).

This file restates those rules in Python and checks, against the oracle
(the reference's task-at-a-time semantics, src/parallelMatrix.cpp:148-236):
the partition's lists at many run lengths and phase counts, chains that
start and end inside rows, unsorted rows and columns outside the feature
matrix.  The band sort is checked against what it means (the copy is a
per-row permutation of the row's nonzeros, band p of a row is exactly its
band-p nonzeros, in their original order), and planted mistakes in the
restated rules make the comparison fail.
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
    """band_of in col_phases.hip: c mod P, columns outside [0, h_rows) in band 0."""
    c = ci.astype(np.int64)
    return np.where((c < 0) | (c >= h_rows), 0, c % P)


def row_ok(rp, nnz):
    p0, p1 = rp[:-1].astype(np.int64), rp[1:].astype(np.int64)
    return (p0 >= 0) & (p1 >= p0) & (p1 <= nnz)


def phase_bounds(rp, ci, h_rows, P):
    """cwlb_column_phase_sort: out[p - 1][r] = B_p(r), p in [1, P)."""
    n, nnz = len(rp) - 1, len(ci)
    out = np.zeros((P - 1, n), np.int64)
    b = bands(ci, h_rows, P)
    ok = row_ok(rp, nnz)
    p0 = rp[:-1].astype(np.int64)
    s0, s1 = np.where(ok, p0, 0), np.where(ok, rp[1:].astype(np.int64), 0)
    for q in range(1, P):
        cs = np.concatenate([[0], np.cumsum(b < q)])
        out[q - 1] = np.where(ok, p0 + cs[s1] - cs[s0], 0)
    return out


def band_copy(rp, ci, val, h_rows, P):
    """The band-sorted copy: each well-formed row's nonzeros stably sorted
    by band (rows with bad offsets are not copied: left as `fill`)."""
    ci_b, val_b = np.zeros_like(ci), np.zeros_like(val)
    b = bands(ci, h_rows, P)
    ok = row_ok(rp, len(ci))
    for r in np.nonzero(ok)[0]:
        p0, p1 = int(rp[r]), int(rp[r + 1])
        order = np.argsort(b[p0:p1], kind="stable")
        ci_b[p0:p1] = ci[p0:p1][order]
        val_b[p0:p1] = val[p0:p1][order]
    return ci_b, val_b


def run_pieces(tasks, M):
    """The pieces every run executes (spmm_mean.hip, PH branch): (rs, re,
    fo, ln, banded) -- the whole rows whose first nonzero lies in the run,
    band by band; the chain's partial first and last rows at the task
    offsets, from the caller's arrays, in the first phase only."""
    T = len(tasks)
    zl = tasks[T - 1]
    out = []
    for t0 in range(0, T, M):
        a = tasks[t0]
        z = tasks[min(t0 + M, T) - 1]
        head = t0 == 0
        rs = int(a[0]) if (head or a[2] == 0) else int(a[0]) + 1
        re = int(z[1])
        fo = int(a[2]) if head else 0
        ln = int(zl[3]) if z[1] == zl[1] else 0
        if rs >= re:
            continue
        bs = rs + (1 if fo > 0 else 0)
        be = max(bs, re - (1 if ln > 0 else 0))
        if bs < be:
            out.append((bs, be, 0, 0, True))
        if fo > 0:
            out.append((rs, rs + 1, fo, ln if (ln > 0 and re == rs + 1) else 0, False))
        if ln > 0 and not (fo > 0 and re == rs + 1):
            out.append((re - 1, re, 0, ln, False))
    return out


def emulate_phased(rp, ci, val, origin, H, tasks, M, P, C0, rng, copy=None,
                   pieces_of=run_pieces, later_phase_adds=True):
    """C after the clearing pass and the P phase launches (float64)."""
    n_rows, nnz = len(rp) - 1, len(ci)
    C = C0.astype(np.float64)
    for o in cleared_rows(rp, origin, tasks, M, n_rows, nnz):
        C[o] = 0.0
    B = phase_bounds(rp, ci, H.shape[0], P)
    ci_b, val_b = band_copy(rp, ci, val, H.shape[0], P) if copy is None else copy
    pieces = pieces_of(tasks, M)
    for p in range(P):
        first = p == 0
        for k in rng.permutation(len(pieces)):
            rs, re, fo, ln, banded = pieces[k]
            if not banded and not first:
                continue
            cx, vx = (ci_b, val_b) if banded else (ci, val)
            for r in range(max(rs, 0), min(re, n_rows)):
                base, b, e, d = row_chunk(rp, r, (rs, re, fo, ln), nnz)
                o = origin[r]
                if d < 0:
                    continue
                if d == 0:
                    if first:
                        C[o] = 0.0
                    continue
                own = b == 0 and e == d
                if banded:
                    lo = 0 if p == 0 else min(max(int(B[p - 1, r]) - base, 0), d)
                    hi = d if p == P - 1 else min(max(int(B[p, r]) - base, lo), d)
                    b, e = max(b, lo), max(min(e, hi), max(b, lo))
                cols = cx[base + b:base + e]
                acc = (vx[base + b:base + e, None].astype(np.float64) * H[cols]).sum(0) / d
                if own and (first or not later_phase_adds):
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
    owners = np.zeros(p.n, np.int64)
    for rs, re, _, _, banded in run_pieces(p.tasks, M):
        assert banded  # the partition's chain starts and ends on row boundaries
        owners[rs:re] += 1
    assert (owners == 1).all()
    check(p, H, p.tasks, M, P, zero_output=False, rng=np.random.default_rng(P * M))


@pytest.mark.parametrize("M", [1, 4, 64])
def test_chains_that_start_and_end_inside_rows(M):
    """Sub-lists of the partition's list start and end inside split rows:
    the chain's first and last rows are partial, summed from the caller's
    arrays and added to; rows outside keep C's contents (the reference's
    zeroed C here)."""
    rng = np.random.default_rng(M)
    p, H = small_problem(4, 3, 5)
    split = np.nonzero(p.tasks[:, 2] > 0)[0]
    assert len(split) > 10
    for _ in range(6):
        k, j = np.sort(rng.choice(split, 2, replace=False))
        sub = p.tasks[k:j + 1]
        assert sub[0, 2] > 0
        owners = np.zeros(p.n, np.int64)
        for rs, re, _, _, _ in run_pieces(sub, M):
            owners[rs:re] += 1
        assert owners.max() == 1
        check(p, H, sub, M, 4, zero_output=True, rng=rng)
    # a chain inside one row
    one = np.nonzero((p.tasks[:, 2] > 0) & (p.tasks[:, 3] > 0))[0]
    sub = p.tasks[one[0]:one[0] + 1]
    assert run_pieces(sub, 1) == [(int(sub[0, 0]), int(sub[0, 1]), int(sub[0, 2]),
                                   int(sub[0, 3]), False)]
    check(p, H, sub, 1, 3, zero_output=True, rng=rng)


def test_band_sort_meaning():
    """The copy is each row's nonzeros, stably sorted by band (c mod P):
    the copy's range [B_p, B_{p+1}) of a row holds exactly the row's band-p
    nonzeros, in their original order; columns outside [0, h_rows) are in
    band 0; rows with bad offsets get bounds 0."""
    rng = np.random.default_rng(0)
    n, h = 300, 1000
    deg = rng.integers(0, 40, n)
    rp = np.concatenate([[0], np.cumsum(deg)]).astype(np.int64)
    ci = rng.integers(-2, h + 3, rp[-1])
    val = rng.normal(size=rp[-1]).astype(np.float32)
    for P in (2, 7, 64):
        B = phase_bounds(rp, ci, h, P)
        full = np.concatenate([rp[None, :-1], B, rp[None, 1:]])
        assert (np.diff(full, axis=0) >= 0).all()
        ci_b, val_b = band_copy(rp, ci, val, h, P)
        for r in range(0, n, 7):
            row = slice(rp[r], rp[r + 1])
            c, v = ci[row], val[row]
            b = np.where((c < 0) | (c >= h), 0, c % P)
            for q in range(P):
                got_c = ci_b[full[q, r]:full[q + 1, r]]
                got_v = val_b[full[q, r]:full[q + 1, r]]
                assert np.array_equal(got_c, c[b == q]) and np.array_equal(got_v, v[b == q])
    bad = rp.copy()
    bad[10] = bad[11] + 3
    assert (phase_bounds(bad, ci, h, 5)[:, 10] == 0).all()


def test_unsorted_rows():
    """Rows whose columns are in any order: the result is the reference's."""
    rng = np.random.default_rng(3)
    p, H = small_problem(3, 6, 4)
    ci = p.col_idx.copy()
    for r in range(p.n):
        seg = ci[p.row_ptr[r]:p.row_ptr[r + 1]]
        rng.shuffle(seg)
    p.col_idx = ci
    check(p, H, p.tasks, 16, 6, zero_output=False, rng=rng)


def test_planted_mistakes_fail():
    """Each plausible mistake in the run rule or the phase writes breaks
    the comparison: no +1 for a run that starts inside a row begun
    earlier, the chain's last or first offset dropped, the partial rows
    read from the band-sorted copy at the caller's offsets, a later phase
    storing instead of adding.  (A copy left unsorted is no mistake of the
    result: the bounds still split each row into P ranges that cover it
    once; test_band_sort_meaning pins the sort.)"""
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
        out = []
        for t0 in range(0, len(tasks), M):
            a, z = tasks[t0], tasks[min(t0 + M, len(tasks)) - 1]
            out.append((int(a[0]), int(z[1]), int(a[2]) if t0 == 0 else 0,
                        int(tasks[-1][3]) if z[1] == tasks[-1][1] else 0, False))
        return out

    def no_tail(tasks, M):
        return [x if x[4] or x[3] == 0 else x[:3] + (0, False) for x in run_pieces(tasks, M)]

    def no_head(tasks, M):
        return [x if x[4] or x[2] == 0 else (x[0], x[1], 0, x[3], False)
                for x in run_pieces(tasks, M)]

    def partial_from_copy(tasks, M):
        return [x[:4] + (True,) for x in run_pieces(tasks, M)]

    assert differs(sub, pieces_of=no_plus_one)
    assert differs(sub, pieces_of=no_tail)
    assert differs(sub, pieces_of=no_head)
    assert differs(sub, pieces_of=partial_from_copy)
    assert differs(sub, later_phase_adds=False)
    assert not differs(sub, copy=(p.col_idx, p.val))


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
