"""Host emulation of how the aggregation kernel executes a task list.

The kernel (cwlb-spmm_amd/csrc/spmm_mean.hip) runs runs of M consecutive
tasks per wave.  Inside a run it executes *segments*: maximal stretches of
consecutive tasks in which each task continues exactly where the previous
one ended (checked 64 tasks at a time).  A segment is executed as one task:
rows it covers whole are stored, rows it leaves open are added atomically.
The clearing pass (zero_split_rows) zeroes every row that some segment
leaves open, deciding per task with a look-ahead that stops at the end of
its 64-lane wave.

This file restates both rules in Python, exactly as the kernels state them,
and checks that the result equals the reference's task-at-a-time semantics
(reference src/parallelMatrix.cpp:148-236, restated in the oracle) for the
partition's task lists and for lists that are shuffled, reversed or have
gaps, at many run lengths M.  Any order of the segments gives the same
result when no two tasks share a nonzero, so the emulation also runs the
segments in a random order.
"""
import numpy as np
import pytest

import oracle
from conftest import SKEWED_COSTS, UNIT_COSTS
from cwlb_amd import synth, workloads


def well_formed(t, n_rows):
    rs, re, fo, ln = (int(x) for x in t)
    return (0 <= rs < re <= n_rows and fo >= 0 and ln >= 0
            and (re - rs > 1 or ln == 0 or fo < ln))


def continues(a, b):
    if a[3] == 0:
        return b[0] == a[1] and b[2] == 0
    return b[0] == a[1] - 1 and b[2] == a[3]


def segment_break(prev, cur, in_run, n_rows):
    """spmm_mean.hip segment_break."""
    return (in_run % 64 == 0 or not well_formed(prev, n_rows) or not well_formed(cur, n_rows)
            or not continues(prev, cur))


def row_chunk(rp, r, t, nnz):
    """spmm_mean.hip row_chunk: (base, b, e, d); d = -1 for malformed offsets."""
    rs, re, fo, ln = (int(x) for x in t)
    p0, p1 = int(rp[r]), int(rp[r + 1])
    if p0 < 0 or p1 < p0 or p1 > nnz:
        return p0, 0, 0, -1
    d = p1 - p0
    if d == 0:
        return p0, 0, 0, 0
    b = fo if r == rs else 0
    e = ln if (r == re - 1 and ln > 0) else d
    b = min(max(b, 0), d)
    e = min(max(e, b), d)
    return p0, b, e, d


def segments(tasks, M, n_rows):
    """The (first, last) task index of every segment, as the aggregation
    kernel forms them: per run of M tasks, per 64-task window."""
    out = []
    T = len(tasks)
    for t0 in range(0, T, M):
        cnt = min(M, T - t0)
        for w in range(0, cnt, 64):
            wn = min(64, cnt - w)
            starts = [0] + [i for i in range(1, wn)
                            if segment_break(tasks[t0 + w + i - 1], tasks[t0 + w + i], w + i,
                                             n_rows)]
            ends = starts[1:] + [wn]
            out += [(t0 + w + s, t0 + w + e - 1) for s, e in zip(starts, ends)]
    return out


def cleared_rows(rp, origin, tasks, M, n_rows, nnz):
    """Original ids of the C rows zero_split_rows clears."""
    T = len(tasks)
    rows = set()
    for base in range(0, T, 64):  # one 64-lane wave
        lanes = range(base, min(base + 64, T))
        brk, ends, o = [True] * 64, [False] * 64, [-1] * 64
        for t in lanes:
            i = t - base
            cur = tasks[t]
            prev = tasks[t - 1] if t > 0 else cur
            brk[i] = segment_break(prev, cur, t % M, n_rows)
            rs, re, fo, ln = (int(x) for x in cur)
            r = -1
            if well_formed(cur, n_rows):
                ends[i] = re - rs > 1 or ln == 0
                if ln > 0 and (re - rs > 1 or fo == 0):
                    r = re - 1
            elif max(rs, 0) < min(re, n_rows):
                r = min(re, n_rows) - 1
            if r >= 0:
                _, b, e, d = row_chunk(rp, r, cur, nnz)
                if d > 0 and b == 0 and 0 < e < d:
                    o[i] = origin[r]
        for i in range(64):
            if o[i] >= 0 and i < 63:
                ahead = [u for u in range(i + 1, 64) if brk[u] or ends[u]]
                if ahead and not brk[ahead[0]]:
                    o[i] = -1  # completed inside the segment
        rows.update(int(x) for x in o if 0 <= x < n_rows)
    return rows


def emulate(rp, ci, val, origin, H, tasks, M, C0, rng):
    """C after the clearing pass and the aggregation kernel (float64)."""
    n_rows, nnz = len(rp) - 1, len(ci)
    C = C0.astype(np.float64)
    for o in cleared_rows(rp, origin, tasks, M, n_rows, nnz):
        C[o] = 0.0
    segs = segments(tasks, M, n_rows)
    for k in rng.permutation(len(segs)):
        first, last = segs[k]
        seg = (tasks[first][0], tasks[last][1], tasks[first][2], tasks[last][3])
        for r in range(max(int(seg[0]), 0), min(int(seg[1]), n_rows)):
            base, b, e, d = row_chunk(rp, r, seg, nnz)
            o = origin[r]
            if d < 0:
                continue
            if d == 0:
                C[o] = 0.0
                continue
            if e <= b:
                continue
            cols = ci[base + b:base + e]
            acc = (val[base + b:base + e, None].astype(np.float64) * H[cols]).sum(0) / d
            if b == 0 and e == d:
                C[o] = acc
            else:
                C[o] += acc
    return C


def check_list(p, H, tasks, M, zero_output, rng):
    n = p.n
    ref = oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H, tasks)
    C0 = np.zeros((n, H.shape[1])) if zero_output else np.full((n, H.shape[1]), np.nan)
    # Without a cleared C every row starts as NaN: each one must be defined
    # by the clearing pass or a store.
    got = emulate(p.row_ptr, p.col_idx, p.val, p.origin, H.astype(np.float64), tasks, M, C0, rng)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-6)


def small_problem(cfg, S, seed, costs=SKEWED_COSTS):
    g = workloads.small(cfg, seed=seed)
    p = workloads.prepare(g, costs, S)
    H = synth.features(g.n, 4, seed)
    return p, H


@pytest.mark.parametrize("M", [1, 2, 3, 7, 64, 65, 130])
@pytest.mark.parametrize("cfg,S", [(4, 3), (4, 16), (2, 5), (5, 4)])
def test_partition_lists_tile(cfg, S, M):
    """The partition's lists: every run (64-task window) is one segment,
    and the clearing pass plus segment execution equal the reference."""
    p, H = small_problem(cfg, S, 3)
    segs = segments(p.tasks, M, p.n)
    windows = sum((min(M, len(p.tasks) - t0) + 63) // 64 for t0 in range(0, len(p.tasks), M))
    assert len(segs) == windows
    check_list(p, H, p.tasks, M, zero_output=False, rng=np.random.default_rng(M))


@pytest.mark.parametrize("M", [2, 5, 64, 100])
@pytest.mark.parametrize("how", ["shuffled", "reversed", "swapped_pairs", "gaps"])
def test_lists_that_do_not_tile(how, M):
    """Shuffled, reversed and gapped lists break into segments that stay
    consistent with the clearing pass: with C cleared first (the
    reference's zeroed C) the result equals the reference's."""
    rng = np.random.default_rng(len(how) * 100 + M)
    p, H = small_problem(4, 3, 5)
    t = p.tasks.copy()
    if how == "shuffled":
        t = t[rng.permutation(len(t))]
    elif how == "reversed":
        t = t[::-1].copy()
    elif how == "swapped_pairs":
        idx = np.arange(len(t))
        sw = rng.choice(len(t) // 2, len(t) // 8, replace=False) * 2
        idx[sw], idx[sw + 1] = sw + 1, sw
        t = t[idx]
    else:
        t = t[rng.random(len(t)) > 0.2]
    check_list(p, H, t, M, zero_output=True, rng=rng)
    if how != "gaps":
        # Every row's first nonzero is in some task: the clearing pass alone
        # defines every row.
        check_list(p, H, t, M, zero_output=False, rng=rng)


def test_per_row_tasks_shuffled_many():
    """One task per row, shuffled, at run lengths that merge many of them."""
    rng = np.random.default_rng(9)
    g = workloads.small(2, seed=6)
    p = workloads.prepare(g, UNIT_COSTS, 4)
    per_row = np.stack([np.arange(g.n), np.arange(1, g.n + 1), np.zeros(g.n), np.zeros(g.n)],
                       1).astype(np.int32)
    H = synth.features(g.n, 3, 1)
    for M in (12, 64):
        t = per_row[rng.permutation(g.n)]
        segs = segments(t, M, g.n)
        assert len(segs) > 0.9 * len(t)  # almost no neighbours stay adjacent
        check_list(p, H, t, M, zero_output=False, rng=rng)


def test_malformed_tasks_are_single_segments():
    """Tasks with inverted, empty or out-of-range bounds never merge with a
    neighbour."""
    n = 10
    good = np.array([[0, 2, 0, 0], [2, 4, 0, 0]], np.int32)
    for bad in ([4, 4, 0, 0], [4, 3, 0, 0], [-1, 5, 0, 0], [4, 11, 0, 0], [4, 5, 3, 2],
                [4, 5, -1, 0], [4, 5, 0, -2]):
        t = np.concatenate([good, np.array([bad], np.int32), [[5, 6, 0, 0]]]).astype(np.int32)
        segs = segments(t, 64, n)
        assert (2, 2) in segs and (3, 3) in segs, (bad, segs)
    assert segments(good, 64, n) == [(0, 1)]


def test_window_boundary_breaks_and_clears():
    """A row split across the 64-task window boundary inside a long run is
    left open by both windows and cleared; the result still matches."""
    n = 1
    deg = 200
    rp = np.array([0, deg], np.int32)
    ci = np.zeros(deg, np.int32)
    val = np.ones(deg, np.float32)
    tasks = np.array([[0, 1, 2 * i, 2 * i + 2 if i < 99 else 0] for i in range(100)], np.int32)
    origin = np.zeros(1, np.int32)
    H = np.ones((1, 2))
    p = workloads.Prepared(n, deg, origin, rp, ci, val, tasks, 2, 0.0)
    assert segments(tasks, 100, n) == [(0, 63), (64, 99)]
    assert cleared_rows(rp, origin, tasks, 100, n, deg) == {0}
    check_list(p, H, tasks, 100, zero_output=False, rng=np.random.default_rng(0))
    # A run that fits one window completes the row: nothing is cleared.
    t50 = tasks[:50].copy()
    t50[-1, 3] = 0
    t50[-1] = [0, 1, 98, 0]
    t50[:, 3] = np.where(np.arange(50) < 49, t50[:, 3], 0)
    rp50 = np.array([0, 100], np.int32)
    assert segments(t50, 64, n) == [(0, 49)]
    assert cleared_rows(rp50, origin, t50, 64, n, 100) == set()


def test_emulation_catches_planted_mistakes(monkeypatch):
    """The harness fails when the clearing pass forgets the look-ahead's
    segment starts, or when runs are merged without the tiling check."""
    rng = np.random.default_rng(4)
    p, H = small_problem(4, 3, 5)
    p.tasks = p.tasks[-400:]  # the highest-degree rows, split by S = 3
    shuffled = p.tasks[rng.permutation(len(p.tasks))]
    ref = oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H, shuffled)
    zeros = np.zeros((p.n, H.shape[1]))

    def differs(tasks, M, reference):
        got = emulate(p.row_ptr, p.col_idx, p.val, p.origin, H.astype(np.float64), tasks, M,
                      zeros, rng)
        return not np.allclose(got, reference, rtol=1e-5, atol=1e-6)

    assert not differs(shuffled, 8, ref)
    # Runs merged as whole tasks (no tiling check): the old behaviour.
    monkeypatch.setattr(__import__(__name__), "segment_break",
                        lambda prev, cur, in_run, n_rows: in_run % 64 == 0)
    assert differs(shuffled, 8, ref)
    monkeypatch.undo()
    # A look-ahead that treats every continuation as completing the row.
    real_ballot = cleared_rows

    def no_clear(rp, origin, tasks, M, n_rows, nnz):
        return set()
    monkeypatch.setattr(__import__(__name__), "cleared_rows", no_clear)
    ref_tiled = oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H, p.tasks)
    nan0 = np.full((p.n, H.shape[1]), np.nan)
    got = emulate(p.row_ptr, p.col_idx, p.val, p.origin, H.astype(np.float64), p.tasks, 3, nan0,
                  rng)
    assert np.isnan(got).any() and real_ballot is not None
    assert not np.allclose(np.nan_to_num(got), ref_tiled)


def test_one_row_task_past_the_row_end():
    """A one-row task whose end offset passes the row's degree is not
    counted as ending the row by the look-ahead (the clearing pass then
    clears a row that the segment later stores whole): the result is
    still the reference's, with and without a following segment break."""
    rp = np.array([0, 5, 9, 12], np.int32)
    ci = np.array([0, 1, 2, 1, 0, 2, 2, 1, 0, 1, 0, 2], np.int32)
    val = np.linspace(0.5, 2.0, 12).astype(np.float32)
    origin = np.array([2, 0, 1], np.int32)
    H = np.arange(6, dtype=np.float64).reshape(3, 2)
    p = workloads.Prepared(3, 12, origin, rp, ci, val, None, 2, 0.0)
    # (list, whether row 0 -- original id 2 -- is cleared)
    lists = [
        # the next task does not continue at offset 10: a segment break, so
        # the look-ahead clears row 0, which the segment then stores whole
        (np.array([[0, 1, 0, 3], [0, 1, 3, 10], [1, 3, 0, 0]], np.int32), True),
        # the segment goes on into a task with more rows: row 0 complete
        (np.array([[0, 1, 0, 3], [0, 1, 3, 10], [0, 2, 10, 0], [2, 3, 0, 0]], np.int32), False),
    ]
    for t, cleared in lists:
        assert (2 in cleared_rows(rp, origin, t, 64, 3, 12)) == cleared
        p.tasks = t
        check_list(p, H, t, 64, zero_output=False, rng=np.random.default_rng(1))
