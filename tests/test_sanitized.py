"""Differential fuzzing of the host code under AddressSanitizer and
UndefinedBehaviorSanitizer (tests/cxx/bin/dropin_probe_san: the partition,
reordering, S selection, cost file, loader and validator sources compiled
with -fsanitize=address,undefined).

Every generated input must either give the oracle's answer (the reference's
own partition too, where oracle/_ref builds) or end in one of the
reference's exceptions; any sanitizer report fails the test.
"""
import os
import subprocess

import numpy as np
import pytest
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

import oracle
from dropin_util import ProbeError, write_csr, write_order

HERE = os.path.dirname(os.path.abspath(__file__))
SAN = os.path.join(HERE, "cxx", "bin", "dropin_probe_san")
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0:exitcode=86",
           UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1:exitcode=87")
SETTINGS = settings(max_examples=60, deadline=None,
                    suppress_health_check=[HealthCheck.function_scoped_fixture,
                                           HealthCheck.too_slow])


def san(*args, cwd=None):
    if not os.path.exists(SAN):
        pytest.fail(f"{SAN} missing: build with __graft_entry__.build()")
    r = subprocess.run([SAN, *map(str, args)], capture_output=True, text=True, cwd=cwd, env=ENV,
                       timeout=120)
    assert "Sanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr[-3000:]
    assert r.returncode in (0, 3), (r.returncode, r.stderr[-3000:])
    if r.returncode == 3:
        line = [ln for ln in r.stdout.splitlines() if "EXC " in ln][-1]
        _, kind, msg = line[line.index("EXC "):].split(" ", 2)
        raise ProbeError(kind, msg)
    return r.stdout


degrees = st.lists(st.integers(0, 60), min_size=0, max_size=120)
cost_value = st.one_of(st.sampled_from([0.0, 0.25, 0.5, 1.0, 1e-9, 3.5, -0.5]),
                       st.floats(0.001, 8.0, allow_nan=False))


@SETTINGS
@given(degs=degrees, costs=st.tuples(cost_value, cost_value, cost_value, cost_value),
       S=st.integers(1, 70))
def test_partition_fuzz(tmp_path, degs, costs, S):
    rp = np.concatenate([[0], np.cumsum(degs)]).astype(np.int32)
    n = len(degs)
    write_order(tmp_path / "ord", np.arange(n), rp, np.zeros(rp[-1]), np.ones(rp[-1]))
    san("partition", tmp_path / "ord", *costs, S, tmp_path / "t")
    raw = open(tmp_path / "t", "rb").read()
    cap = float(np.frombuffer(raw[:8], np.float64)[0])
    got = np.frombuffer(raw[8:], np.int32).reshape(-1, 4)
    assert cap == oracle.capacity_from_s(S, costs)
    assert np.array_equal(got, oracle.partition(rp, costs, cap))
    if oracle.ref() is not None:
        assert np.array_equal(got, oracle.ref_partition(rp, costs, cap))
    # the GPU partition's decomposition, for the costs it takes
    try:
        san("partition-emul", tmp_path / "ord", *costs, S, tmp_path / "e")
    except ProbeError as e:
        assert e.kind == "invalid_argument" and "unsupported costs" in e.msg
    else:
        emul = np.frombuffer(open(tmp_path / "e", "rb").read()[8:], np.int32).reshape(-1, 4)
        assert np.array_equal(emul, got)


@SETTINGS
@given(degs=degrees, data=st.data())
def test_reorder_fuzz(tmp_path, degs, data):
    rp = np.concatenate([[0], np.cumsum(degs)]).astype(np.int32)
    nnz = int(rp[-1])
    ci = np.array(data.draw(st.lists(st.integers(0, 1000), min_size=nnz, max_size=nnz)), np.int32)
    val = np.arange(nnz, dtype=np.float32)
    corrupt = data.draw(st.sampled_from([None, "decrease", "overflow"]))
    if corrupt == "decrease" and len(rp) > 2:
        rp[1] = rp[2] + 1
    elif corrupt == "overflow" and len(rp) > 1:
        rp[-1] += 3
    write_csr(tmp_path / "in", rp, ci, val)
    try:
        san("reorder-cpu", tmp_path / "in", tmp_path / "out")
    except ProbeError as e:
        assert corrupt is not None and e.kind == "runtime_error"
        return
    assert corrupt is None or len(rp) <= 2
    from dropin_util import read_order
    got = read_order(tmp_path / "out")
    if len(rp) < 2:  # fewer than two offsets: an empty CSR_Order (main.cpp:199-201)
        assert all(len(a) == 0 for a in got)
        return
    exp = oracle.reorder_by_degree(rp, ci, val)
    for a, b in zip(got, exp):
        assert np.array_equal(a, b)


csr_text = st.text(alphabet="0123456789,-\n\r x", max_size=60)


@SETTINGS
@given(text=csr_text)
def test_loader_fuzz(tmp_path, text):
    build = tmp_path / "build"
    data = tmp_path / "resources" / "datasets"
    build.mkdir(exist_ok=True)
    data.mkdir(parents=True, exist_ok=True)
    (data / "g.csr").write_text(text)
    try:
        out = san("load", build, "g")
    except ProbeError as e:
        assert e.kind in ("runtime_error", "invalid_argument", "out_of_range"), e
        return
    lines = out.splitlines()
    V, E = int(lines[0].split()[1]), int(lines[0].split()[3])
    rp = [int(x) for x in lines[1].split()[1:]]
    ci = [int(x) for x in lines[2].split()[1:]]
    assert V == len(rp) - 1 and E == rp[-1] == len(ci) and rp[0] == 0
    assert all(a <= b for a, b in zip(rp, rp[1:])) and all(c >= 0 for c in ci)


@SETTINGS
@given(rows=st.integers(0, 6), cols=st.integers(0, 5), drows=st.integers(0, 4),
       tol=st.sampled_from([0.0, 1e-4, 0.5, -1.0]), data=st.data())
def test_validator_fuzz(tmp_path, rows, cols, drows, tol, data):
    vals = st.sampled_from([0.0, 1.0, -1.0, 0.5, np.nan, np.inf, -np.inf])
    A = np.array(data.draw(st.lists(vals, min_size=rows * cols, max_size=rows * cols)),
                 np.float32).reshape(rows, cols)
    B = np.array(data.draw(st.lists(vals, min_size=rows * cols, max_size=rows * cols)),
                 np.float32).reshape(rows, cols)
    np.ascontiguousarray(A).tofile(tmp_path / "A")
    np.ascontiguousarray(B).tofile(tmp_path / "B")
    np.ones((drows, cols), np.float32).tofile(tmp_path / "D")
    write_csr(tmp_path / "csr", np.arange(rows + 1), np.zeros(rows), np.ones(rows))
    out = san("validate", tmp_path / "A", tmp_path / "B", tmp_path / "csr", tmp_path / "D",
              rows, cols, drows, tol)
    passed = out.strip().splitlines()[-1] == "RESULT pass"
    if tol < 0 or drows <= 0:
        assert not passed
        return
    with np.errstate(invalid="ignore"):
        diff = np.abs(A.astype(np.float64) - B.astype(np.float64))
    ok = np.where(np.isnan(A) | np.isnan(B), np.isnan(A) & np.isnan(B),
                  np.where(np.isinf(A) | np.isinf(B), A == B, diff <= np.float32(tol)))
    assert passed == bool(ok.all())


@SETTINGS
@given(lo=st.integers(-3, 40), hi=st.integers(-3, 60), third=st.integers(-2, 30),
       mode=st.sampled_from(["count", "step"]))
def test_search_grid_fuzz(lo, hi, third, mode):
    try:
        got = [int(x) for x in san("search", lo, hi, mode, third).split()[1:]]
    except ProbeError as e:
        assert e.kind == "invalid_argument"
        with pytest.raises(ValueError):
            (oracle.candidate_search_by_count if mode == "count"
             else oracle.candidate_search_by_step)(lo, hi, third)
        return
    fn = oracle.candidate_search_by_count if mode == "count" else oracle.candidate_search_by_step
    assert got == fn(lo, hi, third)


# ---------------------------------------------------------------- ThreadSanitizer
TSAN = os.path.join(HERE, "cxx", "bin", "dropin_probe_tsan")
TSAN_ENV = dict(os.environ, TSAN_OPTIONS="halt_on_error=1:exitcode=66:report_signal_unsafe=0")


def tsan(*args):
    if not os.path.exists(TSAN):
        pytest.fail(f"{TSAN} missing: build with __graft_entry__.build()")
    r = subprocess.run([TSAN, *map(str, args)], capture_output=True, text=True, env=TSAN_ENV,
                       timeout=600)
    assert "ThreadSanitizer" not in r.stderr, r.stderr[-4000:]
    assert r.returncode == 0, (r.returncode, r.stderr[-3000:])
    return r.stdout


@pytest.mark.parametrize("shape", ["rmat", "hub"])
def test_threaded_reorder_under_tsan(tmp_path, shape):
    """The host degree reordering (sortCSRByDegreeDPLCPU over
    cwlb_reorder_by_degree: up to 16 threads over shared per-thread degree
    histograms and row offsets) and the partition of its output, under
    ThreadSanitizer, on a skewed R-MAT graph of 2^18 rows and about 4M
    nonzeros (enough rows and nonzeros for every thread the host offers, up
    to 16) and on one with a single hub row of 1M nonzeros: no race
    reported, and the results are the oracle's."""
    from cwlb_amd import synth
    if shape == "rmat":
        g = synth.rmat(18, 1 << 22, 0.57, 0.19, 0.19, 18)
        rp, ci = g.row_ptr, g.col_idx
    else:
        n = 300_000
        deg = np.ones(n, np.int64)
        deg[12_345] = 1_000_000
        rp = np.concatenate([[0], np.cumsum(deg)]).astype(np.int32)
        ci = np.random.default_rng(5).integers(0, n, rp[-1]).astype(np.int32)
    val = (np.arange(len(ci)) % 7 + 1).astype(np.float32)
    write_csr(tmp_path / "in", rp, ci, val)
    tsan("reorder-cpu", tmp_path / "in", tmp_path / "out")
    from dropin_util import read_order
    got = read_order(tmp_path / "out")
    exp = oracle.reorder_by_degree(rp, ci, val)
    for a, b in zip(got, exp):
        assert np.array_equal(a, b)
    costs = (0.125, 1.375, 0.75, 3.5)
    tsan("partition", tmp_path / "out", *costs, 40, tmp_path / "t")
    raw = open(tmp_path / "t", "rb").read()
    cap = float(np.frombuffer(raw[:8], np.float64)[0])
    tasks = np.frombuffer(raw[8:], np.int32).reshape(-1, 4)
    assert np.array_equal(tasks, oracle.partition(exp[1], costs, cap))


def test_host_pointer_threads_under_tsan():
    """The host-pointer entry's threaded loops (csrc/host_threads.h: the
    staged copies in ~8 MiB parts on up to 8 threads, the row-offset and
    column-index checks with their shared flag) under ThreadSanitizer, on
    buffers large enough for every thread, with bad entries in one part and
    in every part (all threads raising the flag at once): no race reported
    and every answer right.  (The entry itself needs a GPU.)"""
    path = os.path.join(HERE, "cxx", "bin", "threads_probe_tsan")
    if not os.path.exists(path):
        pytest.fail(f"{path} missing: build with __graft_entry__.build()")
    r = subprocess.run([path], capture_output=True, text=True, env=TSAN_ENV, timeout=600)
    assert "ThreadSanitizer" not in r.stderr, r.stderr[-4000:]
    assert r.returncode == 0 and r.stdout.strip() == "OK", (r.returncode, r.stdout, r.stderr[-2000:])
