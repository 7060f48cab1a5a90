"""The product library's host side (no GPU needed): exports, partition,
reorder, S selection and the cost file, bit-exact against the oracle and the
reference extract; and the error behaviour of the C ABI."""
import os
import re

import numpy as np
import pytest

import oracle
from conftest import SKEWED_COSTS, UNIT_COSTS
from cwlb_amd import capi, paths, synth, workloads



def header_functions():
    text = open(os.path.join(paths.INCLUDE_DIR, "cwlb.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cwlb_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_function():
    import ctypes
    lib = ctypes.CDLL(capi.lib_path())
    declared = header_functions()
    assert declared, "no declarations found"
    missing = [f for f in declared if not hasattr(lib, f)]
    assert not missing, missing
    assert sorted(capi.EXPORTS) == declared


def test_flag_constants_match_header():
    text = open(os.path.join(paths.INCLUDE_DIR, "cwlb.h")).read()
    for name, value in [("ZERO_OUTPUT", capi.ZERO_OUTPUT), ("PER_TASK", capi.PER_TASK),
                        ("KEEP_EMPTY_ROWS", capi.KEEP_EMPTY_ROWS)]:
        m = re.search(rf"#define CWLB_SPMM_{name} (0x[0-9a-fA-F]+)u", text)
        assert m and int(m.group(1), 16) == value, name


def test_library_is_gfx950_only():
    """The shared object carries gfx950 code objects only."""
    data = open(capi.lib_path(), "rb").read()
    archs = set(re.findall(rb"amdgcn-amd-amdhsa--(gfx[0-9a-f]+)", data))
    assert archs == {b"gfx950"}, archs


def test_version():
    assert capi.version().startswith("0.")


@pytest.mark.parametrize("cfg", [1, 2, 3, 4, 5])
def test_partition_bit_exact(cfg):
    g = workloads.small(cfg)
    _, rp, _, _ = capi.reorder_by_degree(g.row_ptr, g.col_idx, g.val)
    for costs in (UNIT_COSTS, SKEWED_COSTS, (0.0171, 0.4126, 0.0532, 2.2409)):
        for S in workloads.candidate_s(g.nnz, 256) + [1, 2, 5, 100]:
            cap = capi.capacity_from_s(S, costs)
            assert cap == oracle.capacity_from_s(S, costs)
            got = capi.partition(rp, costs, cap)
            assert np.array_equal(got, oracle.partition(rp, costs, cap))
            if oracle.ref() is not None:
                assert np.array_equal(got, oracle.ref_partition(rp, costs, cap))


def test_partition_random_bit_exact(rng):
    for _ in range(3000):
        n = int(rng.integers(0, 60))
        degs = rng.integers(0, int(rng.integers(1, 90)), n)
        if rng.random() < 0.7:
            degs = np.sort(degs)
        rp = np.concatenate([[0], np.cumsum(degs)]).astype(np.int32)
        costs = tuple(float(rng.choice([0.0, 0.01, 0.125, 0.5, 1.0, 2.5, 7.0])) for _ in range(4))
        cap = float(rng.random() * 40) if rng.random() < 0.3 else capi.capacity_from_s(
            int(rng.integers(1, 30)), costs)
        want = oracle.ref_partition(rp, costs, cap) if oracle.ref() is not None else oracle.partition(
            rp, costs, cap)
        assert np.array_equal(capi.partition(rp, costs, cap), want)


def test_partition_special_values():
    rp = np.array([0, 3, 10, 10, 40], np.int32)
    for costs, cap in [((0.0, 0.0, 0.0, 0.0), 0.0), ((1.0, 1.0, 1.0, 1.0), float("inf")),
                       ((1.0, 1.0, 1.0, 1.0), float("nan")), ((0.5, 0.5, 1.0, 1.0), -3.0),
                       ((1e-40, 0.0, 1.0, 1.0), 5.0), ((1.0, 1.0, 1.0, 1.0), 1e300)]:
        got = capi.partition(rp, costs, cap)
        assert np.array_equal(got, oracle.partition(rp, costs, cap))
        if oracle.ref() is not None:
            assert np.array_equal(got, oracle.ref_partition(rp, costs, cap))


def test_partition_leaves_out_empty_rows_above_capacity():
    """A row without nonzeros whose slot cost Cs exceeds the capacity gets no
    task (utils.cpp:972-976: nothing of it remains to split); with Cs within
    the capacity it is packed like any row.  Degrees 0, 0, 3, 0, 5 at S = 2
    (capacity 0.5 + 1 * 2 = 2.5), derived by hand from the packing rules."""
    rp = np.array([0, 0, 0, 3, 3, 8], np.int32)
    cases = [((0.5, 0.5, 4.0, 0.5),   # Cs = 4 > 2.5: rows 0, 1, 3 left out
              [[2, 3, 0, 2], [2, 3, 2, 0], [4, 5, 0, 2], [4, 5, 2, 4], [4, 5, 4, 0]]),
             ((0.5, 0.5, 1.0, 0.5),   # Cs = 1: rows 0 and 1 packed, row 3 leads row 4
              [[0, 2, 0, 0], [2, 3, 0, 2], [2, 3, 2, 0], [3, 5, 0, 1], [4, 5, 1, 3],
               [4, 5, 3, 0]])]
    for costs, want in cases:
        cap = capi.capacity_from_s(2, costs)
        assert cap == 2.5
        got = capi.partition(rp, costs, cap)
        assert got.tolist() == want
        assert np.array_equal(got, oracle.partition(rp, costs, cap))
        if oracle.ref() is not None:
            assert np.array_equal(got, oracle.ref_partition(rp, costs, cap))


def test_partition_empty_and_buffer_sizing():
    assert len(capi.partition(np.zeros(1, np.int32), UNIT_COSTS, 4.5)) == 0
    import ctypes as C
    rp = np.array([0, 10], np.int32)
    cnt = C.c_int64()
    st = capi.lib().cwlb_partition(rp.ctypes.data, 1, C.byref(capi.costs(UNIT_COSTS)), 4.5, None,
                                   0, C.byref(cnt))
    assert st == capi.INSUFFICIENT and cnt.value == 3


@pytest.mark.parametrize("cfg", [1, 2, 4, 5])
def test_reorder_bit_exact(cfg):
    g = workloads.small(cfg)
    a = capi.reorder_by_degree(g.row_ptr, g.col_idx, g.val)
    b = oracle.reorder_by_degree(g.row_ptr, g.col_idx, g.val)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)


def test_reorder_threads_bit_exact(rng):
    """A graph large enough for the threaded reordering (several row chunks,
    chunks of the copies cut by nonzeros) with empty rows, runs of equal
    degrees across chunk boundaries and rows at and above the 65,536-degree
    histogram limit: identical to the oracle and to a stable argsort."""
    n = 600_000
    deg = rng.choice([0, 0, 1, 2, 3, 5, 8, 40], n).astype(np.int64)
    deg[rng.integers(0, n, 6)] = [65535, 65536, 65537, 100000, 65536, 70000]
    rp = np.concatenate([[0], np.cumsum(deg)]).astype(np.int32)
    ci = rng.integers(0, n, rp[-1]).astype(np.int32)
    val = rng.standard_normal(rp[-1]).astype(np.float32)
    a = capi.reorder_by_degree(rp, ci, val)
    b = oracle.reorder_by_degree(rp, ci, val)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)
    assert np.array_equal(a[0], np.argsort(deg, kind="stable"))


def test_reorder_rejects_bad_csr():
    with pytest.raises(capi.CwlbError) as e:
        capi.reorder_by_degree(np.array([0, 5, 3], np.int32), np.zeros(5, np.int32),
                               np.ones(5, np.float32))
    assert e.value.status == capi.INVALID_ARG


def test_s_selection_matches_oracle(rng):
    for _ in range(2000):
        nnz = int(rng.integers(0, 2**40))
        assert capi.recommended_candidate_w(nnz) == oracle.recommended_candidate_w(nnz)
        cu, w = int(rng.integers(1, 300)), int(rng.integers(1, 9000))
        assert capi.wave_based_s(nnz, 2, cu, w) == oracle.wave_based_s(nnz, 2, cu, w)
        s = int(rng.integers(-3, 300))
        costs = tuple(float(rng.choice([0.0, 0.5, 1.5, -1.0, 3.25])) for _ in range(4))
        assert capi.capacity_from_s(s, costs) == oracle.capacity_from_s(s, costs)
        v = np.sort(rng.integers(1, 60, 3))
        best = int(rng.integers(0, 3))
        assert capi.candidate_search_bounds(v, best) == oracle.candidate_search_bounds(v, best)
        lo, hi = capi.candidate_search_bounds(v, best)
        c = int(rng.integers(1, 12))
        assert capi.candidate_search_by_count(lo, hi, c) == oracle.candidate_search_by_count(lo, hi, c)
        assert capi.candidate_search_by_step(lo, hi, c) == oracle.candidate_search_by_step(lo, hi, c)
    assert capi.wave_based_s(10, 0, 256, 64) == 1
    for bad in ((10, 2, 0, 64), (10, 2, 256, 0), (10, 2, -1, 5)):
        with pytest.raises(capi.CwlbError) as e:
            capi.wave_based_s(*bad)
        assert e.value.status == capi.INVALID_ARG
    for bad in (([0, 1, 2], 0), ([3, 2, 4], 1), ([1, 2, 3], 3)):
        with pytest.raises(capi.CwlbError):
            capi.candidate_search_bounds(*bad)
    with pytest.raises(capi.CwlbError):
        capi.candidate_search_by_step(1, 20001, 2)
    with pytest.raises(capi.CwlbError):
        capi.candidate_search_by_count(1, 20001, 10001)


def test_cost_file_roundtrip_and_format(tmp_path):
    c4 = (0.0123456789, 12.3456789, 1e-9, 123456.7)
    p = tmp_path / "sub" / "dir" / "spmm_costs.txt"
    capi.save_costs(c4, p)
    text = p.read_text()
    assert text == oracle.format_costs(c4, 6)
    if oracle.ref() is not None:
        assert text == oracle.ref_format_costs(c4, 6)
    assert capi.read_costs(p) == tuple(float(f"{x:.6f}") for x in c4)
    capi.save_costs(c4, p, append=True, precision=2)
    assert p.read_text() == text + oracle.format_costs(c4, 2)


def test_cost_file_errors(tmp_path):
    f = tmp_path / "afile"
    f.write_text("x")
    with pytest.raises(capi.CwlbError) as e:
        capi.save_costs(UNIT_COSTS, f / "costs.txt")
    assert e.value.status == capi.IO_ERROR
    with pytest.raises(capi.CwlbError) as e:
        capi.read_costs(tmp_path / "missing.txt")
    assert e.value.status == capi.IO_ERROR
    bad = tmp_path / "bad.txt"
    bad.write_text("1.0\n2.0\nthree\n4.0\n")
    with pytest.raises(capi.CwlbError) as e:
        capi.read_costs(bad)
    assert e.value.status == capi.IO_ERROR
    with pytest.raises(capi.CwlbError):
        capi.save_costs(UNIT_COSTS, "")


def test_committed_gfx950_cost_file_parses():
    path = os.path.join(paths.PKG_DIR, "resources", "spmm_costs_gfx950.txt")
    if not os.path.exists(path):
        pytest.skip("calibrated gfx950 cost file not committed yet")
    c = capi.read_costs(path)
    assert all(np.isfinite(x) and x > 0 for x in c)


def test_context_without_gpu_fails_cleanly():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    with pytest.raises(capi.CwlbError) as e:
        capi.Context(0)
    assert e.value.status in (capi.HIP_ERROR, capi.INVALID_ARG)


def cxx_header_functions():
    """Free functions and members declared in the C++17 drop-in headers."""
    names = set()
    for h in ("Matrix.h", "utils.h", "parallelMatrix.h", "data.h", "cwlb_device.h",
              "cwlb_driver.h"):
        text = open(os.path.join(paths.INCLUDE_DIR, h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        for m in re.finditer(r"(?m)^\s*(?:[\w:<>,*&]+\s+)+?[*&]?(\w+)\s*\(", text):
            name = m.group(1)
            # declarations only: a body in the header is inline, not exported
            depth, i = 1, m.end()
            while depth and i < len(text):
                depth += {"(": 1, ")": -1}.get(text[i], 0)
                i += 1
            after = text[i:].lstrip()
            if after.startswith("const"):
                after = after[5:].lstrip()
            if not after.startswith(";"):
                continue
            if name not in ("if", "return", "check", "operator", "explicit", "inline"):
                names.add(name)
    return sorted(names)


def test_library_exports_the_cxx_layer():
    """Every function the drop-in headers declare is defined in libcwlb.so."""
    import subprocess
    out = subprocess.run(["nm", "-DC", "--defined-only", capi.lib_path()], capture_output=True,
                         text=True, check=True).stdout
    declared = cxx_header_functions()
    for must in ("spmmKernel", "spmmKernelLargeKFallback", "costWeightedTaskPartitioning",
                 "costWeightedTaskPartitioning_HIP", "loadDatasetToCSR", "sortCSRByDegreeDPLCPU",
                 "sortCSRByDegree_HIP", "measure_spmm_costs", "run_single_s",
                 "validate_custom_csr_result", "wave_based_s", "capacity_from_s"):
        assert must in declared, must
    missing = [f for f in declared if not re.search(r"(?:^|[ :])" + f + r"\(", out, re.M)]
    assert not missing, missing
    assert re.search(r" CSR::CSR\(", out) and re.search(r" cwlb::Device::Device\(", out)
