"""Partition and reordering parity against fixtures written by the
reference's own costWeightedTaskPartitioning (utils.cpp:832-1021) and
capacity_from_s (main.cpp:281-292), compiled from the reference sources
(tests/golden/make_partition_golden.py).  These checks need neither the
reference sources nor oracle/_ref: they pin the oracle's partition and the
product's host partition wherever the tests run.

Bar: bit-exact (SHA-256 over the int32 arrays, exact capacity bits).
"""
import hashlib
import json
import os

import numpy as np
import pytest

import oracle
from cwlb_amd import capi, workloads

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                     "partition_golden.json")))


def sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).astype("<i4", copy=False).tobytes()).hexdigest()


def check_graph(g, rec):
    assert (g.n, g.nnz) == (rec["n"], rec["nnz"])
    assert sha(g.row_ptr) == rec["row_ptr_sha256"], "synthetic generator drifted (row_ptr)"
    assert sha(g.col_idx) == rec["col_idx_sha256"], "synthetic generator drifted (col_idx)"


def check_partitions(rp, rec, fns):
    for p in rec["partitions"]:
        costs = GOLDEN["costs"][p["costs"]]
        cap = float.fromhex(p["capacity"])
        assert capi.capacity_from_s(p["S"], costs) == cap
        assert oracle.capacity_from_s(p["S"], costs) == cap
        for name, fn in fns:
            tasks = fn(rp, costs, cap)
            assert len(tasks) == p["n_tasks"], (name, p["costs"], p["S"])
            assert sha(tasks) == p["tasks_sha256"], (name, p["costs"], p["S"])
            if "tasks" in p:
                assert tasks.tolist() == p["tasks"]


@pytest.mark.parametrize("cfg", [1, 2, 3, 4, 5])
def test_small_workloads_match_reference_fixture(cfg):
    rec = GOLDEN["small"][str(cfg)]
    g = workloads.small(cfg)
    check_graph(g, rec)
    origin, rp, _, _ = oracle.reorder_by_degree(g.row_ptr, g.col_idx, g.val)
    assert sha(origin) == rec["origin_sha256"]
    assert sha(rp) == rec["sorted_row_ptr_sha256"]
    h_origin, h_rp, _, _ = capi.reorder_by_degree(g.row_ptr, g.col_idx, g.val)
    assert sha(h_origin) == rec["origin_sha256"] and sha(h_rp) == rec["sorted_row_ptr_sha256"]
    check_partitions(rp, rec, [("oracle", oracle.partition), ("host", capi.partition)])


@pytest.mark.parametrize("cfg", [1, 2, 3, 4, 5])
def test_full_workloads_match_reference_fixture(cfg):
    """Full-size graphs at the three wave-based S (and the mesh's S sweep)
    with the committed gfx950 costs."""
    rec = GOLDEN["full"][str(cfg)]
    g = workloads.graph(cfg)
    check_graph(g, rec)
    origin, rp, _, _ = capi.reorder_by_degree(g.row_ptr, g.col_idx, g.val)
    del g
    assert sha(origin) == rec["origin_sha256"]
    assert sha(rp) == rec["sorted_row_ptr_sha256"]
    check_partitions(rp, rec, [("oracle", oracle.partition), ("host", capi.partition)])


def test_fixture_agrees_with_reference_extract_when_built():
    """Where oracle/_ref is built, the fixture's small cases are re-derived
    from it (guards against a stale fixture)."""
    if oracle.ref() is None:
        pytest.skip("oracle/_ref not built (no reference sources)")
    for cfg in (1, 4):
        rec = GOLDEN["small"][str(cfg)]
        g = workloads.small(cfg)
        _, rp, _, _ = oracle.reorder_by_degree(g.row_ptr, g.col_idx, g.val)
        check_partitions(rp, rec, [("reference", oracle.ref_partition)])


def random_case(c):
    degs = np.array([int(x) for x in c["degrees"].split()], np.int64)
    rp = np.concatenate([[0], np.cumsum(degs)]).astype(np.int32)
    return rp, c["costs"], float.fromhex(c["capacity"])


def test_random_cases_match_reference_fixture():
    """Short sorted and unsorted degree sequences under assorted costs and
    capacities (these meet the current-row prefix absorption often)."""
    assert len(GOLDEN["random"]) >= 100
    for i, c in enumerate(GOLDEN["random"]):
        rp, costs, cap = random_case(c)
        if c["S"] is not None:
            assert oracle.capacity_from_s(c["S"], costs) == cap
            assert capi.capacity_from_s(c["S"], costs) == cap
        for fn in (oracle.partition, capi.partition):
            tasks = fn(rp, costs, cap)
            assert (len(tasks), sha(tasks)) == (c["n_tasks"], c["tasks_sha256"]), (i, c)


@pytest.mark.parametrize("m", [1, 2, 3])
def test_planted_partition_mistake_fails_fixture(m):
    """Each planted partition mistake in the oracle (no next-row prefix, no
    current-row prefix, strict packing) changes fixture digests; no
    reference library needed."""
    wrong = 0
    try:
        oracle.set_mutation(m)
        for c in GOLDEN["random"]:
            rp, costs, cap = random_case(c)
            wrong += sha(oracle.partition(rp, costs, cap)) != c["tasks_sha256"]
    finally:
        oracle.set_mutation(0)
    assert wrong > 0


# ------------------------------------------- S selection and the cost file
HOST = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "host_golden.json")))


def test_candidate_w_and_capacity_match_reference_fixture():
    for c in HOST["recommended_candidate_w"]:
        assert oracle.recommended_candidate_w(c["nnz"]) == c["w"], c
        assert capi.recommended_candidate_w(c["nnz"]) == c["w"], c
    for c in HOST["capacity_from_s"]:
        cap = float.fromhex(c["capacity"])
        assert oracle.capacity_from_s(c["s"], c["costs"]) == cap, c
        assert capi.capacity_from_s(c["s"], c["costs"]) == cap, c


def test_wave_based_s_matches_reference_fixture():
    for c in HOST["wave_based_s"]:
        if c["error"] is None:
            assert oracle.wave_based_s(c["nnz"], 2, c["cu"], c["wave"]) == c["s"], c
            assert capi.wave_based_s(c["nnz"], 2, c["cu"], c["wave"]) == c["s"], c
        else:
            assert oracle.wave_based_s(c["nnz"], 2, c["cu"], c["wave"]) == -1, c
            with pytest.raises(capi.CwlbError) as e:
                capi.wave_based_s(c["nnz"], 2, c["cu"], c["wave"])
            assert e.value.status == capi.INVALID_ARG


def test_candidate_search_matches_reference_fixture():
    for c in HOST["candidate_search_bounds"]:
        if c["error"] is None:
            assert list(oracle.candidate_search_bounds(c["values"], c["best"])) == c["bounds"]
            assert list(capi.candidate_search_bounds(c["values"], c["best"])) == c["bounds"]
        else:
            with pytest.raises(ValueError):
                oracle.candidate_search_bounds(c["values"], c["best"])
            with pytest.raises(capi.CwlbError):
                capi.candidate_search_bounds(c["values"], c["best"])
    for name in ("candidate_search_by_count", "candidate_search_by_step"):
        for c in HOST[name]:
            args = (c["lower"], c["upper"], c["third"])
            if c["error"] is None:
                assert getattr(oracle, name)(*args) == c["values"], (name, c)
                assert getattr(capi, name)(*args) == c["values"], (name, c)
            else:
                with pytest.raises(ValueError):
                    getattr(oracle, name)(*args)
                with pytest.raises(capi.CwlbError):
                    getattr(capi, name)(*args)


def test_positive_search_argument_matches_reference_fixture():
    from dropin_util import ProbeError, probe
    for c in HOST["positive_search_argument"]:
        if c["error"] is None:
            assert probe("posarg", c["text"]).split()[1] == str(c["value"]), c
        else:
            with pytest.raises(ProbeError) as e:
                probe("posarg", c["text"])
            assert (e.value.kind == "invalid_argument") == (c["error"] == "invalid_argument"), c


def test_cost_files_match_reference_fixture(tmp_path):
    for c in HOST["cost_files"]:
        assert oracle.format_costs(c["costs"], c["precision"]) == c["text"], c
        path = tmp_path / "costs.txt"
        capi.save_costs(c["costs"], path, precision=c["precision"])
        assert path.read_text() == c["text"], c
        if c["precision"] == 6:
            assert list(capi.read_costs(path)) == [float(f"{x:.6f}") for x in c["costs"]]
