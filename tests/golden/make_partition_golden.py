"""Writes tests/golden/partition_golden.json: task-list digests computed by
the reference's own costWeightedTaskPartitioning (utils.cpp:832-1021) and
capacity_from_s (main.cpp:281-292), compiled from the reference sources by
oracle/ref_build.sh into oracle/_ref/libcwlb_ref.so.

Run in a container where that library is built:

    python tests/golden/make_partition_golden.py

For every workload (the five full-size graphs and their scaled-down
siblings) the fixture stores
  - SHA-256 of the generated CSR (row_ptr, col_idx) so that drift of the
    synthetic generators is caught before the partition is compared;
  - SHA-256 of the degree permutation and reordered row offsets from numpy's
    stable argsort of the degrees (the (degree, id) order of
    main.cpp:229-238) and the exclusive prefix of the sorted degrees
    (main.cpp:247-253);
  - per (cost vector, S): the reference's capacity (as a hex float), the
    task count and SHA-256 of the (T, 4) int32 task array in row-major
    little-endian order.
Task arrays themselves are small enough to keep only for the scaled-down
graphs' smallest cases; the digests pin the rest.

A "random" section adds short degree sequences (sorted and unsorted, with
empty rows and hub rows) under assorted cost vectors and capacities, drawn
from a seeded generator and stored with their inputs (degrees as a
space-separated string): sorted graphs meet the
current-row prefix absorption (utils.cpp:879-912) at most once, at the first
long row, so these cases are what exercise it often.
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (ROOT, os.path.join(ROOT, "cwlb-spmm_amd"), os.path.dirname(HERE)):
    if p not in sys.path:
        sys.path.insert(0, p)

import oracle  # noqa: E402
from conftest import SKEWED_COSTS, UNIT_COSTS  # noqa: E402
from cwlb_amd import workloads  # noqa: E402

OUT = os.path.join(HERE, "partition_golden.json")
COST_FILE = os.path.join(ROOT, "cwlb-spmm_amd", "resources", "spmm_costs_gfx950.txt")
MESH_SWEEP = [32, 64, 128, 256, 512]


def sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).astype("<i4", copy=False).tobytes()).hexdigest()


def degree_order(rp):
    deg = np.diff(rp.astype(np.int64))
    perm = np.argsort(deg, kind="stable").astype(np.int32)
    rp_sorted = np.concatenate([[0], np.cumsum(deg[perm])]).astype(np.int32)
    return perm, rp_sorted


def ref_capacity(S, costs):
    return oracle.ref().cwlbref_capacity_from_s(int(S), *(float(c) for c in costs))


def entry(g, cost_sets, keep_tasks_below=0):
    perm, rp = degree_order(g.row_ptr)
    parts = []
    for name, costs, s_list in cost_sets:
        for S in s_list:
            cap = ref_capacity(S, costs)
            tasks = oracle.ref_partition(rp, costs, cap)
            rec = {"costs": name, "S": int(S), "capacity": float(cap).hex(),
                   "n_tasks": int(len(tasks)), "tasks_sha256": sha(tasks)}
            if len(tasks) <= keep_tasks_below:
                rec["tasks"] = tasks.tolist()
            parts.append(rec)
    return {"n": int(g.n), "nnz": int(g.nnz), "row_ptr_sha256": sha(g.row_ptr),
            "col_idx_sha256": sha(g.col_idx), "origin_sha256": sha(perm),
            "sorted_row_ptr_sha256": sha(rp), "partitions": parts}


COST_CHOICES = [0.0, 0.01, 0.125, 0.25, 0.5, 1.0, 1.7, 3.3, 12.5]


def random_cases(count=160, seed=2024):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(count):
        n = int(rng.integers(1, 60))
        kind = i % 4
        if kind == 0:
            degs = np.sort(rng.integers(0, int(rng.integers(1, 100)), n))
        elif kind == 1:
            degs = np.sort(rng.zipf(1.6, n).clip(0, 2000) - 1)
        elif kind == 2:
            degs = rng.integers(0, 40, n)
        else:
            degs = np.sort(np.concatenate([np.zeros(n // 2, int),
                                           rng.integers(20, 300, n - n // 2)]))
        costs = [float(rng.choice(COST_CHOICES)) for _ in range(4)]
        if rng.random() < 0.8:
            S = int(rng.integers(1, 40))
            cap = ref_capacity(S, costs)
        else:
            S, cap = None, float(rng.random() * 40)
        rp = np.concatenate([[0], np.cumsum(degs)]).astype(np.int32)
        tasks = oracle.ref_partition(rp, costs, cap)
        cases.append({"degrees": " ".join(str(int(d)) for d in degs), "costs": costs,
                      "S": S, "capacity": float(cap).hex(), "n_tasks": int(len(tasks)),
                      "tasks_sha256": sha(tasks)})
    return cases


def main():
    if oracle.ref() is None:
        sys.exit("oracle/_ref/libcwlb_ref.so is not built (needs the reference sources)")
    gfx950 = [float(x) for x in open(COST_FILE).read().split()]
    costs = {"unit": list(UNIT_COSTS), "skewed": list(SKEWED_COSTS), "gfx950": gfx950}
    out = {"generator": "tests/golden/make_partition_golden.py", "costs": costs,
           "small": {}, "full": {}, "random": random_cases()}
    for cfg in (1, 2, 3, 4, 5):
        g = workloads.small(cfg)
        s_list = workloads.candidate_s(g.nnz, 256) + [1, 3, 64]
        sets = [(k, costs[k], s_list) for k in ("unit", "skewed", "gfx950")]
        out["small"][str(cfg)] = entry(g, sets, keep_tasks_below=64)
        print(f"small {cfg}: n={g.n} nnz={g.nnz}", flush=True)
    for cfg in (1, 2, 3, 4, 5):
        g = workloads.graph(cfg)
        s_list = workloads.candidate_s(g.nnz, 256)
        if cfg == 5:
            s_list = sorted(set(s_list + MESH_SWEEP))
        out["full"][str(cfg)] = entry(g, [("gfx950", costs["gfx950"], s_list)])
        print(f"full {cfg} ({workloads.NAMES[cfg]}): n={g.n} nnz={g.nnz} S={s_list}", flush=True)
        del g
    with open(OUT, "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
        f.write("\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
