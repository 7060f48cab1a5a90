"""Writes tests/golden/host_golden.json: input/output vectors of the
reference's own segment-size selection (main.cpp:87-167, 281-321) and cost
file writer (utils.cpp:1024-1072), compiled from the reference sources by
oracle/ref_build.sh into oracle/_ref/libcwlb_ref.so.

Run in a container where that library is built:

    python tests/golden/make_host_golden.py

Each entry holds the inputs and the reference's output (or the kind of
error it raised: "invalid_argument" or "other").  Doubles are stored as hex
floats; cost files as their exact text.
"""
import ctypes as C
import json
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (ROOT, os.path.join(ROOT, "cwlb-spmm_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

import oracle  # noqa: E402

OUT = os.path.join(HERE, "host_golden.json")
ERR = {0: None, 1: "invalid_argument", 2: "other"}
COST_CHOICES = [0.0, 0.01, 0.125, 0.25, 0.5, 1.0, 1.7, 3.3, 12.5, -1.0]


def main():
    R = oracle.ref()
    if R is None:
        sys.exit("oracle/_ref/libcwlb_ref.so is not built (needs the reference sources)")
    rng = np.random.default_rng(77)
    out = {"generator": "tests/golden/make_host_golden.py"}

    # recommended_candidate_w: every threshold and its neighbours, then random nnz.
    nnzs = [0, 1]
    for t in (100_000, 500_000, 1_000_000, 5_000_000, 10_000_000, 50_000_000):
        nnzs += [t - 1, t, t + 1]
    nnzs += [int(x) for x in rng.integers(0, 2**40, 40)]
    rec = []
    for nnz in nnzs:
        w = np.zeros(3, np.int32)
        R.cwlbref_recommended_candidate_w(nnz, w)
        rec.append({"nnz": nnz, "w": w.tolist()})
    out["recommended_candidate_w"] = rec

    # capacity_from_s
    cap = []
    for _ in range(200):
        s = int(rng.integers(-3, 5000))
        c4 = [float(rng.choice(COST_CHOICES)) * float(rng.choice([1.0, 0.0137, 3.91])) for _ in range(4)]
        cap.append({"s": s, "costs": c4, "capacity": float(R.cwlbref_capacity_from_s(s, *c4)).hex()})
    out["capacity_from_s"] = cap

    # wave_based_s (row_ptr = [0, nnz]): valid and invalid compute units / waves.
    wb = []
    for _ in range(200):
        nnz = int(rng.integers(0, 2**31 - 1))
        cu = int(rng.choice([-1, 0, 1, 104, 256, 304, int(rng.integers(1, 1000))]))
        w = int(rng.choice([-1, 0, 1, 64, 1024, 4096, 8192, int(rng.integers(1, 100000))]))
        rp = np.array([0, nnz], np.int32)
        err = C.c_int()
        s = R.cwlbref_wave_based_s(rp, 2, cu, w, C.byref(err))
        wb.append({"nnz": nnz, "cu": cu, "wave": w, "s": s if err.value == 0 else None,
                   "error": ERR[err.value]})
    out["wave_based_s"] = wb

    # candidate_search_bounds
    bounds = []
    for _ in range(150):
        v = np.sort(rng.integers(-3, 80, 3)).astype(np.int32)
        if rng.random() < 0.2:
            v = rng.integers(-3, 80, 3).astype(np.int32)
        best = int(rng.integers(-1, 4))
        lo, hi = C.c_int(), C.c_int()
        rc = R.cwlbref_candidate_search_bounds(v, best, C.byref(lo), C.byref(hi))
        bounds.append({"values": v.tolist(), "best": best,
                       "bounds": None if rc else [lo.value, hi.value], "error": ERR[rc]})
    out["candidate_search_bounds"] = bounds

    # candidate_search_by_count / by_step
    for name, fn in (("candidate_search_by_count", R.cwlbref_candidate_search_by_count),
                     ("candidate_search_by_step", R.cwlbref_candidate_search_by_step)):
        cases = []
        for _ in range(150):
            a, b, c = (int(x) for x in rng.integers(-2, 300, 3))
            if rng.random() < 0.7:
                a, b = min(a, b), max(a, b)
            err = C.c_int()
            buf = np.zeros(20000, np.int32)
            n = fn(a, b, c, buf, len(buf), C.byref(err))
            cases.append({"lower": a, "upper": b, "third": c,
                          "values": buf[:n].tolist() if err.value == 0 else None,
                          "error": ERR[err.value]})
        out[name] = cases

    # positive_search_argument
    args = []
    for text in ["1", "7", "42", "0", "-3", "3x", "", " 5", "5 ", "+4", "2147483647",
                 "2147483648", "007", "1e3", "abc"]:
        err = C.c_int()
        v = R.cwlbref_positive_search_argument(text.encode(), C.byref(err))
        args.append({"text": text, "value": v if err.value == 0 else None,
                     "error": ERR[err.value]})
    out["positive_search_argument"] = args

    # cost files: the writer's exact text.
    files = []
    vecs = [[0.004519, 0.015617, 0.010667, 0.540499], [0.25, 0.75, 0.5, 0.5],
            [0.0, -1.5, 1e-9, 123456.789], [1.0 / 3.0, 2.0 / 3.0, 1e-7, 5e-7]]
    vecs += [[float(x) for x in rng.random(4) * 10.0 ** rng.integers(-6, 4)] for _ in range(8)]
    with tempfile.TemporaryDirectory() as d:
        for c4 in vecs:
            for prec in (6, 3, 10):
                path = os.path.join(d, "c.txt")
                assert R.cwlbref_save_costs(*c4, path.encode(), 0, prec)
                files.append({"costs": c4, "precision": prec, "text": open(path).read()})
    out["cost_files"] = files

    with open(OUT, "w") as f:
        json.dump(out, f, separators=(",", ":"))
        f.write("\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
