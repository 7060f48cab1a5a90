"""ctypes binding of the oracle (test infrastructure only).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
import this package.  The product library (``cwlb-spmm_amd``) never does.

``lib()`` loads ``oracle/liboracle.so`` (the C restatement in oracle.c);
``ref()`` loads ``oracle/_ref/libcwlb_ref.so`` (the reference's own pure-C++
host functions, compiled by oracle/ref_build.sh) and returns None when that
library was not built.
"""
from __future__ import annotations

import ctypes as C
import os
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None
_REF = None

i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"oracle not built: {path} (run make -C oracle)")
        L = C.CDLL(path)
        L.oracle_set_mutation.argtypes = [C.c_int]
        L.oracle_reorder_by_degree.argtypes = [C.c_int, i32p, i32p, f32p, i32p, i32p, i32p, f32p]
        L.oracle_reorder_by_degree.restype = C.c_int
        L.oracle_partition.argtypes = [i32p, C.c_long, C.c_double, C.c_double, C.c_double,
                                       C.c_double, C.c_double, C.c_void_p, C.c_long]
        L.oracle_partition.restype = C.c_long
        L.oracle_capacity_from_s.argtypes = [C.c_int] + [C.c_double] * 4
        L.oracle_capacity_from_s.restype = C.c_double
        L.oracle_wave_based_s.argtypes = [C.c_ulonglong, C.c_long, C.c_int, C.c_int]
        L.oracle_wave_based_s.restype = C.c_int
        L.oracle_recommended_candidate_w.argtypes = [C.c_ulonglong, i32p]
        L.oracle_candidate_search_bounds.argtypes = [i32p, C.c_long, C.POINTER(C.c_int),
                                                     C.POINTER(C.c_int)]
        L.oracle_candidate_search_bounds.restype = C.c_int
        for fn in (L.oracle_candidate_search_by_count, L.oracle_candidate_search_by_step):
            fn.argtypes = [C.c_int, C.c_int, C.c_int, i32p, C.c_long, C.POINTER(C.c_int)]
            fn.restype = C.c_long
        L.oracle_spmm_mean_f32.argtypes = [C.c_int, i32p, i32p, f32p, i32p, f32p, C.c_int,
                                           i32p, C.c_long, f32p]
        L.oracle_spmm_mean_f64.argtypes = [C.c_int, i32p, i32p, f32p, f32p, C.c_int, f64p]
        L.oracle_spmm_mean_f32_omp.argtypes = [C.c_int, i32p, i32p, f32p, i32p, f32p, C.c_int,
                                               i32p, C.c_long, f32p, C.c_int]
        L.oracle_max_threads.restype = C.c_int
        L.oracle_cost_coefficients.argtypes = [f64p, C.c_int, C.c_int, C.c_int, f64p,
                                               np.ctypeslib.ndpointer(dtype=np.int64,
                                                                      flags="C_CONTIGUOUS")]
        L.oracle_format_costs.argtypes = [f64p, C.c_int, C.c_char_p, C.c_long]
        L.oracle_format_costs.restype = C.c_int
        L.oracle_parse_costs.argtypes = [C.c_char_p, f64p]
        L.oracle_parse_costs.restype = C.c_int
        _LIB = L
    return _LIB


def ref_built() -> bool:
    """Whether oracle/_ref/libcwlb_ref.so exists (checked without loading it)."""
    return os.path.exists(os.path.join(HERE, "_ref", "libcwlb_ref.so"))


def ref():
    """The reference's own partition / S-selection / cost-file functions, or
    None.  Loaded on first use, so that merely collecting tests does not map
    the library."""
    global _REF
    if _REF is None:
        path = os.path.join(HERE, "_ref", "libcwlb_ref.so")
        if not os.path.exists(path):
            return None
        R = C.CDLL(path)
        R.cwlbref_partition.argtypes = [i32p, C.c_long] + [C.c_double] * 5 + [C.c_void_p, C.c_long]
        R.cwlbref_partition.restype = C.c_long
        R.cwlbref_capacity_from_s.argtypes = [C.c_int] + [C.c_double] * 4
        R.cwlbref_capacity_from_s.restype = C.c_double
        R.cwlbref_wave_based_s.argtypes = [i32p, C.c_long, C.c_int, C.c_int, C.POINTER(C.c_int)]
        R.cwlbref_wave_based_s.restype = C.c_int
        R.cwlbref_recommended_candidate_w.argtypes = [C.c_ulonglong, i32p]
        R.cwlbref_candidate_search_bounds.argtypes = [i32p, C.c_long, C.POINTER(C.c_int),
                                                      C.POINTER(C.c_int)]
        R.cwlbref_candidate_search_bounds.restype = C.c_int
        for fn in (R.cwlbref_candidate_search_by_count, R.cwlbref_candidate_search_by_step):
            fn.argtypes = [C.c_int, C.c_int, C.c_int, i32p, C.c_long, C.POINTER(C.c_int)]
            fn.restype = C.c_long
        R.cwlbref_positive_search_argument.argtypes = [C.c_char_p, C.POINTER(C.c_int)]
        R.cwlbref_positive_search_argument.restype = C.c_int
        R.cwlbref_save_costs.argtypes = [C.c_double] * 4 + [C.c_char_p, C.c_int, C.c_int]
        R.cwlbref_save_costs.restype = C.c_int
        R.cwlbref_read_costs.argtypes = [C.c_char_p, f64p]
        R.cwlbref_read_costs.restype = C.c_int
        _REF = R
    return _REF


def set_mutation(m: int) -> None:
    lib().oracle_set_mutation(int(m))


# ---------------------------------------------------------------- helpers
def _i32(a):
    return np.ascontiguousarray(a, dtype=np.int32)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def reorder_by_degree(rp, ci, val):
    """main.cpp:197-278 -> (origin, rp_out, ci_out, val_out)."""
    rp, ci, val = _i32(rp), _i32(ci), _f32(val)
    n = len(rp) - 1
    origin = np.zeros(max(n, 0), np.int32)
    rp_out = np.zeros(max(n + 1, 1), np.int32)
    ci_out = np.zeros(len(ci), np.int32)
    val_out = np.zeros(len(val), np.float32)
    rc = lib().oracle_reorder_by_degree(n, rp, ci, val, origin, rp_out, ci_out, val_out)
    if rc != 0:
        raise RuntimeError(f"oracle reorder failed ({rc})")
    return origin, rp_out, ci_out, val_out


def _partition_call(fn, rp, costs, capacity):
    rp = _i32(rp)
    cc, cl, cs, ca = (float(x) for x in costs)
    n = fn(rp, len(rp), cc, cl, cs, ca, float(capacity), None, 0)
    out = np.zeros((max(n, 1), 4), np.int32)
    n2 = fn(rp, len(rp), cc, cl, cs, ca, float(capacity), out.ctypes.data, n)
    assert n2 == n
    return out[:n].copy()


def partition(rp, costs, capacity):
    """utils.cpp:832-1021 -> int32 array (T, 4): row_start, row_end, first_row_offset, last_row_nnz."""
    return _partition_call(lib().oracle_partition, rp, costs, capacity)


def ref_partition(rp, costs, capacity):
    R = ref()
    if R is None:
        return None
    return _partition_call(R.cwlbref_partition, rp, costs, capacity)


def capacity_from_s(s, costs):
    return lib().oracle_capacity_from_s(int(s), *(float(x) for x in costs))


def wave_based_s(nnz, rp_len, cu, wave):
    return lib().oracle_wave_based_s(int(nnz), int(rp_len), int(cu), int(wave))


def recommended_candidate_w(nnz):
    out = np.zeros(3, np.int32)
    lib().oracle_recommended_candidate_w(int(nnz), out)
    return [int(x) for x in out]


def candidate_search_bounds(values, best):
    lo, hi = C.c_int(), C.c_int()
    rc = lib().oracle_candidate_search_bounds(_i32(values), int(best), C.byref(lo), C.byref(hi))
    if rc:
        raise ValueError("invalid candidate values or index")
    return lo.value, hi.value


def _search(fn, a, b, c):
    err = C.c_int()
    n = fn(int(a), int(b), int(c), np.zeros(1, np.int32), 0, C.byref(err))
    if err.value:
        raise ValueError("invalid search plan")
    out = np.zeros(max(n, 1), np.int32)
    fn(int(a), int(b), int(c), out, n, C.byref(err))
    return [int(x) for x in out[:n]]


def candidate_search_by_count(lo, hi, count):
    return _search(lib().oracle_candidate_search_by_count, lo, hi, count)


def candidate_search_by_step(lo, hi, step):
    return _search(lib().oracle_candidate_search_by_step, lo, hi, step)


def spmm_mean_f32(rp, ci, val, origin, H, tasks):
    """parallelMatrix.cpp:148-236 in reference value order (sequential)."""
    H = _f32(H)
    n = len(rp) - 1
    K = H.shape[1] if H.ndim == 2 else 0
    C_out = np.zeros((n, K), np.float32)
    t = _i32(tasks).reshape(-1, 4) if len(tasks) else np.zeros((0, 4), np.int32)
    lib().oracle_spmm_mean_f32(n, _i32(rp), _i32(ci), _f32(val), _i32(origin), H.reshape(-1)
                               if H.size else np.zeros(1, np.float32), K,
                               np.ascontiguousarray(t.reshape(-1)) if t.size else np.zeros(4, np.int32),
                               len(t), C_out.reshape(-1) if C_out.size else np.zeros(1, np.float32))
    return C_out


def spmm_mean_f32_omp(rp, ci, val, origin, H, tasks, threads=0, out=None):
    H = _f32(H)
    n = len(rp) - 1
    K = H.shape[1]
    C_out = np.zeros((n, K), np.float32) if out is None else out
    t = _i32(tasks).reshape(-1)
    lib().oracle_spmm_mean_f32_omp(n, _i32(rp), _i32(ci), _f32(val), _i32(origin), H.reshape(-1), K,
                                   t, len(t) // 4, C_out.reshape(-1), int(threads))
    return C_out


def spmm_mean_f64(rp, ci, val, H):
    """Closed form on the ORIGINAL csr: C[i] = (A H)[i] / deg(i), 0 for deg 0."""
    H = _f32(H)
    n = len(rp) - 1
    K = H.shape[1]
    out = np.zeros((n, K), np.float64)
    lib().oracle_spmm_mean_f64(n, _i32(rp), _i32(ci), _f32(val), H.reshape(-1), K, out.reshape(-1))
    return out


def cost_coefficients(ms4, K, WI, writers):
    """utils.cpp:419-421, 522-524, 583-585, 791-806 -> (coefficients[4], ops[4])."""
    out = np.zeros(4, np.float64)
    ops = np.zeros(4, np.int64)
    lib().oracle_cost_coefficients(np.ascontiguousarray(ms4, np.float64), int(K), int(WI),
                                   int(writers), out, ops)
    return [float(x) for x in out], [int(x) for x in ops]


def max_threads():
    return lib().oracle_max_threads()


def format_costs(c4, precision=6):
    buf = C.create_string_buffer(4096)
    n = lib().oracle_format_costs(np.asarray(c4, np.float64), int(precision), buf, 4096)
    return buf.value[:n].decode()


def parse_costs(text):
    out = np.zeros(4, np.float64)
    ok = lib().oracle_parse_costs(text.encode(), out)
    return [float(x) for x in out] if ok else None


def ref_format_costs(c4, precision=6):
    """Bytes written by the reference's save_costs_one_per_line, or None."""
    R = ref()
    if R is None:
        return None
    with tempfile.TemporaryDirectory() as d:
        p = os.path.join(d, "costs.txt")
        ok = R.cwlbref_save_costs(*(float(x) for x in c4), p.encode(), 0, int(precision))
        if not ok:
            return None
        with open(p) as f:
            return f.read()
