"""ctypes binding of libcwlb_synth.so: seeded synthetic graphs and features.

Graphs come back as ``Graph(n, row_ptr, col_idx, val)`` with int32 CSR arrays
(rows are sources, columns sorted and unique within a row) and unit float32
edge values.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

from . import paths


class _Csr(C.Structure):
    _fields_ = [("n", C.c_int32), ("nnz", C.c_int64),
                ("row_ptr", C.POINTER(C.c_int32)), ("col_idx", C.POINTER(C.c_int32))]


@dataclass
class Graph:
    n: int
    row_ptr: np.ndarray
    col_idx: np.ndarray
    val: np.ndarray

    @property
    def nnz(self) -> int:
        return int(self.row_ptr[-1])


_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(paths.LIB_DIR, "libcwlb_synth.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} missing: build with __graft_entry__.build()")
        L = C.CDLL(path)
        P = C.POINTER(_Csr)
        L.synth_free.argtypes = [P]
        L.synth_erdos_renyi.argtypes = [C.c_int32, C.c_double, C.c_uint64, C.c_int, P]
        L.synth_chung_lu.argtypes = [C.c_int32, C.c_double, C.c_double, C.c_double, C.c_uint64, P]
        L.synth_sbm.argtypes = [C.c_int32, C.c_int32, C.c_double, C.c_double, C.c_uint64, P]
        L.synth_rmat.argtypes = [C.c_int32, C.c_int64, C.c_double, C.c_double, C.c_double,
                                 C.c_uint64, C.c_int, P]
        L.synth_mesh.argtypes = [C.c_int32, C.c_double, C.c_int64, C.c_uint64, P]
        L.synth_features.argtypes = [C.c_int64, C.c_int32, C.c_uint64,
                                     np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")]
        L.synth_max_threads.restype = C.c_int
        for f in (L.synth_erdos_renyi, L.synth_chung_lu, L.synth_sbm, L.synth_rmat, L.synth_mesh):
            f.restype = C.c_int
        _LIB = L
    return _LIB


def _take(fn, *args) -> Graph:
    g = _Csr()
    rc = fn(*args, C.byref(g))
    if rc != 0:
        lib().synth_free(C.byref(g))
        raise RuntimeError(f"synthetic graph generation failed ({rc})")
    try:
        n, nnz = int(g.n), int(g.nnz)
        rp = np.ctypeslib.as_array(g.row_ptr, shape=(n + 1,)).copy()
        ci = (np.ctypeslib.as_array(g.col_idx, shape=(nnz,)).copy() if nnz
              else np.zeros(0, np.int32))
    finally:
        lib().synth_free(C.byref(g))
    return Graph(n, rp, ci, np.ones(nnz, np.float32))


def erdos_renyi(n, avg_deg, seed, exact_pairs=None) -> Graph:
    if exact_pairs is None:
        exact_pairs = n <= 8192
    return _take(lib().synth_erdos_renyi, n, float(avg_deg), seed, int(bool(exact_pairs)))


def chung_lu(n, avg_deg, gamma, max_deg, seed) -> Graph:
    return _take(lib().synth_chung_lu, n, float(avg_deg), float(gamma), float(max_deg), seed)


def sbm(n, n_blocks, p_in, p_out, seed) -> Graph:
    return _take(lib().synth_sbm, n, n_blocks, float(p_in), float(p_out), seed)


def rmat(scale, edges, a, b, c, seed, relabel=True) -> Graph:
    return _take(lib().synth_rmat, scale, edges, float(a), float(b), float(c), seed, int(relabel))


def mesh(side, p_keep, shortcuts, seed) -> Graph:
    return _take(lib().synth_mesh, side, float(p_keep), int(shortcuts), seed)


def features(rows, K, seed=42) -> np.ndarray:
    """U[-1,1) features; identical bits to the device generator in libcwlb."""
    out = np.empty((rows, K), np.float32)
    if rows * K:
        lib().synth_features(rows, K, seed, out.reshape(-1))
    return out
