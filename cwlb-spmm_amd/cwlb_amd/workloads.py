"""The synthetic workloads the SpMM is checked and measured on.

Five configurations (rows are sources, unit edge values, features U[-1,1)
with seed 42, graph seed = configuration number):

  1 er4096_k32      Erdos-Renyi, N=4,096, average out-degree 8, K=32
  2 chunglu1m_k64   Chung-Lu power law, N=1,000,000, average degree 10,
                    exponent 2.1, weights capped at 50,000, K=64
  3 sbm240k_k600    stochastic block model, 50 blocks of 4,800,
                    p_in:p_out = 20:1, average degree 480, K=600
  4 rmat22_k128     R-MAT a=.57 b=c=.19 d=.05, N=2^22, 2^26 samples,
                    relabelled, duplicates removed, K=128
  5 mesh16m_k32     4,000 x 4,000 lattice, 95% lattice edges + 5% uniform
                    shortcuts, average degree 2.5, K=32

``small(i)`` gives a scaled-down graph of the same family for parity tests
that must finish in seconds on the CPU oracle.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import capi, synth

FEATURE_SEED = 42

SBM_P_OUT = 480.0 / (20 * 4799 + 235200)
SBM_P_IN = 20 * SBM_P_OUT
MESH_SIDE = 4000
MESH_P_KEEP = 0.95 * 2.5 * MESH_SIDE**2 / (4 * MESH_SIDE**2 - 4 * MESH_SIDE)
MESH_SHORTCUTS = int(0.05 * 2.5 * MESH_SIDE**2)

NAMES = {1: "er4096_k32", 2: "chunglu1m_k64", 3: "sbm240k_k600", 4: "rmat22_k128",
         5: "mesh16m_k32"}
FEATURE_DIM = {1: 32, 2: 64, 3: 600, 4: 128, 5: 32}


def graph(cfg: int) -> synth.Graph:
    """Full-size graph of configuration cfg."""
    if cfg == 1:
        return synth.erdos_renyi(4096, 8, 1)
    if cfg == 2:
        return synth.chung_lu(1_000_000, 10, 2.1, 50_000, 2)
    if cfg == 3:
        return synth.sbm(240_000, 50, SBM_P_IN, SBM_P_OUT, 3)
    if cfg == 4:
        return synth.rmat(22, 1 << 26, 0.57, 0.19, 0.19, 4)
    if cfg == 5:
        return synth.mesh(MESH_SIDE, MESH_P_KEEP, MESH_SHORTCUTS, 5)
    raise ValueError(cfg)


def small(cfg: int, seed: int | None = None) -> synth.Graph:
    """A scaled-down member of configuration cfg's family."""
    s = cfg if seed is None else seed
    if cfg == 1:
        return synth.erdos_renyi(4096, 8, s)
    if cfg == 2:
        return synth.chung_lu(20_000, 10, 2.1, 2_000, s)
    if cfg == 3:
        p_out = 48.0 / (20 * 499 + 4500)
        return synth.sbm(5_000, 10, 20 * p_out, p_out, s)
    if cfg == 4:
        return synth.rmat(14, 1 << 18, 0.57, 0.19, 0.19, s)
    if cfg == 5:
        side = 150
        p = 0.95 * 2.5 * side**2 / (4 * side**2 - 4 * side)
        return synth.mesh(side, p, int(0.05 * 2.5 * side**2), s)
    raise ValueError(cfg)


@dataclass
class Prepared:
    """Reordered CSR + task list of one graph at one segment size S."""
    n: int
    nnz: int
    origin: np.ndarray
    row_ptr: np.ndarray
    col_idx: np.ndarray
    val: np.ndarray
    tasks: np.ndarray
    S: int
    capacity: float


def prepare(g: synth.Graph, costs4, S: int) -> Prepared:
    origin, rp, ci, val = capi.reorder_by_degree(g.row_ptr, g.col_idx, g.val)
    cap = capi.capacity_from_s(S, costs4)
    tasks = capi.partition(rp, costs4, cap)
    return Prepared(g.n, g.nnz, origin, rp, ci, val, tasks, S, cap)


def candidate_s(nnz: int, compute_units: int):
    """The three wave-based segment sizes of the --candidates mode (main.cpp:548-549)."""
    return [capi.wave_based_s(nnz, 2, compute_units, w) for w in capi.recommended_candidate_w(nnz)]


def algorithmic_bytes(n: int, nnz: int, K: int, n_tasks: int) -> int:
    """Bytes a launch must move at least once per access, counted per access:
    row_ptr 4(N+1) + col_idx/val 8 nnz + one K-float row gather per nonzero
    4 nnz K + C written once 4 N K + Origin_local 4 N + task descriptors 16 T."""
    return 4 * (n + 1) + 8 * nnz + 4 * nnz * K + 4 * n * K + 4 * n + 16 * n_tasks


def compulsory_bytes(g_rows_with_input: int, n: int, nnz: int, K: int) -> int:
    """CSR once, every referenced H row once, C once."""
    return 4 * (n + 1) + 8 * nnz + 4 * g_rows_with_input * K + 4 * n * K + 4 * n
