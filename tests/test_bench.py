"""bench.py's host-side helpers (no GPU): the measured-traffic lookup reads
the committed rocprofv3 summaries by segment size, and the algorithmic-bytes
formula matches its per-unit statement."""
import importlib
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def bench():
    sys.path.insert(0, ROOT)
    return importlib.import_module("bench")


# The S values the summaries were measured at (the three wave-based
# candidates of each workload with 256 CUs).
MEASURED = {4: (32, 63, 125), 5: (39, 77, 153), 2: (35, 70, 139), 3: (55, 110, 220)}


@pytest.mark.parametrize("cfg", sorted(MEASURED))
def test_traffic_figure_per_candidate_s(bench, cfg):
    for S in MEASURED[cfg]:
        t = bench.measured_traffic(cfg, S)
        assert t is not None and t > 0, (cfg, S)


def test_traffic_unknown_s_or_workload_is_none(bench):
    assert bench.measured_traffic(4, 64) is None
    assert bench.measured_traffic(3, 56) is None
    assert bench.measured_traffic(1, 9) is None  # no summary for the small ER graph


def test_traffic_figures_are_consistent_with_algorithmic_bytes(bench):
    """Measured traffic below the algorithmic bytes where caches serve
    repeated feature rows (R-MAT, Chung-Lu, mesh), and within a few percent
    above it where every gather misses and rows straddle cache lines (SBM)."""
    from cwlb_amd import workloads
    ratios = {4: (63, 4194304, 65245138, 128, 1084009), 3: (55, 240000, 115180734, 600, 2217632)}
    for cfg, (S, n, nnz, K, T) in ratios.items():
        r = bench.measured_traffic(cfg, S) / workloads.algorithmic_bytes(n, nnz, K, T)
        assert (0.5 < r < 1.0) if cfg == 4 else (1.0 < r < 1.05), (cfg, r)


def test_algorithmic_bytes_formula():
    """4(N+1) + 8 nnz + 4 nnz K + 4 N K + 4 N + 16 T, the per-unit figures
    stated next to the roofline: 8 B + 4K B per nonzero, 4 B + 4K B + 4 B per
    row, 16 B per task."""
    from cwlb_amd import workloads
    n, nnz, K, T = 7, 11, 3, 5
    assert workloads.algorithmic_bytes(n, nnz, K, T) == (
        4 * (n + 1) + 8 * nnz + 4 * nnz * K + 4 * n * K + 4 * n + 16 * T)
    assert workloads.algorithmic_bytes(4194304, 65245138, 128, 1084009) == 36125853988
