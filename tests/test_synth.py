"""Synthetic workload generators: determinism, CSR validity, family shape."""
import numpy as np
import pytest

from cwlb_amd import synth, workloads


def assert_csr(g):
    assert g.row_ptr[0] == 0 and np.all(np.diff(g.row_ptr) >= 0)
    assert len(g.col_idx) == g.row_ptr[-1] == len(g.val)
    assert g.col_idx.min(initial=0) >= 0 and g.col_idx.max(initial=0) < max(g.n, 1)
    for r in range(0, g.n, max(1, g.n // 300)):
        row = g.col_idx[g.row_ptr[r]:g.row_ptr[r + 1]]
        assert np.all(np.diff(row) > 0), "columns sorted and unique"


@pytest.mark.parametrize("cfg", [1, 2, 3, 4, 5])
def test_small_generators_valid_and_deterministic(cfg):
    a, b = workloads.small(cfg), workloads.small(cfg)
    assert_csr(a)
    assert np.array_equal(a.row_ptr, b.row_ptr) and np.array_equal(a.col_idx, b.col_idx)
    assert workloads.small(cfg, seed=99).nnz != a.nnz or not np.array_equal(
        workloads.small(cfg, seed=99).col_idx, a.col_idx)


def test_config1_shape():
    g = workloads.graph(1)
    assert g.n == 4096
    assert abs(g.nnz / g.n - 8) < 0.3
    for r in range(g.n):
        assert r not in g.col_idx[g.row_ptr[r]:g.row_ptr[r + 1]]


def test_rmat_skew():
    g = synth.rmat(16, 1 << 20, 0.57, 0.19, 0.19, 4)
    d = np.diff(g.row_ptr)
    assert (d == 0).mean() > 0.3 and d.max() > 50 * d.mean()


def test_features_range_and_exactness():
    H = synth.features(300, 37, 42)
    assert H.min() >= -1.0 and H.max() < 1.0
    assert np.array_equal(H * 2**23, np.round(H * 2**23))
    assert np.array_equal(H, synth.features(300, 37, 42))
    assert not np.array_equal(H, synth.features(300, 37, 43))
    assert abs(H.mean()) < 0.02
