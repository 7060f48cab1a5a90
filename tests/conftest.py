"""Test configuration: paths, the `gpu` marker and shared fixtures.

`-m "not gpu"` runs on any machine (oracle checks, host library, exports);
`-m gpu` needs an MI355X and calls the HIP path through the C ABI.
"""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "cwlb-spmm_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

# Cost vectors used for partitions in the tests (exact binary fractions, and
# one with the calibrated gfx950 coefficients' magnitudes).
UNIT_COSTS = (0.25, 0.75, 0.5, 0.5)
SKEWED_COSTS = (0.125, 1.375, 0.75, 3.5)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def gpu_ctx():
    import torch
    from cwlb_amd import capi
    if not torch.cuda.is_available():
        pytest.fail("gpu test selected but no GPU is visible")
    torch.cuda.init()
    ctx = capi.Context(0, torch.cuda.current_stream().cuda_stream)
    yield ctx
    ctx.close()


@pytest.fixture
def rng():
    return np.random.default_rng(12345)
