"""Shared test setup: markers, import paths, builds, seeded model helpers."""
import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "lfm2-w9100-rust_amd")
ORACLE = os.path.join(REPO, "oracle")
for p in (PKG, ORACLE):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device; parity through the C ABI")
    config.addinivalue_line("markers", "slow: full-size model checks")


@pytest.fixture(scope="session", autouse=True)
def _release_engines():
    """Engines and device buffers the tests left open are released when the
    session ends, while the HIP runtime is still up."""
    yield
    import lfm_hip
    lfm_hip._close_live_engines()


@pytest.fixture(scope="session")
def lfm():
    import lfm_hip
    lfm_hip.lib()
    return lfm_hip


@pytest.fixture(scope="session")
def oracle():
    import lfm_oracle
    lfm_oracle.lib()
    lfm_oracle.set_threads(min(16, os.cpu_count() or 1))
    return lfm_oracle


@pytest.fixture(scope="session")
def gpu(lfm):
    """GPU tests fail (not skip) when no device is visible: the HIP path must run."""
    n = lfm.device_count()
    assert n > 0, "no HIP device visible: GPU parity tests need an MI355X"
    return lfm


def rel_l2(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))
