import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "mlx-bun_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built libmlxq.so")


@pytest.fixture(scope="session")
def O():
    """The CPU oracle (built on first use)."""
    from oracle import oracle

    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def mlxq_dev():
    """libmlxq initialised on device 0 (fails loudly without a GPU or library)."""
    import mlxq

    mlxq.ensure_init(0)
    return mlxq


def assert_close(got, ref, atol=1e-2, rtol=1e-3, what=""):
    """|got - ref| <= atol + rtol * |ref| elementwise (the attention / matmul
    tolerance against the fp32 reference: max-abs 1e-2, relative 1e-3)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = np.abs(got - ref)
    bad = err > atol + rtol * np.abs(ref)
    if bad.any():
        i = np.unravel_index(np.argmax(err - (atol + rtol * np.abs(ref))), err.shape)
        raise AssertionError(f"{what}: {bad.sum()} / {bad.size} elements out of tolerance; worst at {i}: "
                             f"got {got[i]} ref {ref[i]} (max abs err {err.max():.3g})")
