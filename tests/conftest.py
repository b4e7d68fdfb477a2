"""Shared test set-up: import paths, the `gpu` marker, common fixtures."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "ane-infer_amd"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle

    if not os.path.exists(oracle.LIB_PATH):
        oracle.build()
    return oracle


def rel_errs(y, ref):
    """(relative L2 error, max-abs error relative to max |ref|), both in float64."""
    import numpy as np

    y = np.asarray(y, np.float64).reshape(-1)
    ref = np.asarray(ref, np.float64).reshape(-1)
    l2 = float(np.linalg.norm(y - ref) / max(np.linalg.norm(ref), 1e-300))
    mx = float(np.max(np.abs(y - ref)) / max(np.max(np.abs(ref)), 1e-300)) if ref.size else 0.0
    return l2, mx


@pytest.fixture(scope="session")
def anehip_mod():
    import anehip

    return anehip


@pytest.fixture(scope="session")
def gpu_ctx(anehip_mod):
    """One bare context on device 0 for the whole GPU session (fails loudly if the
    library or the device is missing: no CPU fallback)."""
    rc = anehip_mod.lib().anehip_init()
    assert rc == 0, anehip_mod.lib().anehip_last_error(None).decode()
    ctx = anehip_mod.Context(0)
    yield ctx
    ctx.close()
