"""Shared fixtures. `gpu` tests need an MI355X and the built libxpose.so; the
rest run on the CPU (oracle, host logic, ABI surface)."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (gfx950) and libxpose.so")


@pytest.fixture(scope="session")
def xh():
    """The product binding for host-side entry points (synthetic inputs, ABI
    surface); does not touch the GPU."""
    import xpose_amd
    xpose_amd.lib()
    return xpose_amd


@pytest.fixture(scope="session")
def xp():
    """The product binding, initialised on device 0 (GPU tests only)."""
    import xpose_amd
    xpose_amd.init(0)
    return xpose_amd


@pytest.fixture(scope="session")
def xo():
    import oracle
    oracle.lib()
    return oracle


def allclose_report(got, want, rtol, atol):
    """numpy-allclose verdict plus the worst element, for assertion messages."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want)
    bad = err > atol + rtol * np.abs(want)
    i = int(np.argmax(err - (atol + rtol * np.abs(want))))
    return (not bad.any() and np.isfinite(got).all(),
            f"max_abs={err.max():.3e} worst[{i}] got={got.flat[i]!r} want={want.flat[i]!r} "
            f"n_bad={int(bad.sum())}/{bad.size}")


# Device buffers handed to the library as raw pointers must outlive the call
# and the kernels it queues: a DeviceBuffer created inside an argument list
# would be freed before the launch. `hold` keeps them until the test ends.
_held = []


def hold(buf):
    _held.append(buf)
    return buf.vp


@pytest.fixture(autouse=True)
def _release_held_buffers():
    yield
    if _held:
        import xpose_amd
        try:
            xpose_amd.synchronize()
        finally:
            _held.clear()
