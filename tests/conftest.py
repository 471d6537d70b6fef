"""Shared test setup: import paths, the `gpu` marker and device fixtures."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("prism-inference_amd", "oracle"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); runs through the C ABI")


@pytest.fixture(scope="session")
def hip():
    import prism_amd as P
    h = P.Hip()
    if h.device_count() < 1:
        raise RuntimeError("gpu test selected but no HIP device is visible")
    return h


@pytest.fixture(scope="session")
def engine(hip):
    import prism_amd as P
    e = P.Engine(0)
    yield e
    e.close()


class DeviceArena:
    """A device allocation freed when the test ends."""

    def __init__(self, hip, nbytes, zero=True):
        self.hip = hip
        self.nbytes = int(nbytes)
        self.ptr = hip.malloc(self.nbytes)
        if zero:
            hip.memset(self.ptr, 0, self.nbytes)

    def free(self):
        if self.ptr:
            self.hip.free(self.ptr)
            self.ptr = 0


@pytest.fixture
def device_arena(hip):
    made = []

    def make(nbytes, zero=True):
        a = DeviceArena(hip, nbytes, zero)
        made.append(a)
        return a

    yield make
    hip.sync()
    for a in made:
        a.free()


def errors(got: np.ndarray, ref: np.ndarray):
    d = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    return float(d.max()), float(d.mean())
