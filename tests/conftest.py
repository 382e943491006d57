import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "self-evolve-diffusion-cpp_amd")
for p in (PKG, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: full-size north-star shape")


@pytest.fixture(scope="session")
def oracle():
    import pyoracle

    pyoracle.lib()
    return pyoracle


@pytest.fixture(scope="session")
def ref():
    import pyoracle

    if not pyoracle.Ref.available():
        pytest.skip("oracle/_ref (reference-compiled oracle) not built")
    return pyoracle.Ref()


@pytest.fixture(scope="session")
def sdq_dev():
    """Initialised sdq on cuda:0; fails (not skips) when the library is missing."""
    import torch

    import sdq

    sdq.load_library()
    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    sdq.init(0)
    return torch.device("cuda:0")


def bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


def assert_bitexact(got, want, what=""):
    got = np.ascontiguousarray(got)
    want = np.ascontiguousarray(want)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    if got.dtype == np.float32:
        g, w = bits(got), bits(want)
    else:
        g, w = got, want
    bad = np.argwhere(g != w)
    if bad.size:
        i = tuple(bad[0])
        raise AssertionError(f"{what}: {len(bad)} of {got.size} differ; first at {i}: "
                             f"got {got[i]!r} want {want[i]!r}")
