"""Shared fixtures.  CPU tests (-m "not gpu") pin the oracle and check the
library's exports; GPU tests (-m gpu) compare the HIP path, called through
the C ABI, with the oracle on identical seeded inputs."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "ane-lm_amd"), os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")
    config.addinivalue_line("markers", "slow: full-size configuration (seconds of GPU time)")


@pytest.fixture(scope="session")
def orc():
    import oracle

    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def hip():
    """The HIP library on cuda:0; fails (never skips) if it cannot be used."""
    import torch

    assert torch.cuda.is_available(), "GPU test run without a GPU"
    import anelm

    anelm.lib()
    torch.cuda.set_device(0)
    return anelm


@pytest.fixture
def rng():
    return np.random.default_rng(20261201)
