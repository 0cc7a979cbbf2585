"""The reference-signature C++ layer (ane_lm::rmsnorm, ane_lm::sample_token,
...) called from C++ the way the reference's model and generation code
call it, checked against the oracle by tests/cpp/dropin_check."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu
BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "dropin_check")


def test_dropin_layer(hip):
    assert os.path.exists(BIN), "tests/cpp/dropin_check not built (python ane-lm_amd/build.py)"
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "FAIL" not in r.stdout
