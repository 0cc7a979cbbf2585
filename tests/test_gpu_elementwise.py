"""SwiGLU / SiLU / mul-sigmoid (core/cpu_ops.cpp:7-23, core/ane_runtime.cpp:393-395)
within 1e-5 relative, and the residual add (qwen3.cpp:516/:527) bit-exact."""
import numpy as np
import pytest

from helpers import REL_TOL, assert_bitexact, dev, host, max_rel_err

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,inter", [(1, 3072), (2048, 3072), (64, 9728), (256, 12288), (3, 1001), (1, 5)])
def test_silu_mul(hip, orc, rng, rows, inter):
    import torch

    g = rng.standard_normal((rows, inter), dtype=np.float32)
    u = rng.standard_normal((rows, inter), dtype=np.float32)
    h = torch.empty(rows, inter, device="cuda")
    hip.silu_mul(h, dev(g), dev(u))
    assert max_rel_err(host(h), orc.silu_mul(g, u)) <= REL_TOL


def test_silu_mul_wide_range(hip, orc, rng):
    import torch

    g = np.concatenate([np.linspace(-80, 80, 40001, dtype=np.float32),
                        np.array([0.0, -0.0, 1e-30, -1e-30, 1e-45, 88.0, -87.0], np.float32)])
    g = np.pad(g, (0, (-g.size) % 4))
    u = rng.uniform(-3, 3, g.size).astype(np.float32)
    h = torch.empty(1, g.size, device="cuda")
    hip.silu_mul(h, dev(g[None]), dev(u[None]))
    assert max_rel_err(host(h)[0], orc.silu_mul(g, u)) <= REL_TOL


def test_silu_mul_strided_gate_up(hip, orc, rng):
    """gate and up as the two halves of one [rows, 2*inter] buffer."""
    import torch

    rows, inter = 17, 3072
    gu = rng.standard_normal((rows, 2 * inter), dtype=np.float32)
    t = dev(gu)
    h = torch.empty(rows, inter, device="cuda")
    hip.silu_mul(h, t[:, :inter], t[:, inter:])
    assert max_rel_err(host(h), orc.silu_mul(gu[:, :inter], gu[:, inter:])) <= REL_TOL


def test_silu_and_mul_sigmoid(hip, orc, rng):
    x = rng.normal(0, 4, 100_003).astype(np.float32)
    z = rng.normal(0, 4, 100_003).astype(np.float32)
    xt = dev(x)
    hip.silu(xt)
    assert max_rel_err(host(xt), orc.silu(x)) <= REL_TOL
    yt = dev(x)
    hip.mul_sigmoid(yt, dev(z))
    assert max_rel_err(host(yt), orc.mul_sigmoid(x, z)) <= REL_TOL


@pytest.mark.parametrize("n,offset", [(8192 * 4096, 0), (2048 * 1024, 0), (1, 0), (1023, 0), (4096, 1)])
def test_residual_add(hip, rng, n, offset):
    x = rng.standard_normal(n + offset, dtype=np.float32)
    y = rng.standard_normal(n + offset, dtype=np.float32)
    xt = dev(x)
    hip.residual_add(xt[offset:], dev(y)[offset:])
    got = host(xt)
    assert_bitexact(got[offset:], x[offset:] + y[offset:], "x + y")
    assert np.array_equal(got[:offset], x[:offset])
