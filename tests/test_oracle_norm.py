"""Pins the oracle's RMSNorm (core/cpu_ops.cpp:25-31), activations
(core/cpu_ops.cpp:7-23) and residual add (models/llm/qwen3.cpp:516) with
closed forms, invariants and fp64 brute force."""
import math

import numpy as np


def test_rmsnorm_constant_row_closed_form(orc):
    # x = c everywhere: ss/dim = c^2, out = c / sqrt(c^2 + eps) * w
    for c, dim in [(0.5, 1024), (3.0, 4096), (-2.0, 128), (1e-3, 2560)]:
        x = np.full(dim, c, np.float32)
        w = np.linspace(0.5, 1.5, dim).astype(np.float32)
        got = orc.rmsnorm(x, w, 1e-6)
        want = c / math.sqrt(c * c + 1e-6) * w.astype(np.float64)
        assert np.max(np.abs(got - want) / np.abs(want)) < 3e-7


def test_rmsnorm_eps_matters(orc):
    # x tiny: without eps the result would be +-1; with eps it is x/sqrt(x^2+eps)
    x = np.full(64, 1e-4, np.float32)
    got = orc.rmsnorm(x, np.ones(64, np.float32), 1e-6)
    want = 1e-4 / math.sqrt(1e-8 + 1e-6)
    assert abs(got[0] - want) / want < 1e-6


def test_rmsnorm_unit_rms_and_scale_invariance(orc, rng):
    x = rng.normal(0, 1, (16, 4096)).astype(np.float32)
    w = np.ones(4096, np.float32)
    y = orc.rmsnorm_rows(x, w, 0.0)
    rms = np.sqrt(np.mean(y.astype(np.float64) ** 2, axis=1))
    assert np.max(np.abs(rms - 1.0)) < 1e-6
    y2 = orc.rmsnorm_rows(x * np.float32(8.0), w, 0.0)   # power-of-two scale: exact invariance
    assert np.array_equal(y, y2)


def test_rmsnorm_fp64_brute_force_tiny(orc, rng):
    for dim in (1, 2, 3, 7, 16):
        x = rng.normal(0, 2, dim).astype(np.float32)
        w = rng.normal(1, 0.1, dim).astype(np.float32)
        got = orc.rmsnorm(x, w, 1e-6)
        xd = x.astype(np.float64)
        want = xd / np.sqrt(np.sum(xd * xd) / dim + 1e-6) * w
        assert np.max(np.abs(got - want) / np.abs(want)) < 5e-7


def test_rmsnorm_rows_equals_single(orc, rng):
    x = rng.normal(0, 1, (5, 1024)).astype(np.float32)
    w = rng.normal(1, 0.02, 1024).astype(np.float32)
    rows = orc.rmsnorm_rows(x, w, 1e-6)
    for i in range(5):
        assert np.array_equal(rows[i], orc.rmsnorm(x[i], w, 1e-6))


def test_silu_closed_forms(orc):
    ln3 = np.float32(math.log(3.0))
    x = np.array([0.0, ln3, 50.0, -120.0, -20.0], np.float32)
    y = orc.silu(x)
    assert y[0] == 0.0
    assert abs(y[1] - 0.75 * float(ln3)) < 1e-7          # sigmoid(ln 3) = 3/4
    assert y[2] == np.float32(50.0)                       # 1 + e^-50 == 1 in fp32
    assert y[3] == 0.0 and np.signbit(y[3])               # exp overflows: x/inf = -0
    assert abs(y[4] - (-20.0 * math.exp(-20) / (1 + math.exp(-20)))) < 1e-12


def test_silu_reflection_identity(orc, rng):
    # silu(-x) = silu(x) - x  (x*s(x) - x = -x*(1 - s(x)) = -x*s(-x))
    x = rng.normal(0, 3, 4096).astype(np.float32)
    a = orc.silu(-x).astype(np.float64)
    b = orc.silu(x).astype(np.float64) - x
    assert np.max(np.abs(a - b)) < 4e-6 * np.max(np.abs(x))


def test_silu_mul_is_silu_times_up(orc, rng):
    g = rng.normal(0, 1, 3072).astype(np.float32)
    u = rng.normal(0, 1, 3072).astype(np.float32)
    h = orc.silu_mul(g, u)
    gd = g.astype(np.float64)
    want = gd / (1 + np.exp(-gd)) * u
    assert np.max(np.abs(h - want) / np.maximum(np.abs(want), 1e-30)) < 3e-7


def test_mul_sigmoid(orc, rng):
    y = rng.normal(0, 1, 1000).astype(np.float32)
    z = rng.normal(0, 2, 1000).astype(np.float32)
    got = orc.mul_sigmoid(y, z)
    want = y.astype(np.float64) / (1 + np.exp(-z.astype(np.float64)))
    assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-30)) < 3e-7


def test_residual_add_is_ieee_add(orc, rng):
    x = rng.normal(0, 1, 10000).astype(np.float32)
    y = rng.normal(0, 1, 10000).astype(np.float32)
    assert np.array_equal(orc.residual_add(x, y), x + y)
