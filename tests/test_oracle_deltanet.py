"""Pins of the oracle's Qwen3.5 linear-attention ops and matvec
(core/cpu_ops.cpp:33-39, :100-171) against closed forms, invariants and
float64 computations written independently of the restatement."""
import numpy as np
import pytest


def test_rmsnorm_gated_zero_gate_gives_zeros(orc, rng):
    x = rng.standard_normal(128).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    out = orc.rmsnorm_gated(x, np.zeros(128, np.float32), w)
    assert np.array_equal(out, np.zeros(128, np.float32))     # out / (1 + 1) * 0


def test_rmsnorm_gated_is_rmsnorm_times_silu(orc, rng):
    for dim in (16, 128, 1000):
        x = rng.standard_normal(dim).astype(np.float32)
        z = (3 * rng.standard_normal(dim)).astype(np.float32)
        w = (1 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
        xd, zd = x.astype(np.float64), z.astype(np.float64)
        ref = xd / np.sqrt(np.mean(xd * xd) + 1e-6) * w * zd / (1 + np.exp(-zd))
        out = orc.rmsnorm_gated(x, z, w)
        assert np.max(np.abs(out - ref) / (np.abs(ref) + 1e-30)) < 4e-6


def test_rmsnorm_gated_constant_row(orc):
    c, dim = np.float32(0.75), 64
    out = orc.rmsnorm_gated(np.full(dim, c), np.full(dim, 2.0, np.float32), np.ones(dim, np.float32))
    want = c / np.sqrt(c * c + 1e-6) * 2.0 / (1 + np.exp(-2.0))
    assert np.allclose(out, want, rtol=2e-7)


def test_l2_normalize(orc, rng):
    x = rng.standard_normal(128).astype(np.float32)
    y = orc.l2_normalize(x)
    assert abs(np.linalg.norm(y.astype(np.float64)) - 1) < 1e-6
    assert np.allclose(y, x / np.linalg.norm(x.astype(np.float64)), rtol=1e-6)
    assert np.array_equal(orc.l2_normalize(x * np.float32(8)), y)   # exact power-of-two invariance
    assert np.array_equal(orc.l2_normalize(np.zeros(32, np.float32)), np.zeros(32, np.float32))
    c = orc.l2_normalize(np.full(16, 3.0, np.float32))
    assert np.allclose(c, 0.25, rtol=1e-7)                          # 3 / sqrt(16 * 9)


@pytest.mark.parametrize("K", [4, 3, 6])
def test_conv1d_matches_direct_convolution(orc, rng, K):
    """Feeding inputs x_0, x_1, ... through the state ring gives
    y_t = sum_j w_j x_{t-(K-1)+j} with zeros before t = 0."""
    ch, steps = 37, 11
    w = rng.standard_normal((ch, K)).astype(np.float32)
    xs = rng.standard_normal((steps, ch)).astype(np.float32)
    state = np.zeros((ch, K - 1), np.float32)
    pos = np.zeros(1, np.int32)
    hist = np.zeros((K - 1 + steps, ch))
    hist[K - 1:] = xs
    for t in range(steps):
        y = orc.conv1d_update(state, pos, xs[t], w)
        ref = sum(w[:, j].astype(np.float64) * hist[t + j] for j in range(K))
        assert np.allclose(y, ref, rtol=1e-5, atol=1e-6)
        assert pos[0] == (t + 1) % (K - 1)


def test_ssm_step_brute_force(orc, rng):
    kd, vd = 128, 128
    S = rng.standard_normal((kd, vd)).astype(np.float32) * 0.1
    q, k, v = (rng.standard_normal(kd).astype(np.float32), rng.standard_normal(kd).astype(np.float32),
               rng.standard_normal(vd).astype(np.float32))
    decay, beta = np.float32(0.93), np.float32(0.4)
    Sd = S.astype(np.float64)
    delta = v - Sd.T @ k
    Sn = decay * Sd + beta * np.outer(k, delta)
    yref = Sn.T @ q
    y = orc.ssm_step(S, q, k, v, decay, beta)
    assert np.max(np.abs(S - Sn) / (np.abs(decay * Sd) + np.abs(beta * np.outer(k, delta)) + 1e-30)) < 2e-6
    assert np.max(np.abs(y - yref) / (np.abs(Sn.T) @ np.abs(q) + 1e-30)) < 2e-6


def test_ssm_step_identities(orc, rng):
    kd, vd = 64, 128
    S = rng.standard_normal((kd, vd)).astype(np.float32)
    S0 = S.copy()
    q = rng.standard_normal(kd).astype(np.float32)
    y = orc.ssm_step(S, q, rng.standard_normal(kd).astype(np.float32), rng.standard_normal(vd).astype(np.float32),
                     1.0, 0.0)
    assert np.array_equal(S, S0)                                  # decay 1, beta 0: unchanged
    assert np.allclose(y, S0.T.astype(np.float64) @ q, rtol=1e-5, atol=1e-5)
    k = rng.standard_normal(kd)
    k = (k / np.linalg.norm(k)).astype(np.float32)
    v = rng.standard_normal(vd).astype(np.float32)
    orc.ssm_step(S, q, k, v, 1.0, 1.0)                            # delta rule stores v at key k
    assert np.allclose(S.T.astype(np.float64) @ k, v, atol=1e-4)


def test_matvec(orc, rng):
    x = rng.standard_normal(300).astype(np.float32)
    assert np.array_equal(orc.matvec(np.eye(300, dtype=np.float32), x), x)
    W = rng.standard_normal((77, 300)).astype(np.float32)
    ref = W.astype(np.float64) @ x
    assert np.max(np.abs(orc.matvec(W, x) - ref) / (np.abs(W) @ np.abs(x))) < 1e-7
