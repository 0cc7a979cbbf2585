"""Pins the oracle's RoPE table (models/llm/qwen3.cpp:200-219), Qwen3
rotation (qwen3.cpp:17-52), qk-norm order (qwen3.cpp:444-472) and
apply_rope_cached (core/cpu_ops.cpp:56-80)."""
import math

import numpy as np

THETA = 1e6
D = 128
HALF = 64


def test_inv_freq_closed_forms(orc):
    inv = orc.rope_inv_freq(D, THETA)
    assert inv[0] == 1.0                                            # theta^0
    assert abs(inv[32] - 1e-3) / 1e-3 < 2e-7                        # theta^(-64/128) = 1e6^-0.5
    ratio = inv[1:].astype(np.float64) / inv[:-1]
    assert np.max(np.abs(ratio - THETA ** (-2.0 / D))) < 1e-6       # geometric progression


def test_table_row0_identity_and_fp64(orc):
    c, s = orc.rope_table(4096, D, THETA)
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)
    inv = orc.rope_inv_freq(D, THETA).astype(np.float64)
    pos = np.arange(4096, dtype=np.float64)[:, None]
    ang = (pos.astype(np.float32) * inv.astype(np.float32)).astype(np.float64)  # fp32 angle, as the reference
    assert np.max(np.abs(c - np.cos(ang))) < 2.0 ** -23
    assert np.max(np.abs(s - np.sin(ang))) < 2.0 ** -23


def _qk(rng, T, nq, nk):
    return (rng.normal(0, 1, (T, nq * D)).astype(np.float32), rng.normal(0, 1, (T, nk * D)).astype(np.float32))


def test_pos0_is_identity(orc, rng):
    q, k = _qk(rng, 1, 4, 2)
    c, s = orc.rope_table(8, D, THETA)
    q2, k2 = orc.qknorm_rope(q, k, None, None, np.array([0], np.int32), c, s, THETA, 4, 2, D)
    assert np.array_equal(q2, q) and np.array_equal(k2, k)


def test_half_split_is_complex_multiply(orc, rng):
    """(v[j], v[j+64]) rotated by angle a_j is z_j * exp(i a_j) with z_j = v[j] + i v[j+64]."""
    T, nq, nk = 6, 4, 2
    q, k = _qk(rng, T, nq, nk)
    pos = np.array([1, 7, 100, 2047, 4095, 12345], np.int32)
    c, s = orc.rope_table(16384, D, THETA)
    q2, _ = orc.qknorm_rope(q, k, None, None, pos, c, s, THETA, nq, nk, D)
    inv = orc.rope_inv_freq(D, THETA)
    for t in range(T):
        ang = (np.float32(pos[t]) * inv).astype(np.float64)
        for h in range(nq):
            v = q[t, h * D:(h + 1) * D].astype(np.float64)
            z = (v[:HALF] + 1j * v[HALF:]) * np.exp(1j * ang)
            got = q2[t, h * D:(h + 1) * D]
            den = np.abs(v[:HALF] * np.cos(ang)) + np.abs(v[HALF:] * np.sin(ang)) + 1e-30
            assert np.max(np.abs(got[:HALF] - z.real) / den) < 4e-7
            den2 = np.abs(v[HALF:] * np.cos(ang)) + np.abs(v[:HALF] * np.sin(ang)) + 1e-30
            assert np.max(np.abs(got[HALF:] - z.imag) / den2) < 4e-7


def test_rotation_preserves_pair_norms_and_adds_angles(orc, rng):
    q, k = _qk(rng, 1, 1, 1)
    c, s = orc.rope_table(64, D, THETA)
    a, _ = orc.qknorm_rope(q, k, None, None, np.array([5], np.int32), c, s, THETA, 1, 1, D)
    b, _ = orc.qknorm_rope(a, k, None, None, np.array([9], np.int32), c, s, THETA, 1, 1, D)
    d, _ = orc.qknorm_rope(q, k, None, None, np.array([14], np.int32), c, s, THETA, 1, 1, D)
    n0 = q[0, :HALF].astype(np.float64) ** 2 + q[0, HALF:].astype(np.float64) ** 2
    n1 = a[0, :HALF].astype(np.float64) ** 2 + a[0, HALF:].astype(np.float64) ** 2
    assert np.max(np.abs(n1 - n0) / n0) < 1e-6
    assert np.max(np.abs(b - d)) < 1e-5 * np.max(np.abs(q))     # rot(9)∘rot(5) = rot(14)


def test_fallback_equals_table(orc, rng):
    """Positions past the table use the on-the-fly formula, which is the
    table formula (qwen3.cpp:41-44 vs :208, :214-216): same floats."""
    q, k = _qk(rng, 4, 3, 2)
    pos = np.array([0, 17, 3000, 16383], np.int32)
    c, s = orc.rope_table(16384, D, THETA)
    a = orc.qknorm_rope(q, k, None, None, pos, c, s, THETA, 3, 2, D)
    b = orc.qknorm_rope(q, k, None, None, pos, None, None, THETA, 3, 2, D)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def test_qk_norm_runs_before_rope(orc, rng):
    """Norm then rotate: the per-pair norms after the op are those of the
    normalised (not the raw) head."""
    q, k = _qk(rng, 1, 1, 1)
    q *= 5.0
    w = np.ones(D, np.float32)
    c, s = orc.rope_table(64, D, THETA)
    a, _ = orc.qknorm_rope(q, k, w, w, np.array([33], np.int32), c, s, THETA, 1, 1, D)
    qn = orc.rmsnorm(q[0], w, 1e-6)
    pn = qn[:HALF].astype(np.float64) ** 2 + qn[HALF:].astype(np.float64) ** 2
    pa = a[0, :HALF].astype(np.float64) ** 2 + a[0, HALF:].astype(np.float64) ** 2
    assert np.max(np.abs(pa - pn) / pn) < 1e-6


def test_rope_cached_table_path_is_half_split(orc, rng):
    q = rng.normal(0, 1, 2 * D * 2).astype(np.float32)   # 2 heads at stride 2*D (q|gate layout)
    k = rng.normal(0, 1, D).astype(np.float32)
    c, s = orc.rope_table(64, D, THETA)
    q2, k2 = orc.rope_cached(q, k, 2, 1, D, 2 * D, D, D, 10, THETA, c[10], s[10])
    qq, kk = orc.qknorm_rope(q.reshape(2, 2 * D)[:, :D].reshape(1, -1), k.reshape(1, -1), None, None,
                             np.array([10], np.int32), c, s, THETA, 2, 1, D)
    assert np.array_equal(q2.reshape(2, 2 * D)[:, :D].reshape(-1), qq.reshape(-1))
    assert np.array_equal(q2.reshape(2, 2 * D)[:, D:], q.reshape(2, 2 * D)[:, D:])   # gate untouched
    assert np.array_equal(k2, kk.reshape(-1))


def test_rope_cached_fallback_is_adjacent_pairs(orc, rng):
    """Without a row the reference rotates (v[2i], v[2i+1]) (cpu_ops.cpp:68-77)."""
    rot = 64
    q = rng.normal(0, 1, D).astype(np.float32)
    k = rng.normal(0, 1, D).astype(np.float32)
    q2, _ = orc.rope_cached(q, k, 1, 1, D, D, D, rot, 3, THETA)
    inv = orc.rope_inv_freq(rot, THETA)
    ang = (np.float32(3) * inv).astype(np.float64)
    z = (q[0:rot:2].astype(np.float64) + 1j * q[1:rot:2]) * np.exp(1j * ang)
    assert np.max(np.abs(q2[0:rot:2] - z.real)) < 1e-6
    assert np.max(np.abs(q2[1:rot:2] - z.imag)) < 1e-6
    assert np.array_equal(q2[rot:], q[rot:])                          # partial rotary: tail untouched
