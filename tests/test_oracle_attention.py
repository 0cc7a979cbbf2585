"""Pins of the oracle's KV ring (models/llm/qwen3.cpp:475-488) and GQA decode
attention (core/cpu_ops.cpp:173-240) against checks that do not restate it:
a list model of the ring, exact closed forms, a float64 brute force that
enumerates ring positions independently, and the ring-rotation identity."""
import numpy as np
import pytest

from helpers import attention_fp64 as brute_force


def test_ring_matches_list_model(orc, rng):
    cap, nk, D = 5, 2, 3
    kc = np.zeros((cap, nk * D), np.float32)
    vc = np.zeros_like(kc)
    st = np.zeros(2, np.int32)
    hist = []
    for i in range(13):
        row = rng.standard_normal(nk * D).astype(np.float32)
        slot = orc.kv_ring_append(kc, vc, row, -row, st)
        hist.append(row)
        assert slot == i % cap
        n = len(hist)
        assert st[1] == min(n, cap) and st[0] == (max(0, n - cap)) % cap
        live = hist[-cap:]
        for t, want in enumerate(live):         # logical order = append order of the live rows
            s = (st[0] + t) % cap
            assert np.array_equal(kc[s], want) and np.array_equal(vc[s], -want)


@pytest.mark.parametrize("length", [0, -3])
def test_empty_cache_gives_zeros(orc, rng, length):
    kc = rng.standard_normal((16, 2 * 8)).astype(np.float32)
    out = orc.gqa_attention(rng.standard_normal(4 * 8).astype(np.float32), kc, kc, 4, 2, 8, 3, length)
    assert np.array_equal(out, np.zeros((4, 8), np.float32))


def test_single_position_returns_v_exactly(orc, rng):
    nq, nk, D, cap = 8, 2, 16, 10
    kc = rng.standard_normal((cap, nk * D)).astype(np.float32)
    vc = rng.standard_normal((cap, nk * D)).astype(np.float32)
    out = orc.gqa_attention(rng.standard_normal(nq * D).astype(np.float32), kc, vc, nq, nk, D, 7, 1)
    for h in range(nq):
        assert np.array_equal(out[h], vc[7].reshape(nk, D)[h // 4])


def test_uniform_keys_average_values_exactly(orc, rng):
    """Equal keys: every score ties, p = 1/8 exactly, and small-integer values
    make each product and partial sum exact, so out is the exact mean."""
    nq, nk, D, cap, length = 4, 2, 8, 12, 8
    kc = np.tile(rng.standard_normal(nk * D).astype(np.float32), (cap, 1))
    vc = rng.integers(-64, 64, (cap, nk * D)).astype(np.float32)
    start = 9                                                     # wraps after 3 rows
    out = orc.gqa_attention(rng.standard_normal(nq * D).astype(np.float32), kc, vc, nq, nk, D, start, length)
    slots = (start + np.arange(length)) % cap
    mean = vc[slots].reshape(length, nk, D).astype(np.float64).mean(0)
    for h in range(nq):
        assert np.array_equal(out[h].astype(np.float64), mean[h // 2])


def test_dominant_key_selects_its_value(orc, rng):
    nq, nk, D, cap = 2, 1, 32, 64
    q = np.zeros(nq * D, np.float32)
    q[:D] = 1.0
    q[D:] = 1.0
    kc = (0.01 * rng.standard_normal((cap, D))).astype(np.float32)
    kc[40] = 40.0                                                 # score 40*32/sqrt(32) ~ 226
    vc = rng.standard_normal((cap, D)).astype(np.float32)
    out = orc.gqa_attention(q, kc, vc, nq, nk, D, 20, 30)
    assert np.array_equal(out[0], vc[40]) and np.array_equal(out[1], vc[40])


@pytest.mark.parametrize("nq,nk,D,cap,start,length,qs", [
    (4, 4, 16, 32, 0, 32, None), (8, 2, 32, 50, 37, 41, None), (16, 8, 128, 64, 63, 64, None),
    (32, 8, 128, 300, 290, 177, 256), (6, 3, 64, 20, 5, 9, 80)])
def test_brute_force_float64(orc, rng, nq, nk, D, cap, start, length, qs):
    qsz = (nq - 1) * (qs or D) + D
    q = rng.standard_normal(qsz).astype(np.float32)
    kc = rng.standard_normal((cap, nk * D)).astype(np.float32)
    vc = rng.standard_normal((cap, nk * D)).astype(np.float32)
    out = orc.gqa_attention(q, kc, vc, nq, nk, D, start, length, q_head_stride=qs)
    ref, bound = brute_force(q, kc, vc, nq, nk, D, start, length, qs)
    assert np.max(np.abs(out - ref) / (bound + 1e-30)) < 2e-6


def test_ring_rotation_is_bit_identical(orc, rng):
    """The same logical rows stored from a different start give the same bits."""
    nq, nk, D, cap, length = 8, 4, 32, 40, 33
    q = rng.standard_normal(nq * D).astype(np.float32)
    kc = rng.standard_normal((cap, nk * D)).astype(np.float32)
    vc = rng.standard_normal((cap, nk * D)).astype(np.float32)
    base = orc.gqa_attention(q, kc, vc, nq, nk, D, 0, length)
    for s in (1, 7, 39):
        rolled = orc.gqa_attention(q, np.roll(kc, s, 0), np.roll(vc, s, 0), nq, nk, D, s, length)
        assert np.array_equal(base, rolled)


def test_gqa_head_mapping(orc, rng):
    """kv heads with disjoint value supports: head h must read kv head h // groups."""
    nq, nk, D, cap = 8, 4, 8, 6
    kc = rng.standard_normal((cap, nk * D)).astype(np.float32)
    vc = np.zeros((cap, nk, D), np.float32)
    for j in range(nk):
        vc[:, j, :] = j + 1                                       # constant per kv head
    out = orc.gqa_attention(rng.standard_normal(nq * D).astype(np.float32), kc, vc.reshape(cap, -1), nq, nk, D, 2, 5)
    for h in range(nq):
        assert np.allclose(out[h], h // 2 + 1, rtol=1e-6)
