"""Pins the oracle's softmax (core/cpu_ops.cpp:83-99) and sample_token
(core/sampling.cpp:10-66) with exp accuracy bounds, closed forms and the
hand-computed known-answer cases in tests/golden/sampler_kat.json."""
import json
import math
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _ulps(a, b):
    return np.abs(np.asarray(a, np.float32).view(np.int32).astype(np.int64)
                  - np.asarray(b, np.float32).view(np.int32).astype(np.int64))


def test_sampler_exp_within_one_ulp(orc, rng):
    xs = np.concatenate([np.linspace(-104.0, 0.0, 200001), rng.uniform(-104, 0, 100000),
                         rng.uniform(-1, 0, 50000), -np.logspace(-30, 2, 2000)]).astype(np.float32)
    got = np.array([orc.sampler_expf(float(x)) for x in xs], np.float32)
    want = np.exp(xs.astype(np.float64)).astype(np.float32)
    assert int(_ulps(got, want).max()) <= 1


def test_sampler_exp_special_values(orc):
    assert orc.sampler_expf(0.0) == 1.0
    assert orc.sampler_expf(-0.0) == 1.0
    assert orc.sampler_expf(-200.0) == 0.0
    assert orc.sampler_expf(float("-inf")) == 0.0
    assert math.isnan(orc.sampler_expf(float("nan")))
    assert orc.sampler_expf(-103.2789) > 0.0                      # smallest subnormals reached
    assert orc.sampler_expf(100.0) == float("inf")


def test_softmax_uniform_is_exact_reciprocal(orc):
    for n in (1, 3, 4, 1000, 151936):
        p = orc.softmax(np.full(n, -7.25, np.float32))
        assert np.all(p == np.float32(1.0) / np.float32(n))


def test_softmax_two_way_closed_form(orc):
    for d in (0.1, 1.0, 5.0, 17.0):
        p = orc.softmax(np.array([0.0, d], np.float32))
        want = 1.0 / (1.0 + math.exp(-d))
        assert abs(p[1] - want) / want < 3e-7
        assert abs(p[0] - (1 - want)) / (1 - want) < 3e-7


def test_softmax_shift_invariance_and_sum(orc, rng):
    x = rng.normal(0, 3, 151936).astype(np.float32) / np.float32(0.6)
    xq = (np.round(x * 1024) / 1024).astype(np.float32)   # on a 2^-10 grid, so x + 16 is exact
    assert np.array_equal(orc.softmax(xq), orc.softmax(xq + np.float32(16.0)))
    p = orc.softmax(x)
    assert abs(float(np.sum(p.astype(np.float64))) - 1.0) < 1e-5
    xd = x.astype(np.float64)
    ref = np.exp(xd - xd.max())
    ref /= ref.sum()
    big = ref > 1e-30
    assert np.max(np.abs(p[big] - ref[big]) / ref[big]) < 1e-5


def test_softmax_fixed_point_sum_matches_exact(orc, rng):
    """The sum is floor(e*2^shift) summed exactly: within n*2^-shift of the true sum."""
    x = rng.normal(0, 2, 5000).astype(np.float32)
    p = orc.softmax(x)
    shift = orc.softmax_shift(5000)
    assert shift == 63 - 13
    e = np.array([orc.sampler_expf(float(v)) for v in (x - x.max())], np.float64)
    true_sum = e.sum()
    inv = np.float32(1.0) / np.float32(true_sum)
    assert np.max(_ulps(p, e.astype(np.float32) * inv)) <= 1


def _kat_logits(case):
    if case.get("generator") == "dominant_first":
        x = np.zeros(case["n_small"] + 1, np.float32)
        x[0] = case["big"]
        return x
    return np.array(case["logits"], np.float32)


def _kats():
    with open(os.path.join(GOLDEN, "sampler_kat.json")) as f:
        return json.load(f)["cases"]


@pytest.mark.parametrize("case", _kats(), ids=lambda c: c["name"])
def test_sampler_known_answers(orc, case):
    got = orc.sample_token(_kat_logits(case), temperature=case.get("temperature", 0.6),
                           repetition_penalty=case.get("repetition_penalty", 1.2),
                           repetition_context_size=case.get("repetition_context_size", 256),
                           frequency_penalty=case.get("frequency_penalty", 0.1),
                           recent=np.array(case.get("recent", []), np.int32), r=case.get("r", 0.0))
    assert got == case["expect"], case["why"]


def test_sampler_does_not_modify_logits(orc, rng):
    x = rng.normal(0, 3, 1000).astype(np.float32)
    x0 = x.copy()
    orc.sample_token(x, recent=np.arange(50, dtype=np.int32), r=0.3)
    assert np.array_equal(x, x0)


def test_cdf_walk_equals_sequential_float32_cumsum(orc, rng):
    """np.add.accumulate in float32 is the same sequential running sum."""
    for _ in range(20):
        V = int(rng.integers(1, 3000))
        p = orc.softmax((rng.normal(0, 3, V) / 0.6).astype(np.float32))
        cum = np.add.accumulate(p, dtype=np.float32)
        for r in rng.uniform(0, 1, 20).astype(np.float32):
            hit = np.flatnonzero(cum >= r)
            want = int(hit[0]) if hit.size else V - 1
            assert orc.cdf_walk(p, float(r)) == want


def test_absorbed_tail_leaves_cum_below_one(orc, rng):
    x = (rng.normal(0, 3, 151936) / np.float32(0.6)).astype(np.float32)
    p = orc.softmax(x)
    final = np.add.accumulate(p, dtype=np.float32)[-1]
    assert final < 1.0
    assert orc.cdf_walk(p, float(np.nextafter(final, np.float32(2)))) == 151935
