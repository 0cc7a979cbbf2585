"""Pins the oracle's conversions (include/ane_lm/common.h:21-83) against
derivations that do not share its bit manipulation."""
import os

import numpy as np

from helpers import assert_bitexact

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _derived_table():
    import importlib.util

    spec = importlib.util.spec_from_file_location("mct", os.path.join(GOLDEN, "make_convert_table.py"))
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m.derive()


def test_bf16_to_f16_exhaustive_matches_round_toward_zero(orc):
    pats = np.arange(65536, dtype=np.uint16)
    got = orc.bf16_to_f16(pats)
    assert_bitexact(got, _derived_table(), "bf16->f16 vs exact-real RTZ")


def test_bf16_to_f16_matches_committed_table(orc):
    ref = np.load(os.path.join(GOLDEN, "bf16_to_f16_table.npy"))
    assert_bitexact(orc.bf16_to_f16(np.arange(65536, dtype=np.uint16)), ref, "committed table")


def test_bf16_to_f16_known_patterns(orc):
    # (bf16 bits, fp16 bits): 1.0, -2.0, max bf16 finite -> Inf, Inf, NaN -> Inf,
    # -NaN -> -Inf, 2^-14 (smallest normal fp16), 2^-24 (smallest subnormal),
    # 2^-25 -> 0 (truncation), 1.5*2^-24 -> 2^-24 (truncation, RNE would give 2*2^-24)
    cases = [(0x3F80, 0x3C00), (0xC000, 0xC000), (0x7F7F, 0x7C00), (0x7F80, 0x7C00), (0x7FC1, 0x7C00),
             (0xFF81, 0xFC00), (0x3880, 0x0400), (0x3380, 0x0001), (0x3300, 0x0000), (0x33C0, 0x0001),
             (0x8000, 0x8000), (0x0001, 0x0000), (0x477F, 0x7BF8)]
    src = np.array([c[0] for c in cases], np.uint16)
    want = np.array([c[1] for c in cases], np.uint16)
    assert_bitexact(orc.bf16_to_f16(src), want, "known patterns")


def test_truncation_differs_from_rne_only_where_expected(orc):
    """RNE and the reference's truncation differ on 1,278 patterns: 1,024
    subnormal-range values and 254 NaNs (NaN -> Inf)."""
    pats = np.arange(65536, dtype=np.uint16)
    trunc = orc.bf16_to_f16(pats)
    with np.errstate(invalid="ignore", over="ignore"):
        rne = (pats.astype(np.uint32) << 16).view(np.float32).astype(np.float16).view(np.uint16)
    diff = trunc != rne
    vals = (pats.astype(np.uint32) << 16).view(np.float32)
    nan = np.isnan(vals)
    assert int(diff.sum()) == 1278
    assert int((diff & nan).sum()) == 254
    mags = np.abs(vals[diff & ~nan])
    assert mags.min() >= 2.0 ** -25 and mags.max() < 2.0 ** -14


def test_f16_to_f32_exhaustive(orc):
    pats = np.arange(65536, dtype=np.uint16)
    got = orc.f16_to_f32(pats)
    h = pats.view(np.float16)
    finite = ~np.isnan(h)
    # finite values (incl. subnormals and Inf) widen exactly
    assert_bitexact(got[finite], h[finite].astype(np.float32), "f16->f32 finite")
    # NaN: same sign, mantissa bits preserved exactly (no quieting)
    gb = got.view(np.uint32)[~finite]
    pb = pats[~finite].astype(np.uint32)
    assert np.all(np.isnan(got[~finite]))
    assert np.all((gb >> 31) == (pb >> 15))
    assert np.all(((gb >> 13) & 0x3FF) == (pb & 0x3FF))
    assert np.all((gb & 0x1FFF) == 0)


def test_bf16_to_f32_is_high_half(orc):
    pats = np.arange(65536, dtype=np.uint16)
    got = orc.bf16_to_f32(pats).view(np.uint32)
    assert np.array_equal(got, pats.astype(np.uint32) << 16)


def _rne_f32(x):
    """Exact rational x rounded to nearest-even fp32 (normal range), derived
    from the definition: scale to a 24-bit significand, round half to even."""
    from fractions import Fraction

    if x == 0:
        return 0.0
    sign = -1 if x < 0 else 1
    a = abs(x)
    k = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** k > a:
        k -= 1
    m = a / Fraction(2) ** (k - 23)          # in [2^23, 2^24)
    q, r = divmod(m.numerator, m.denominator)
    twice = 2 * r
    if twice > m.denominator or (twice == m.denominator and q & 1):
        q += 1
    return sign * float(Fraction(q) * Fraction(2) ** (k - 23))


def test_norm_weight_exhaustive_against_exact_rounding(orc):
    """core/safetensors.cpp:299-306: w + 1.0f for every bf16 w, checked
    against the exact sum rounded to nearest even (ties included: w = 2^-24
    rounds to 1, w = 3*2^-25 to 1 + 2^-23)."""
    from fractions import Fraction

    pats = np.arange(65536, dtype=np.uint16)
    got = orc.norm_weight(pats)
    w = orc.bf16_to_f32(pats)
    want = np.empty(65536, np.float32)
    for i in range(65536):
        wi = float(w[i])
        if not np.isfinite(wi):
            want[i] = wi
            continue
        want[i] = _rne_f32(Fraction(wi) + 1)
    fin = np.isfinite(w)
    assert_bitexact(got[fin], want[fin], "norm weight")
    assert np.array_equal(got[np.isinf(w)], w[np.isinf(w)])
    nan = np.isnan(w)                                  # quieted, sign and payload kept (IEEE 754 6.2.3)
    assert np.array_equal(got[nan].view(np.uint32), w[nan].view(np.uint32) | 0x00400000)
    one = lambda bits: float(orc.norm_weight(np.array([bits], np.uint16))[0])
    assert one(0x3380) == 1.0                          # 2^-24: tie, stays at 1 (even)
    assert one(0x33C0) == 1.0 + 2.0 ** -23             # 1.5 * 2^-24: above the tie
    assert one(0xBF80) == 0.0                          # -1 + 1
    assert one(0x8000) == 1.0                          # -0 + 1


def test_norm_weight_count_bounds_the_offset(orc):
    """The reference adds 1 for i < expected_numel only: a non-positive count
    widens only (core/safetensors.cpp:302-303)."""
    bits = np.array([0x3F80, 0x4000, 0xC000], np.uint16)
    assert np.array_equal(orc.norm_weight(bits, 0), orc.bf16_to_f32(bits))
    assert np.array_equal(orc.norm_weight(bits, 2), np.array([2.0, 3.0, -2.0], np.float32))
