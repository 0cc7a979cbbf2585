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
