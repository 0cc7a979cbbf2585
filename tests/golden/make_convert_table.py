"""Writes bf16_to_f16_table.npy: the reference's bf16 -> fp16 convert
(include/ane_lm/common.h:58-75) for all 65,536 bf16 patterns, derived
independently of any bit manipulation from what the convert computes:
  - the bf16 value is exact in float64;
  - finite values are rounded TOWARD ZERO to fp16 (largest-magnitude fp16
    value not above |x|, found by search in the sorted list of all fp16
    magnitudes), |x| >= 2^16 gives Inf;
  - Inf stays Inf and every NaN becomes Inf of the same sign.
Run: python tests/golden/make_convert_table.py
"""
import os

import numpy as np


def derive() -> np.ndarray:
    pats = np.arange(65536, dtype=np.uint32)
    sign = (pats >> 15).astype(bool)
    with np.errstate(invalid="ignore"):  # signalling NaN patterns
        f32 = (pats << 16).view(np.float32).astype(np.float64)
    mag = np.abs(f32)
    fin16 = np.arange(0x7C00, dtype=np.uint16).view(np.float16).astype(np.float64)  # 0 .. 65504, sorted
    idx = np.searchsorted(fin16, np.where(np.isfinite(mag), mag, 0.0), side="right") - 1
    out = idx.astype(np.uint16)
    out = np.where(mag >= 65536.0, np.uint16(0x7C00), out)   # overflow (incl. Inf)
    out = np.where(np.isnan(f32), np.uint16(0x7C00), out)    # NaN -> Inf
    out = np.where(sign, out | np.uint16(0x8000), out).astype(np.uint16)
    return out


if __name__ == "__main__":
    here = os.path.dirname(os.path.abspath(__file__))
    np.save(os.path.join(here, "bf16_to_f16_table.npy"), derive())
    print("wrote bf16_to_f16_table.npy")
