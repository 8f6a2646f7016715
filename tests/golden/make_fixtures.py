"""Writes tests/golden/bf16_rne_cases.json.

Inputs: the 20 FP32 bit patterns of the reference's RNE boundary test
(c_impl/packed_bf16_test.cpp:219-225) and its 20 strategic activations
(:262-268) -- data, not code.  Expected BF16 results are derived here from
the definition of round-to-nearest-even with exact rational arithmetic
(fractions.Fraction), independently of any implementation: the nearest
BF16 value, ties to the even significand, overflow beyond the largest
finite BF16 plus half an ulp to infinity, NaN to the canonical quiet NaN
of its sign (0x7fc0 / 0xffc0), subnormals rounded (not flushed).

Run:  python tests/golden/make_fixtures.py
"""
import json
import os
import struct
from fractions import Fraction

RNE_CASES = [
    0x00000000, 0x80000000, 0x3F800000, 0xBF800000,
    0x3F808000, 0x3F818000, 0xBF808000, 0xBF818000,
    0x3FFFFFFF, 0x7F7FFFFF, 0xFF7FFFFF, 0x00800000,
    0x00000001, 0x007FFFFF, 0x7F800000, 0xFF800000,
    0x7F800001, 0xFF800001, 0x7FC12345, 0xFFC12345,
]
STRATEGIC_ACTIVATIONS = [
    0x00000000, 0x80000000, 0x00000001, 0x007FFFFF,
    0x00800000, 0x00800001, 0x3EFFFFFF, 0x3F000000,
    0x3F7FFFFF, 0x3F800000, 0x3F800001, 0x3FFFFFFF,
    0x40000000, 0x7F7FFFFF, 0xFF7FFFFF, 0x7F800000,
    0xFF800000, 0x7F800001, 0x7FC00000, 0xFFC12345,
]


def f32_value(bits):
    return struct.unpack("<f", struct.pack("<I", bits))[0]


def bf16_value(b16):
    """Exact value of a finite BF16 pattern as a Fraction."""
    sign = -1 if b16 & 0x8000 else 1
    e = (b16 >> 7) & 0xFF
    m = b16 & 0x7F
    if e == 0:
        return sign * Fraction(m, 128) * Fraction(2) ** (-126)
    return sign * (1 + Fraction(m, 128)) * Fraction(2) ** (e - 127)


def rne_bf16_exact(bits):
    e = (bits >> 23) & 0xFF
    frac = bits & 0x7FFFFF
    neg = bool(bits & 0x80000000)
    if e == 0xFF:
        if frac:
            return 0xFFC0 if neg else 0x7FC0
        return 0xFF80 if neg else 0x7F80
    x = abs(Fraction(f32_value(bits)))
    # candidates: all non-negative finite BF16 magnitudes around x
    best = None
    for b in range(0, 0x7F80):
        v = bf16_value(b)
        d = abs(v - x)
        if best is None or d < best[0] or (d == best[0] and (b & 1) == 0 and (best[1] & 1) == 1):
            best = (d, b)
        if v > x:
            break
    max_finite = bf16_value(0x7F7F)
    half_ulp = (bf16_value(0x7F7F) - bf16_value(0x7F7E)) / 2
    if x >= max_finite + half_ulp:
        mag = 0x7F80
    else:
        mag = best[1]
    return mag | (0x8000 if neg else 0)


def main():
    cases = [{"fp32": f"0x{b:08x}", "bf16": f"0x{rne_bf16_exact(b):04x}"} for b in RNE_CASES]
    out = {
        "source": "inputs from c_impl/packed_bf16_test.cpp:219-225 and :262-268; "
                  "expected values from the RNE definition (exact rationals)",
        "rne_cases": cases,
        "strategic_activations": [f"0x{b:08x}" for b in STRATEGIC_ACTIVATIONS],
    }
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "bf16_rne_cases.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    print("wrote", path)


if __name__ == "__main__":
    main()
