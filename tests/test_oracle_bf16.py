"""Pins of the oracle's BF16 primitives (gdn_model.cpp:309-325, :392-467).

* RNE: the 20 boundary cases of the reference's own unit test
  (packed_bf16_test.cpp:219-225) with expected values derived from the RNE
  definition in exact arithmetic (tests/golden/make_fixtures.py), and a sweep
  against torch's FP32->BF16 conversion (round-to-nearest-even; NaN patterns
  checked separately because torch drops the sign): every upper half (sign,
  exponent, 7 kept mantissa bits) with 40 lower halves covering every
  rounding class (exact, below/at/above the tie, the carry), or all 2^32
  patterns with GDN_EXHAUSTIVE=1.
* Widen: exhaustive over all 65,536 BF16 patterns.
* Native product: an independent model written from the rule text of the
  reference (architecture.md:867-878: "round to nearest-even first, then
  flush only if the rounded BF16 exponent is still zero"), evaluated with
  float64 arithmetic on the unbounded-exponent exact product, over every
  weight pattern x 64 structured activations plus 2^20 random pairs, and the
  special-value classes.
"""
import json
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "bf16_rne_cases.json")


def test_rne_golden_cases(orc):
    cases = json.load(open(GOLDEN))["rne_cases"]
    assert len(cases) == 20
    for c in cases:
        got = orc.lib().orc_rne_bits(int(c["fp32"], 16))
        assert got == int(c["bf16"], 16), c


def _rne_sweep_chunks():
    if os.environ.get("GDN_EXHAUSTIVE") == "1":
        chunk = 1 << 26
        for start in range(0, 1 << 32, chunk):
            yield np.arange(start, start + chunk, dtype=np.uint64).astype(np.uint32)
        return
    rng = np.random.default_rng(1)
    lows = np.unique(np.concatenate([
        np.array([0x0000, 0x0001, 0x3FFF, 0x7FFE, 0x7FFF, 0x8000, 0x8001, 0xBFFF, 0xC000, 0xFFFE, 0xFFFF],
                 np.uint32),
        rng.integers(0, 1 << 16, 29, dtype=np.uint32)]))
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    yield (hi[:, None] | lows[None, :]).reshape(-1)


def test_rne_against_torch(orc):
    torch = pytest.importorskip("torch")
    for bits in _rne_sweep_chunks():
        ours = orc.rne_array(bits)
        f = bits.view(np.float32)
        nan = np.isnan(f)
        ref = torch.from_numpy(f.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        ok = (ours == ref) | nan
        assert ok.all(), hex(int(bits[~ok][0]))
        neg = (bits & 0x80000000) != 0
        want_nan = np.where(neg, 0xFFC0, 0x7FC0).astype(np.uint16)
        assert (ours[nan] == want_nan[nan]).all()


def test_widen_exhaustive(orc):
    for b in range(0, 1 << 16, 4099):
        assert orc.lib().orc_widen_bits(b) == b << 16
    b = np.arange(1 << 16, dtype=np.uint32)
    # widening through the product path: w * 1.0 keeps every normal value
    one = np.full(b.size, 0x3F80, np.uint16)
    prod = orc.native_product_array(b.astype(np.uint16), one)
    e = (b >> 7) & 0xFF
    normal = (e != 0) & (e != 0xFF)
    assert (prod[normal] == b[normal]).all()


def text_model(w, x):
    """Independent native-product model from the rule text, vectorised."""
    w = w.astype(np.uint32)
    x = x.astype(np.uint32)
    ew, fw = (w >> 7) & 0xFF, w & 0x7F
    ex, fx = (x >> 7) & 0xFF, x & 0x7F
    sign = ((w ^ x) & 0x8000).astype(np.uint32)
    w_nan, x_nan = (ew == 0xFF) & (fw != 0), (ex == 0xFF) & (fx != 0)
    w_inf, x_inf = (ew == 0xFF) & (fw == 0), (ex == 0xFF) & (fx == 0)
    w_zero, x_zero = ew == 0, ex == 0  # DAZ
    # exact product of the two significands and exponents (float64 exact)
    mw = (128 + fw).astype(np.float64)
    mx = (128 + fx).astype(np.float64)
    prod = mw * mx  # in [2^14, 2^16): exact integer
    e2 = ew.astype(np.int64) + ex.astype(np.int64) - 254 - 14
    # normalise to an 8-bit significand in [128, 256) with unbounded exponent
    big = prod >= 32768
    shift = np.where(big, 8, 7)
    sig = prod / np.exp2(shift)  # in [128, 256), exact multiple of 2^-8
    exp_ = e2 + shift
    fl = np.floor(sig)
    rem = sig - fl
    up = (rem > 0.5) | ((rem == 0.5) & (np.mod(fl, 2) == 1))
    sig_r = fl + up
    carry = sig_r == 256
    sig_r = np.where(carry, 128, sig_r)
    exp_ = exp_ + carry
    # value = sig_r * 2^exp_ ; biased BF16 exponent = exp_ + 7 + 127
    be = exp_ + 7 + 127
    out = np.where(be <= 0, sign,  # flush: rounded exponent still zero (or below)
                   np.where(be >= 0xFF, sign | 0x7F80,
                            sign | (be.clip(0, 0xFE).astype(np.uint32) << 7) | (sig_r.astype(np.uint32) - 128)))
    out = np.where(w_zero | x_zero, sign, out)
    out = np.where(w_inf | x_inf, sign | 0x7F80, out)
    out = np.where(w_nan | x_nan | (w_inf & x_zero) | (x_inf & w_zero), 0x7FC0, out)
    return out.astype(np.uint16)


def _structured_activations():
    acts = []
    for e in list(range(0, 256, 5)) + [0, 1, 2, 125, 126, 127, 128, 129, 253, 254, 255]:
        for f in (0, 1, 0x3F, 0x40, 0x7F):
            for s in (0, 0x8000):
                acts.append(s | (e << 7) | f)
    return np.unique(np.array(acts, np.uint16))[:64]


def test_native_product_all_weights(orc):
    w = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    for a in _structured_activations():
        x = np.full(w.size, a, np.uint16)
        ours = orc.native_product_array(w, x)
        ref = text_model(w, x)
        bad = ours != ref
        assert not bad.any(), (hex(int(a)), hex(int(w[bad][0])), hex(int(ours[bad][0])), hex(int(ref[bad][0])))


def test_native_product_random_pairs(orc):
    rng = np.random.default_rng(20260827)
    w = rng.integers(0, 1 << 16, 1 << 20, dtype=np.uint32).astype(np.uint16)
    x = rng.integers(0, 1 << 16, 1 << 20, dtype=np.uint32).astype(np.uint16)
    assert (orc.native_product_array(w, x) == text_model(w, x)).all()


def test_native_product_select_form(orc):
    """The branch-free form the GEMV rows use (integer selects, special cases
    applied last) equals the pinned scalar form: every weight against the
    structured activations, plus 2^22 random pairs; all 2^32 pairs with
    GDN_EXHAUSTIVE=1."""
    w = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    for a in _structured_activations():
        x = np.full(w.size, a, np.uint16)
        assert (orc.native_product_sel_array(w, x) == orc.native_product_array(w, x)).all(), hex(int(a))
    rng = np.random.default_rng(7)
    w = rng.integers(0, 1 << 16, 1 << 22, dtype=np.uint32).astype(np.uint16)
    x = rng.integers(0, 1 << 16, 1 << 22, dtype=np.uint32).astype(np.uint16)
    assert (orc.native_product_sel_array(w, x) == orc.native_product_array(w, x)).all()
    if os.environ.get("GDN_EXHAUSTIVE") == "1":
        w = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
        for a in range(1 << 16):
            x = np.full(w.size, a, np.uint16)
            assert (orc.native_product_sel_array(w, x) == orc.native_product_array(w, x)).all(), hex(a)


def test_native_product_flush_boundary(orc):
    """146/128 * 224/128 = 2 - 2^-8: with exponents summing to -127 the exact
    product is 0x007fc000 = 2^-126 - 2^-135, a tie that rounds up into the
    smallest normal BF16.  145 * 225 lies just below and flushes to zero."""
    P = lambda w, x: int(orc.native_product_array(np.array([w], np.uint16), np.array([x], np.uint16))[0])
    w = (67 << 7) | (146 - 128)   # 1.140625 * 2^-60
    x = (60 << 7) | (224 - 128)   # 1.75 * 2^-67
    assert P(w, x) == 0x0080
    assert P(w | 0x8000, x) == 0x8080
    w2 = (67 << 7) | (145 - 128)
    x2 = (60 << 7) | (225 - 128)
    assert P(w2, x2) == 0x0000
    assert P(w2, x2 | 0x8000) == 0x8000   # flushed products keep their sign


def test_native_product_specials(orc):
    P = lambda w, x: int(orc.native_product_array(np.array([w], np.uint16), np.array([x], np.uint16))[0])
    assert P(0x7FC0, 0x3F80) == 0x7FC0          # NaN operand
    assert P(0x7F80, 0x0000) == 0x7FC0          # inf * 0
    assert P(0x7F80, 0x0001) == 0x7FC0          # inf * subnormal (DAZ zero)
    assert P(0xFF80, 0x3F80) == 0xFF80          # -inf * 1
    assert P(0x7F80, 0xBF80) == 0xFF80          # inf * -1
    assert P(0x0001, 0x7F00) == 0x0000          # subnormal weight is zero
    assert P(0x8000, 0x3F80) == 0x8000          # -0 * 1
    assert P(0x7F7F, 0x7F7F) == 0x7F80          # overflow to inf
    assert P(0x3F80, 0x3F80) == 0x3F80          # 1 * 1
    assert P(0x3F81, 0x3F81) == 0x3F82          # (1+2^-7)^2 = 1 + 2^-6 + 2^-14 -> RNE 0x3f82


def test_transcendental_modes_agree(orc):
    """The CR mode (what the HIP kernels evaluate) and glibc agree except on
    rare last-bit cases: exp differs by at most one ULP, the functions built
    on it (one more rounded operation) by at most two."""
    x = np.linspace(-30, 30, 200001, dtype=np.float32)
    for which in ("exp", "sigmoid", "silu", "softplus"):
        a = orc.transcendental_array(which, x, orc.LIBM)
        b = orc.transcendental_array(which, x, orc.CR)
        diff = a.view(np.int32).astype(np.int64) - b.view(np.int32).astype(np.int64)
        assert np.abs(diff).max() <= (1 if which == "exp" else 2), which
        assert (diff != 0).mean() < 1e-2, which
