"""The engine's expf / log1pf (gateddeltanet_amd/csrc/gdn_libm.h) against the
reference's C library, on the CPU.

The reference's native decode calls glibc's expf and log1pf
(gdn_model.cpp:1307-1330).  The engine restates glibc 2.35's methods (the
Arm Optimized Routines table method for expf in its FMA build, the fdlibm
method for log1pf); the same header code runs in the kernels and, through
gdn_test_libm_array, on the host here.  Checks:
  * the expf table: 2^(i/32) rounded to nearest double (found with exact
    rational arithmetic), minus i << 47, equals the header's 32 entries;
  * both functions equal glibc's (called by the oracle's ORC_LIBM mode) on a
    strided sweep of 2^24 bit patterns plus special values -- and on all
    2^32 patterns with GDN_EXHAUSTIVE=1;
  * the sweep distinguishes them from correctly rounded results (glibc's
    are not correctly rounded everywhere), so the comparison pins the method.
"""
import os
import re
import struct
from fractions import Fraction

import numpy as np
import pytest

from gateddeltanet_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "gateddeltanet_amd", "csrc", "gdn_libm.h")


def engine(which, x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    _lib.load().gdn_test_libm_array(which, x.ctypes.data_as(_lib.FP), out.ctypes.data_as(_lib.FP), x.size)
    return out


def same(a, b):
    return (a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))


def nearest_double_pow2(i):
    """The double nearest to 2^(i/32): x -> x^32 is increasing, so compare
    the neighbours' 32nd powers with 2^i exactly."""
    est = struct.unpack("<Q", struct.pack("<d", 2.0 ** (i / 32)))[0]
    best = None
    for b in range(est - 3, est + 4):
        d = Fraction(struct.unpack("<d", struct.pack("<Q", b))[0])
        lo = Fraction(struct.unpack("<d", struct.pack("<Q", b - 1))[0])
        hi = Fraction(struct.unpack("<d", struct.pack("<Q", b + 1))[0])
        # b is nearest when 2^(i/32) lies between the midpoints with its neighbours
        if ((lo + d) / 2) ** 32 <= 2 ** i <= ((d + hi) / 2) ** 32:
            best = b
    return best


def test_expf_table_is_exact_powers_of_two():
    text = open(HEADER).read()
    body = text[text.index("static constexpr uint64_t T[32]"):]
    entries = [int(v, 16) for v in re.findall(r"0x([0-9a-f]{16})ull", body)[:32]]
    assert len(entries) == 32
    for i in range(32):
        assert entries[i] == nearest_double_pow2(i) - (i << 47), i


def _sweep(stride):
    u = np.arange(0, 1 << 32, stride, dtype=np.uint64).astype(np.uint32)
    special = np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0x00000001, 0x807FFFFF,
                        0x42B17218, 0x42B17217, 0xC2CFF1B5, 0xC2CFF1B4, 0xC2AEAC50, 0x3F800000, 0xBF800000,
                        0x3ED413D6, 0x3ED413D7, 0xBE95F61F, 0xBE95F620, 0x31000000, 0x24800000, 0x5A000000,
                        0x4202422F], np.uint32)
    return np.concatenate([u, special]).view(np.float32)


@pytest.mark.parametrize("which,name", [(0, "exp"), (1, "log1p")])
def test_equals_glibc(orc, which, name):
    x = _sweep(1 << 8)
    got = engine(which, x)
    want = orc.transcendental_array(name, x, orc.LIBM)
    bad = ~same(got, want)
    assert not bad.any(), (name, hex(int(x.view(np.uint32)[bad][0])))
    # glibc is not correctly rounded everywhere, and neither is the engine
    cr = orc.transcendental_array(name, x, orc.CR)
    assert (~same(got, cr)).sum() > 0


@pytest.mark.skipif(os.environ.get("GDN_EXHAUSTIVE") != "1", reason="all 2^32 inputs: GDN_EXHAUSTIVE=1")
@pytest.mark.parametrize("which,name", [(0, "exp"), (1, "log1p")])
def test_equals_glibc_exhaustive(orc, which, name):
    for hi in range(256):
        x = (np.arange(1 << 24, dtype=np.uint32) | np.uint32(hi << 24)).view(np.float32)
        assert same(engine(which, x), orc.transcendental_array(name, x, orc.LIBM)).all(), (name, hi)
