// gdn_libm.h -- expf and log1pf evaluated exactly as the reference's C
// library computes them, for device and host code of libgdn_amd.so.
//
// The reference's native decode (gdn_model.cpp:1307-1330) calls glibc's
// expf and log1pf; the rounding of every later operator makes a last-bit
// difference in them grow over a long decode.  These two functions restate
// glibc 2.35's methods so that the engine reproduces them bit for bit:
//
//   gdn_expf    the table-driven method of Arm Optimized Routines (Szabolcs
//               Nagy, 2017), glibc's expf since 2.27: x * 32/ln2 = k + r
//               with k rounded to an integer through the 1.5 * 2^52 shift,
//               2^(k/32) from a 32-entry table of 2^(i/32) whose exponent
//               field is pre-biased by -i << 47, and 2^(r/32) from a cubic
//               polynomial, all in double, then rounded once to float.  The
//               table entries are 2^(i/32) rounded to nearest double
//               (derivable exactly; see tests/test_libm.py); the products
//               fused with additions as the FMA build of that routine does
//               (the code glibc dispatches to on x86-64 with FMA).
//   gdn_log1pf  the fdlibm method (Sun Microsystems, 1993) of glibc's
//               s_log1pf.c: 1 + x = 2^k (1 + f), log(1 + f) = f - hfsq +
//               s (hfsq + R(s^2)) with s = f / (2 + f) and a degree-7
//               polynomial R, a correction term c for the rounding of 1 + x,
//               in float arithmetic without fused operations.
//
// Both equal glibc 2.35's expf / log1pf on all 2^32 float inputs (NaN
// payloads aside), checked on the CPU by tests/test_libm.py.
#ifndef GDN_LIBM_H
#define GDN_LIBM_H

#include <stdint.h>
#include <string.h>

#ifdef __HIPCC__
#define GDN_HD __host__ __device__
#else
#define GDN_HD
#endif

namespace gdn_libm {

GDN_HD inline uint32_t bits_f(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
GDN_HD inline float from_bits_f(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
GDN_HD inline uint64_t bits_d(double d) {
    uint64_t u;
    memcpy(&u, &d, 8);
    return u;
}
GDN_HD inline double from_bits_d(uint64_t u) {
    double d;
    memcpy(&d, &u, 8);
    return d;
}
GDN_HD inline double fused(double a, double b, double c) { return __builtin_fma(a, b, c); }

// 2^(i/32) rounded to nearest double, minus i << 47 (so that adding k << 47
// for k = 32 m + i puts 2^m into the exponent field).
GDN_HD inline uint64_t exp2_table(int i) {
    static constexpr uint64_t T[32] = {
        0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
        0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
        0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
        0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
        0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
        0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
        0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
        0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
    };
    return T[i];
}

// The table as a function of i, for gdn_expf_t: the constant array, or a
// caller's copy (the kernels keep one in LDS, since a lookup in global memory
// costs a memory round trip on a kernel's serial tail).
struct Exp2Const {
    GDN_HD uint64_t operator()(int i) const { return exp2_table(i); }
};

template <class Tab>
GDN_HD inline float gdn_expf_t(float x, const Tab &tab) {
    constexpr double kN = 32.0;
    constexpr double kInvLn2N = 0x1.71547652b82fep+0 * kN;  // 32 / ln 2
    constexpr double kShift = 0x1.8p+52;
    // 2^(r/32) ~ 1 + C2 r + C1 r^2 + C0 r^3 on |r| <= 1/2 (the published
    // minimax coefficients of 2^x, scaled by powers of 1/32)
    constexpr double kC0 = 0x1.c6af84b912394p-5 / kN / kN / kN;
    constexpr double kC1 = 0x1.ebfce50fac4f3p-3 / kN / kN;
    constexpr double kC2 = 0x1.62e42ff0c52d6p-1 / kN;
    const uint32_t abstop = (bits_f(x) >> 20) & 0x7ffu;
    if (abstop >= (bits_f(88.0f) >> 20)) {  // |x| >= 88, infinities, NaN
        if (bits_f(x) == 0xff800000u) return 0.0f;
        if (abstop >= 0x7f8u) return x + x;
        if (x > 0x1.62e42ep6f) return from_bits_f(0x7f800000u);  // beyond log(2^128)
        if (x < -0x1.9fe368p6f) return 0.0f;                     // below log(2^-150)
    }
    const double xd = (double)x;
    double kd = fused(kInvLn2N, xd, kShift);  // k in the low mantissa bits
    const uint64_t ki = bits_d(kd);
    kd -= kShift;
    const double r = fused(kInvLn2N, xd, -kd);
    const double s = from_bits_d(tab((int)(ki % 32u)) + (ki << 47));
    const double z = fused(kC0, r, kC1);
    const double r2 = r * r;
    double y = fused(kC2, r, 1.0);
    y = fused(z, r2, y);
    y = y * s;
    return (float)y;
}

GDN_HD inline float gdn_expf(float x) { return gdn_expf_t(x, Exp2Const{}); }

GDN_HD inline float gdn_log1pf(float x) {
    constexpr float ln2_hi = 6.9313812256e-01f;  // 0x3f317180
    constexpr float ln2_lo = 9.0580006145e-06f;  // 0x3717f7d1
    constexpr float two25 = 3.355443200e+07f;
    constexpr float Lp1 = 6.6666668653e-01f, Lp2 = 4.0000000596e-01f, Lp3 = 2.8571429849e-01f,
                    Lp4 = 2.2222198546e-01f, Lp5 = 1.8183572590e-01f, Lp6 = 1.5313838422e-01f,
                    Lp7 = 1.4798198640e-01f;
    const int32_t hx = (int32_t)bits_f(x);
    const int32_t ax = hx & 0x7fffffff;
    float f = 0.0f, c = 0.0f;
    int32_t k = 1, hu = 0;
    if (hx < 0x3ed413d7) {  // x < sqrt(2) - 1
        if (ax >= 0x3f800000) {  // x <= -1
            if (x == -1.0f) return -two25 / 0.0f;
            return (x - x) / (x - x);
        }
        if (ax < 0x31000000) {  // |x| < 2^-29
            if (ax < 0x24800000) return x;
            return x - x * x * 0.5f;
        }
        if (hx > 0 || hx <= (int32_t)0xbe95f61f) {  // -0.2929 < x < 0.41422
            k = 0;
            f = x;
            hu = 1;
        }
    } else if (hx >= 0x7f800000) {
        return x + x;
    }
    if (k != 0) {
        float u;
        if (hx < 0x5a000000) {
            u = 1.0f + x;
            hu = (int32_t)bits_f(u);
            k = (hu >> 23) - 127;
            c = (k > 0) ? 1.0f - (u - x) : x - (u - 1.0f);  // the rounding error of 1 + x
            c /= u;
        } else {
            u = x;
            hu = (int32_t)bits_f(u);
            k = (hu >> 23) - 127;
            c = 0.0f;
        }
        hu &= 0x007fffff;
        if (hu < 0x3504f7) {
            u = from_bits_f((uint32_t)(hu | 0x3f800000));  // u in [1, sqrt 2)
        } else {
            k += 1;
            u = from_bits_f((uint32_t)(hu | 0x3f000000));  // u / 2 in [sqrt(2)/2, 1)
            hu = (0x00800000 - hu) >> 2;
        }
        f = u - 1.0f;
    }
    const float hfsq = 0.5f * f * f;
    const float kf = (float)k;
    if (hu == 0) {  // |f| < 2^-20
        if (f == 0.0f) {
            if (k == 0) return 0.0f;
            c += kf * ln2_lo;
            return kf * ln2_hi + c;
        }
        const float R = hfsq * (1.0f - 0.66666666666666666f * f);
        if (k == 0) return f - R;
        return kf * ln2_hi - ((R - (kf * ln2_lo + c)) - f);
    }
    const float s = f / (2.0f + f);
    const float z = s * s;
    const float R = z * (Lp1 + z * (Lp2 + z * (Lp3 + z * (Lp4 + z * (Lp5 + z * (Lp6 + z * Lp7))))));
    if (k == 0) return f - (hfsq - s * (hfsq + R));
    return kf * ln2_hi - ((hfsq - (s * (hfsq + R) + (kf * ln2_lo + c))) - f);
}

}  // namespace gdn_libm

#endif
