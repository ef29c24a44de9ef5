// ORACLE — test infrastructure only. Nothing in the shipped library includes this file.
//
// CPU restatement of the reference's deterministic f64 transcendentals
// (/root/reference/src/fmath.hpp), which are FDLIBM 5.3 algorithms:
//   "Developed at SunSoft, a Sun Microsystems business. Permission to use, copy,
//    modify, and distribute this software is freely granted, provided that this
//    notice is preserved."
// The bitwise contract of the reference's twin depends on the exact sequence of
// IEEE operations, so every function below keeps FDLIBM's branch structure and
// operation order; it must be compiled with -ffp-contract=off.
//
// Pinned by: tests/test_oracle_fmath.py (bitwise against oracle/_ref, the
// reference's own tools/oracle_kernels.cpp compiled from /root/reference; ulp
// bounds against libm as tests/fmath_test.cpp:54-185 does; identities).
#pragma once

#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>

namespace orc
{
    inline uint64_t bits(double x) { uint64_t u; std::memcpy(&u, &x, 8); return u; }
    inline double from_bits(uint64_t u) { double x; std::memcpy(&x, &u, 8); return x; }
    inline uint32_t hiw(double x) { return uint32_t(bits(x) >> 32); }
    inline uint32_t low(double x) { return uint32_t(bits(x)); }
    inline double with_hi(double x, uint32_t h) { return from_bits((uint64_t(h) << 32) | (bits(x) & 0xffffffffull)); }
    inline double make_hl(uint32_t h, uint32_t l) { return from_bits((uint64_t(h) << 32) | l); }
    // y * 2^k by exponent arithmetic (result normal) — fmath.hpp:53-56
    inline double ldexp_bits(double y, int k) { return from_bits(bits(y) + (uint64_t(int64_t(k)) << 52)); }

    // fmath::exp — fmath.hpp:60-124 (FDLIBM e_exp.c)
    inline double exp(double x)
    {
        const double ln2_hi[2] = {6.93147180369123816490e-01, -6.93147180369123816490e-01};
        const double ln2_lo[2] = {1.90821492927058770002e-10, -1.90821492927058770002e-10};
        const double half[2] = {0.5, -0.5};
        const double inv_ln2 = 1.44269504088896338700e+00;
        const double P1 = 1.66666666666666019037e-01, P2 = -2.77777777770155933842e-03,
                     P3 = 6.61375632143793436117e-05, P4 = -1.65339022054652515390e-06,
                     P5 = 4.13813679705723846039e-08;
        const double big = 1.0e+300, tiny2 = 9.33263618503218878990e-302;
        uint32_t ax = hiw(x);
        const int neg = int(ax >> 31);
        ax &= 0x7fffffffu;
        if (ax >= 0x40862E42u) {
            if (ax >= 0x7ff00000u) {
                if (((ax & 0xfffffu) | low(x)) != 0) return x + x;
                return neg ? 0.0 : x;
            }
            if (x > 7.09782712893383973096e+02) return big * big;
            if (x < -7.45133219101941108420e+02) return tiny2 * tiny2;
        }
        double hi = 0.0, lo = 0.0;
        int k = 0;
        if (ax > 0x3fd62e42u) {
            if (ax < 0x3FF0A2B2u) {
                hi = x - ln2_hi[neg];
                lo = ln2_lo[neg];
                k = 1 - neg - neg;
            } else {
                k = int(inv_ln2 * x + half[neg]);
                const double kd = k;
                hi = x - kd * ln2_hi[0];
                lo = kd * ln2_lo[0];
            }
            x = hi - lo;
        } else if (ax < 0x3e300000u) {
            if (big + x > 1.0) return 1.0 + x;
        }
        const double t = x * x;
        const double c = x - t * (P1 + t * (P2 + t * (P3 + t * (P4 + t * P5))));
        if (k == 0) return 1.0 - ((x * c) / (c - 2.0) - x);
        const double y = 1.0 - ((lo - (x * c) / (2.0 - c)) - hi);
        if (k >= -1021) return ldexp_bits(y, k);
        return ldexp_bits(y, k + 1000) * tiny2;
    }

    // fmath::log — fmath.hpp:128-185 (FDLIBM e_log.c)
    inline double log(double x)
    {
        const double ln2_hi = 6.93147180369123816490e-01, ln2_lo = 1.90821492927058770002e-10;
        const double two54 = 1.80143985094819840000e+16;
        const double L1 = 6.666666666666735130e-01, L2 = 3.999999999940941908e-01,
                     L3 = 2.857142874366239149e-01, L4 = 2.222219843214978396e-01,
                     L5 = 1.818357216161805012e-01, L6 = 1.531383769920937332e-01,
                     L7 = 1.479819860511658591e-01;
        uint32_t hx = hiw(x);
        const uint32_t lx = low(x);
        int k = 0;
        if (hx < 0x00100000u) {
            if (((hx & 0x7fffffffu) | lx) == 0) return -HUGE_VAL;
            if (hx >> 31) return std::numeric_limits<double>::quiet_NaN();
            k -= 54;
            x *= two54;
            hx = hiw(x);
        }
        if (hx >= 0x7ff00000u) return x + x;
        k += int(hx >> 20) - 1023;
        hx &= 0x000fffffu;
        int i = int((hx + 0x95f64u) & 0x100000u);
        x = with_hi(x, hx | (uint32_t(i) ^ 0x3ff00000u));
        k += i >> 20;
        const double f = x - 1.0;
        if ((0x000fffffu & (2 + hx)) < 3) {
            if (f == 0.0) {
                if (k == 0) return 0.0;
                const double dk = double(k);
                return dk * ln2_hi + dk * ln2_lo;
            }
            const double R = f * f * (0.5 - 0.33333333333333333 * f);
            if (k == 0) return f - R;
            const double dk = double(k);
            return dk * ln2_hi - ((R - dk * ln2_lo) - f);
        }
        const double s = f / (2.0 + f);
        const double dk = double(k);
        const double z = s * s;
        i = int(hx) - 0x6147a;
        const double w = z * z;
        const int j = 0x6b851 - int(hx);
        const double t1 = w * (L2 + w * (L4 + w * L6));
        const double t2 = z * (L1 + w * (L3 + w * (L5 + w * L7)));
        i |= j;
        const double R = t2 + t1;
        if (i > 0) {
            const double hfsq = 0.5 * f * f;
            if (k == 0) return f - (hfsq - s * (hfsq + R));
            return dk * ln2_hi - ((hfsq - (s * (hfsq + R) + dk * ln2_lo)) - f);
        }
        if (k == 0) return f - s * (f - R);
        return dk * ln2_hi - ((s * (f - R) - dk * ln2_lo) - f);
    }

    // fmath::pow — fmath.hpp:265-277: exp(b·log a) with the exact fma residual of b·log a.
    // Domain a > 0 finite; anything else returns NaN here (the reference throws).
    inline double pow(double a, double b)
    {
        if (b == 0.0 || a == 1.0) return 1.0;
        if (!(a > 0.0) || a == HUGE_VAL) return std::numeric_limits<double>::quiet_NaN();
        const double l = orc::log(a);
        const double p = l * b;
        const double e = std::fma(l, b, -p);
        const double y = orc::exp(p);
        return y + y * e;
    }

    // fmath::expm1 — fmath.hpp:281-385 (FDLIBM s_expm1.c)
    inline double expm1(double x)
    {
        const double ln2_hi = 6.93147180369123816490e-01, ln2_lo = 1.90821492927058770002e-10;
        const double inv_ln2 = 1.44269504088896338700e+00;
        const double Q1 = -3.33333333333331316428e-02, Q2 = 1.58730158725481460165e-03,
                     Q3 = -7.93650757867487942473e-05, Q4 = 4.00821782732936239552e-06,
                     Q5 = -2.01099218183624371326e-07;
        const double big = 1.0e+300, tiny = 1.0e-300;
        uint32_t ax = hiw(x);
        const bool neg = (ax & 0x80000000u) != 0;
        ax &= 0x7fffffffu;
        if (ax >= 0x4043687Au) {
            if (ax >= 0x40862E42u) {
                if (ax >= 0x7ff00000u) {
                    if (((ax & 0xfffffu) | low(x)) != 0) return x + x;
                    return neg ? -1.0 : x;
                }
                if (x > 7.09782712893383973096e+02) return big * big;
            }
            if (neg && x + tiny < 0.0) return tiny - 1.0;
        }
        double hi, lo, c = 0.0;
        int k;
        if (ax > 0x3fd62e42u) {
            if (ax < 0x3FF0A2B2u) {
                if (!neg) { hi = x - ln2_hi; lo = ln2_lo; k = 1; }
                else { hi = x + ln2_hi; lo = -ln2_lo; k = -1; }
            } else {
                k = int(inv_ln2 * x + (neg ? -0.5 : 0.5));
                const double kd = k;
                hi = x - kd * ln2_hi;
                lo = kd * ln2_lo;
            }
            x = hi - lo;
            c = (hi - x) - lo;
        } else if (ax < 0x3c900000u) {
            return x;
        } else {
            k = 0;
        }
        const double hfx = 0.5 * x;
        const double hxs = x * hfx;
        const double r1 = 1.0 + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
        double t = 3.0 - r1 * hfx;
        double e = hxs * ((r1 - t) / (6.0 - x * t));
        if (k == 0) return x - (x * e - hxs);
        e = (x * (e - c) - c);
        e -= hxs;
        if (k == -1) return 0.5 * (x - e) - 0.5;
        if (k == 1) {
            if (x < -0.25) return -2.0 * (e - (x + 0.5));
            return 1.0 + 2.0 * (x - e);
        }
        double y;
        if (k <= -2 || k > 56) {
            y = 1.0 - (e - x);
            if (k == 1024) y = y * 2.0 * 8.98846567431157953865e+307;
            else y = ldexp_bits(y, k);
            return y - 1.0;
        }
        if (k < 20) {
            t = make_hl(uint32_t(0x3ff00000 - (0x200000 >> k)), 0);
            y = t - (e - x);
            y = ldexp_bits(y, k);
        } else {
            t = make_hl(uint32_t((0x3ff - k) << 20), 0);
            y = x - (e + t);
            y += 1.0;
            y = ldexp_bits(y, k);
        }
        return y;
    }

    // fmath::tanh — fmath.hpp:389-415 (FDLIBM s_tanh.c)
    inline double tanh(double x)
    {
        const uint32_t jx = hiw(x), ix = jx & 0x7fffffffu;
        if (ix >= 0x7ff00000u) {
            if ((ix & 0xfffffu) | low(x)) return x + x;
            return (jx >> 31) ? -1.0 : 1.0;
        }
        double z;
        if (ix < 0x40360000u) {
            if (ix < 0x3c800000u) return x * (1.0 + x);
            if (ix >= 0x3ff00000u) {
                const double t = orc::expm1(2.0 * std::fabs(x));
                z = 1.0 - 2.0 / (t + 2.0);
            } else {
                const double t = orc::expm1(-2.0 * std::fabs(x));
                z = -t / (t + 2.0);
            }
        } else {
            z = 1.0 - 1.0e-300;
        }
        return (jx >> 31) ? -z : z;
    }

    // FDLIBM __kernel_sin / __kernel_cos — fmath.hpp:419-464
    inline double ksin(double x, double y, int iy)
    {
        const double S1 = -1.66666666666666324348e-01, S2 = 8.33333333332248946124e-03,
                     S3 = -1.98412698298579493134e-04, S4 = 2.75573137070700676789e-06,
                     S5 = -2.50507602534068634195e-08, S6 = 1.58969099521155010221e-10;
        const double z = x * x;
        const double v = z * x;
        const double r = S2 + z * (S3 + z * (S4 + z * (S5 + z * S6)));
        if (iy == 0) return x + v * (S1 + z * r);
        return x - ((z * (0.5 * y - v * r) - y) - v * S1);
    }

    inline double kcos(double x, double y)
    {
        const double C1 = 4.16666666666666019037e-02, C2 = -1.38888888888741095749e-03,
                     C3 = 2.48015872894767294178e-05, C4 = -2.75573143513906633035e-07,
                     C5 = 2.08757232129817482790e-09, C6 = -1.13596475577881948265e-11;
        const uint32_t ix = hiw(x) & 0x7fffffffu;
        const double z = x * x;
        const double r = z * (C1 + z * (C2 + z * (C3 + z * (C4 + z * (C5 + z * C6)))));
        if (ix < 0x3fd33333u) return 1.0 - (0.5 * z - (z * r - x * y));
        const double qx = (ix > 0x3fe90000u) ? 0.28125 : make_hl(ix - 0x00200000u, 0);
        const double hz = 0.5 * z - qx;
        const double a = 1.0 - qx;
        return a - (hz - (z * r - x * y));
    }

    // FDLIBM e_rem_pio2.c medium path — fmath.hpp:469-518. Returns false where the
    // reference throws (|x| >= 2^20·π/2).
    inline bool rem_pio2(double x, double *y, int *quadrant)
    {
        const double invpio2 = 6.36619772367581382433e-01;
        const double pio2_1 = 1.57079632673412561417e+00, pio2_1t = 6.07710050650619224932e-11;
        const double pio2_2 = 6.07710050630396597660e-11, pio2_2t = 2.02226624879595063154e-21;
        const double pio2_3 = 2.02226624871116645580e-21, pio2_3t = 8.47842766036889956997e-32;
        const uint32_t hx = hiw(x), ix = hx & 0x7fffffffu;
        if (ix >= 0x413921fbu) return false;
        double t = std::fabs(x);
        const int n = int(t * invpio2 + 0.5);
        const double fn = double(n);
        double r = t - fn * pio2_1;
        double w = fn * pio2_1t;
        y[0] = r - w;
        const int j = int(ix >> 20);
        int i = j - int((hiw(y[0]) >> 20) & 0x7ff);
        if (i > 16) {
            t = r;
            w = fn * pio2_2;
            r = t - w;
            w = fn * pio2_2t - ((t - r) - w);
            y[0] = r - w;
            i = j - int((hiw(y[0]) >> 20) & 0x7ff);
            if (i > 49) {
                t = r;
                w = fn * pio2_3;
                r = t - w;
                w = fn * pio2_3t - ((t - r) - w);
                y[0] = r - w;
            }
        }
        y[1] = (r - y[0]) - w;
        if (hx >> 31) {
            y[0] = -y[0];
            y[1] = -y[1];
            *quadrant = -n;
        } else {
            *quadrant = n;
        }
        return true;
    }

    // fmath::sin — fmath.hpp:520-543
    inline double sin(double x)
    {
        const uint32_t ix = hiw(x) & 0x7fffffffu;
        if (ix <= 0x3fe921fbu) {
            if (ix < 0x3e500000u) return x;
            return ksin(x, 0.0, 0);
        }
        if (ix >= 0x7ff00000u) return x - x;
        double y[2];
        int n;
        if (!rem_pio2(x, y, &n)) return std::numeric_limits<double>::quiet_NaN();
        switch (n & 3) {
        case 0: return ksin(y[0], y[1], 1);
        case 1: return kcos(y[0], y[1]);
        case 2: return -ksin(y[0], y[1], 1);
        default: return -kcos(y[0], y[1]);
        }
    }

    // fmath::cos — fmath.hpp:617-640
    inline double cos(double x)
    {
        const uint32_t ix = hiw(x) & 0x7fffffffu;
        if (ix <= 0x3fe921fbu) {
            if (ix < 0x3e46a09eu) return 1.0;
            return kcos(x, 0.0);
        }
        if (ix >= 0x7ff00000u) return x - x;
        double y[2];
        int n;
        if (!rem_pio2(x, y, &n)) return std::numeric_limits<double>::quiet_NaN();
        switch (n & 3) {
        case 0: return kcos(y[0], y[1]);
        case 1: return -ksin(y[0], y[1], 1);
        case 2: return -kcos(y[0], y[1]);
        default: return ksin(y[0], y[1], 1);
        }
    }
} // namespace orc
