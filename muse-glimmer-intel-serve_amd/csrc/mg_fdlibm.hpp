// Deterministic f64 transcendentals for host and device, bit-identical to the
// reference's src/fmath.hpp (FDLIBM 5.3 derived).
//
//   FDLIBM: "Developed at SunSoft, a Sun Microsystems business. Permission to
//   use, copy, modify, and distribute this software is freely granted,
//   provided that this notice is preserved."
//
// The reference's bf16/f16 twin evaluates silu/sigmoid/tanh/RoPE angles with
// these algorithms, and its results are pinned to their exact IEEE operation
// sequence. gfx950's f64 add/mul/div/sqrt/fma are IEEE correctly rounded, so
// keeping FDLIBM's branch structure and operation order — and compiling with
// -ffp-contract=off — reproduces the twin bit for bit on the GPU. Only the
// functions the primitives need are here: exp (silu, sigmoid, softmax merge),
// expm1 + tanh (softcap), log (logsumexp merge), pow + sin + cos (RoPE table).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define MG_HD __host__ __device__ __forceinline__

namespace mgm
{
    MG_HD uint64_t d2u(double x) { return __builtin_bit_cast(uint64_t, x); }
    MG_HD double u2d(uint64_t u) { return __builtin_bit_cast(double, u); }
    MG_HD uint32_t hi32(double x) { return uint32_t(d2u(x) >> 32); }
    MG_HD uint32_t lo32(double x) { return uint32_t(d2u(x)); }
    MG_HD double replace_hi(double x, uint32_t h) { return u2d((uint64_t(h) << 32) | (d2u(x) & 0xffffffffull)); }
    MG_HD double pack_hl(uint32_t h, uint32_t l) { return u2d((uint64_t(h) << 32) | l); }
    // y * 2^k through the exponent field; valid while the result stays normal
    MG_HD double mul_pow2(double y, int k) { return u2d(d2u(y) + (uint64_t(int64_t(k)) << 52)); }

    constexpr double kLn2Hi = 6.93147180369123816490e-01;
    constexpr double kLn2Lo = 1.90821492927058770002e-10;
    constexpr double kInvLn2 = 1.44269504088896338700e+00;
    constexpr double kHuge = 1.0e+300;
    constexpr double kTwoM1000 = 9.33263618503218878990e-302;

    // e^x (FDLIBM e_exp.c; reference fmath.hpp:60-124)
    MG_HD double exp(double x)
    {
        uint32_t hx = hi32(x);
        const int sgn = int(hx >> 31);
        hx &= 0x7fffffffu;
        if (hx >= 0x40862E42u) {
            if (hx >= 0x7ff00000u) {
                if (((hx & 0xfffffu) | lo32(x)) != 0) return x + x;
                return sgn == 0 ? x : 0.0;
            }
            if (x > 7.09782712893383973096e+02) return kHuge * kHuge;
            if (x < -7.45133219101941108420e+02) return kTwoM1000 * kTwoM1000;
        }
        double hi = 0.0, lo = 0.0;
        int k = 0;
        if (hx > 0x3fd62e42u) {
            if (hx < 0x3FF0A2B2u) {
                hi = sgn ? x + kLn2Hi : x - kLn2Hi;
                lo = sgn ? -kLn2Lo : kLn2Lo;
                k = sgn ? -1 : 1;
            } else {
                k = int(kInvLn2 * x + (sgn ? -0.5 : 0.5));
                const double t = double(k);
                hi = x - t * kLn2Hi;
                lo = t * kLn2Lo;
            }
            x = hi - lo;
        } else if (hx < 0x3e300000u) {
            if (kHuge + x > 1.0) return 1.0 + x;
        }
        const double t = x * x;
        const double c = x - t * (1.66666666666666019037e-01 +
                                  t * (-2.77777777770155933842e-03 +
                                       t * (6.61375632143793436117e-05 +
                                            t * (-1.65339022054652515390e-06 +
                                                 t * 4.13813679705723846039e-08))));
        if (k == 0) return 1.0 - ((x * c) / (c - 2.0) - x);
        const double y = 1.0 - ((lo - (x * c) / (2.0 - c)) - hi);
        if (k >= -1021) return mul_pow2(y, k);
        return mul_pow2(y, k + 1000) * kTwoM1000;
    }

    // natural log (FDLIBM e_log.c; reference fmath.hpp:128-185). x <= 0 handled as there.
    MG_HD double log(double x)
    {
        constexpr double L1 = 6.666666666666735130e-01, L2 = 3.999999999940941908e-01,
                         L3 = 2.857142874366239149e-01, L4 = 2.222219843214978396e-01,
                         L5 = 1.818357216161805012e-01, L6 = 1.531383769920937332e-01,
                         L7 = 1.479819860511658591e-01;
        uint32_t hx = hi32(x);
        int k = 0;
        if (hx < 0x00100000u) {
            if (((hx & 0x7fffffffu) | lo32(x)) == 0) return -__builtin_huge_val();
            if (hx >> 31) return __builtin_nan("");
            k -= 54;
            x *= 1.80143985094819840000e+16;
            hx = hi32(x);
        }
        if (hx >= 0x7ff00000u) return x + x;
        k += int(hx >> 20) - 1023;
        hx &= 0x000fffffu;
        int i = int((hx + 0x95f64u) & 0x100000u);
        x = replace_hi(x, hx | (uint32_t(i) ^ 0x3ff00000u));
        k += i >> 20;
        const double f = x - 1.0;
        const double dk = double(k);
        if ((0x000fffffu & (2 + hx)) < 3) {
            if (f == 0.0) {
                if (k == 0) return 0.0;
                return dk * kLn2Hi + dk * kLn2Lo;
            }
            const double R = f * f * (0.5 - 0.33333333333333333 * f);
            if (k == 0) return f - R;
            return dk * kLn2Hi - ((R - dk * kLn2Lo) - f);
        }
        const double s = f / (2.0 + f);
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
            return dk * kLn2Hi - ((hfsq - (s * (hfsq + R) + dk * kLn2Lo)) - f);
        }
        if (k == 0) return f - s * (f - R);
        return dk * kLn2Hi - ((s * (f - R) - dk * kLn2Lo) - f);
    }

    // a^b = exp(b log a) with the exact fma residual (reference fmath.hpp:265-277);
    // only a > 0 finite is supported (callers validate theta on the host).
    MG_HD double pow(double a, double b)
    {
        if (b == 0.0 || a == 1.0) return 1.0;
        const double l = mgm::log(a);
        const double p = l * b;
        const double e = __builtin_fma(l, b, -p);
        const double y = mgm::exp(p);
        return y + y * e;
    }

    // e^x - 1 (FDLIBM s_expm1.c; reference fmath.hpp:281-385)
    MG_HD double expm1(double x)
    {
        uint32_t hx = hi32(x);
        const bool neg = (hx & 0x80000000u) != 0;
        hx &= 0x7fffffffu;
        if (hx >= 0x4043687Au) {
            if (hx >= 0x40862E42u) {
                if (hx >= 0x7ff00000u) {
                    if (((hx & 0xfffffu) | lo32(x)) != 0) return x + x;
                    return neg ? -1.0 : x;
                }
                if (x > 7.09782712893383973096e+02) return kHuge * kHuge;
            }
            if (neg && x + 1.0e-300 < 0.0) return 1.0e-300 - 1.0;
        }
        double c = 0.0;
        int k = 0;
        if (hx > 0x3fd62e42u) {
            double hi, lo;
            if (hx < 0x3FF0A2B2u) {
                hi = neg ? x + kLn2Hi : x - kLn2Hi;
                lo = neg ? -kLn2Lo : kLn2Lo;
                k = neg ? -1 : 1;
            } else {
                k = int(kInvLn2 * x + (neg ? -0.5 : 0.5));
                const double t = double(k);
                hi = x - t * kLn2Hi;
                lo = t * kLn2Lo;
            }
            x = hi - lo;
            c = (hi - x) - lo;
        } else if (hx < 0x3c900000u) {
            return x;
        }
        const double hfx = 0.5 * x;
        const double hxs = x * hfx;
        const double r1 = 1.0 + hxs * (-3.33333333333331316428e-02 +
                                       hxs * (1.58730158725481460165e-03 +
                                              hxs * (-7.93650757867487942473e-05 +
                                                     hxs * (4.00821782732936239552e-06 +
                                                            hxs * -2.01099218183624371326e-07))));
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
            y = (k == 1024) ? y * 2.0 * 8.98846567431157953865e+307 : mul_pow2(y, k);
            return y - 1.0;
        }
        if (k < 20) {
            t = pack_hl(uint32_t(0x3ff00000 - (0x200000 >> k)), 0);
            y = t - (e - x);
        } else {
            t = pack_hl(uint32_t((0x3ff - k) << 20), 0);
            y = x - (e + t);
            y += 1.0;
        }
        return mul_pow2(y, k);
    }

    // tanh via expm1 (FDLIBM s_tanh.c; reference fmath.hpp:389-415)
    MG_HD double tanh(double x)
    {
        const uint32_t jx = hi32(x), ix = jx & 0x7fffffffu;
        if (ix >= 0x7ff00000u) {
            if ((ix & 0xfffffu) | lo32(x)) return x + x;
            return (jx >> 31) ? -1.0 : 1.0;
        }
        double z;
        if (ix < 0x40360000u) {
            if (ix < 0x3c800000u) return x * (1.0 + x);
            const double ax = __builtin_fabs(x);
            if (ix >= 0x3ff00000u) {
                const double t = mgm::expm1(2.0 * ax);
                z = 1.0 - 2.0 / (t + 2.0);
            } else {
                const double t = mgm::expm1(-2.0 * ax);
                z = -t / (t + 2.0);
            }
        } else {
            z = 1.0 - 1.0e-300;
        }
        return (jx >> 31) ? -z : z;
    }

    // FDLIBM __kernel_sin / __kernel_cos on the reduced argument y0 + y1
    // (reference fmath.hpp:419-464)
    MG_HD double poly_sin(double x, double y, bool has_tail)
    {
        const double z = x * x;
        const double v = z * x;
        const double r = 8.33333333332248946124e-03 +
                         z * (-1.98412698298579493134e-04 +
                              z * (2.75573137070700676789e-06 +
                                   z * (-2.50507602534068634195e-08 + z * 1.58969099521155010221e-10)));
        if (!has_tail) return x + v * (-1.66666666666666324348e-01 + z * r);
        return x - ((z * (0.5 * y - v * r) - y) - v * -1.66666666666666324348e-01);
    }
    MG_HD double poly_cos(double x, double y)
    {
        const uint32_t ix = hi32(x) & 0x7fffffffu;
        const double z = x * x;
        const double r = z * (4.16666666666666019037e-02 +
                              z * (-1.38888888888741095749e-03 +
                                   z * (2.48015872894767294178e-05 +
                                        z * (-2.75573143513906633035e-07 +
                                             z * (2.08757232129817482790e-09 +
                                                  z * -1.13596475577881948265e-11)))));
        if (ix < 0x3fd33333u) return 1.0 - (0.5 * z - (z * r - x * y));
        const double qx = (ix > 0x3fe90000u) ? 0.28125 : pack_hl(ix - 0x00200000u, 0);
        const double hz = 0.5 * z - qx;
        const double a = 1.0 - qx;
        return a - (hz - (z * r - x * y));
    }

    // x = n·π/2 + (y0 + y1), FDLIBM e_rem_pio2.c medium path (reference
    // fmath.hpp:469-518), valid for |x| < 2^20·π/2; callers check the range on
    // the host (RoPE angles are bounded by the table length).
    MG_HD int reduce_pio2(double x, double &y0, double &y1)
    {
        const uint32_t hx = hi32(x), ix = hx & 0x7fffffffu;
        double t = __builtin_fabs(x);
        const int n = int(t * 6.36619772367581382433e-01 + 0.5);
        const double fn = double(n);
        double r = t - fn * 1.57079632673412561417e+00;
        double w = fn * 6.07710050650619224932e-11;
        y0 = r - w;
        const int j = int(ix >> 20);
        int i = j - int((hi32(y0) >> 20) & 0x7ff);
        if (i > 16) {
            t = r;
            w = fn * 6.07710050630396597660e-11;
            r = t - w;
            w = fn * 2.02226624879595063154e-21 - ((t - r) - w);
            y0 = r - w;
            i = j - int((hi32(y0) >> 20) & 0x7ff);
            if (i > 49) {
                t = r;
                w = fn * 2.02226624871116645580e-21;
                r = t - w;
                w = fn * 8.47842766036889956997e-32 - ((t - r) - w);
                y0 = r - w;
            }
        }
        y1 = (r - y0) - w;
        if (hx >> 31) {
            y0 = -y0;
            y1 = -y1;
            return -n;
        }
        return n;
    }

    // reference fmath.hpp:520-543
    MG_HD double sin(double x)
    {
        const uint32_t ix = hi32(x) & 0x7fffffffu;
        if (ix <= 0x3fe921fbu) return ix < 0x3e500000u ? x : poly_sin(x, 0.0, false);
        if (ix >= 0x7ff00000u) return x - x;
        double y0, y1;
        const int n = reduce_pio2(x, y0, y1);
        switch (n & 3) {
        case 0: return poly_sin(y0, y1, true);
        case 1: return poly_cos(y0, y1);
        case 2: return -poly_sin(y0, y1, true);
        default: return -poly_cos(y0, y1);
        }
    }

    // reference fmath.hpp:617-640
    MG_HD double cos(double x)
    {
        const uint32_t ix = hi32(x) & 0x7fffffffu;
        if (ix <= 0x3fe921fbu) return ix < 0x3e46a09eu ? 1.0 : poly_cos(x, 0.0);
        if (ix >= 0x7ff00000u) return x - x;
        double y0, y1;
        const int n = reduce_pio2(x, y0, y1);
        switch (n & 3) {
        case 0: return poly_cos(y0, y1);
        case 1: return -poly_sin(y0, y1, true);
        case 2: return -poly_cos(y0, y1);
        default: return poly_sin(y0, y1, true);
        }
    }

    // the twin's silu and sigmoid (reference muse_glimmer.hpp:493-494)
    MG_HD double silu(double x) { return x / (1.0 + mgm::exp(-x)); }
    MG_HD double sigmoid(double x) { return 1.0 / (1.0 + mgm::exp(-x)); }
} // namespace mgm
