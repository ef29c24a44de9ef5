// tanh of a value that is rounded to a storage format right afterwards (the
// output tail's rnd(tanh(rnd(z / cap))), src/muse_glimmer.hpp:920-943).
//
// tanh_fast_abs(a) evaluates tanh(a), a >= 0 finite, in f64 with a relative
// error far below kTanhFastMargin. A caller that finds t(1 - m) and t(1 + m)
// (m = kTanhFastMargin) rounding to the same stored value knows that FDLIBM's
// tanh(a), which lies in that interval too, rounds to it as well; otherwise
// it evaluates FDLIBM (rare: about 2m / 2^-24 of the inputs for f32).
//
// Method (Taylor series, ln 2 split into two doubles, all steps fma):
//   a < 1:     the degree-5 Taylor polynomial about a point a0 of a table of
//              tanh(a0) (correctly rounded, gen_tanh_table.py): a0 = 0 for
//              a < 1/128, where the polynomial is tanh's own series
//              a - a^3/3 + 2a^5/15 (truncation below 0.054 a^7, 2^-46.2
//              relative at most), else the interval's midpoint
//              a0 = (k + 0.5) / 128, |d| = |a - a0| <= 2^-8; its coefficients
//              come from t0 = tanh(a0) (every derivative of tanh is a
//              polynomial in tanh), and the remainder stays below 2^-51.8,
//              2^-44.8 relative at a = 2^-7;
//   a < 22:    tanh a = 1 - 2 / (e + 1), e = e^(2a) = 2^n e^r with
//              2a = n ln2 + r, |r| <= ln2 / 2, e^r by its Taylor polynomial
//              to r^12 (truncation below 2e-16). The cancellation in 1 - q is
//              worst at a = 2^-5 and multiplies the relative error by < 33,
//              so the error stays near 3e-14 against a margin of 9.1e-13;
//   a >= 22:   1, FDLIBM's own value (1 - 1e-300 rounds to 1).
// A host test runs every float input below 22 through this function and
// FDLIBM and checks the bound and every accepted rounding (f32, bf16, f16).
//
// Plain C++ with fma: the host and the device evaluate it to the same bits.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define MG_TF __host__ __device__ __forceinline__
#else
#define MG_TF inline
#endif

namespace mgm
{
    constexpr double kTanhFastMargin = 0x1p-40;

    // tanh((k + 0.5) / 128), correctly rounded, and tanh(0) at k = 0 (gen_tanh_table.py)
    alignas(16) inline constexpr double kTanhTab[128] = {
        0x0.0p+0, 0x1.7ffb801032f83p-7, 0x1.3ff595bd7be22p-6, 0x1.bfe36cdabb028p-6,
        0x1.1fe1a3d7a86c8p-5, 0x1.5fc89524d876dp-5, 0x1.9fa48d7b18ff3p-5, 0x1.df73915eafd29p-5,
        0x1.0f99d37864afap-4, 0x1.2f716b16ebeacp-4, 0x1.4f3f9495ba795p-4, 0x1.6f03562adb372p-4,
        0x1.8ebbb755f29f5p-4, 0x1.ae67c0fe4418bp-4, 0x1.ce067d9059519p-4, 0x1.ed96f91b44398p-4,
        0x1.068c20b6ba2adp-3, 0x1.1644b3188c2dcp-3, 0x1.25f4bc8402985p-3, 0x1.359bc6d38dd2ep-3,
        0x1.45395cf8933c6p-3, 0x1.54cd0b089533ap-3, 0x1.64565e4a112b0p-3, 0x1.73d4e54110e95p-3,
        0x1.83482fbb6c3adp-3, 0x1.92afcedcb8772p-3, 0x1.a20b5529e3630p-3, 0x1.b15a569477193p-3,
        0x1.c09c688584c74p-3, 0x1.cfd121e834330p-3, 0x1.def81b33f61f2p-3, 0x1.ee10ee7657cc7p-3,
        0x1.fd1b375c75fb3p-3, 0x1.060b499e06facp-2, 0x1.0d81508e15a87p-2, 0x1.14ef80deb89eep-2,
        0x1.1c55abd0ff2fbp-2, 0x1.23b3a38a75276p-2, 0x1.2b093b18ae071p-2, 0x1.325646749c6ebp-2,
        0x1.399a9a85b57f7p-2, 0x1.40d60d24e0132p-2, 0x1.4808751f2fb62p-2, 0x1.4f31aa386b63dp-2,
        0x1.5651852d60173p-2, 0x1.5d67dfb5ff52dp-2, 0x1.6474948749d36p-2, 0x1.6b777f5506b22p-2,
        0x1.72707cd3474adp-2, 0x1.795f6ab7b84a6p-2, 0x1.804427bac0592p-2, 0x1.871e93986ce2dp-2,
        0x1.8dee8f112d8d7p-2, 0x1.94b3fbea5efc1p-2, 0x1.9b6ebceea589fp-2, 0x1.a21eb5ee18b4cp-2,
        0x1.a8c3cbbe3ffaap-2, 0x1.af5de439e1fa8p-2, 0x1.b5ece640a6b15p-2, 0x1.bc70b9b68db8dp-2,
        0x1.c2e9478339745p-2, 0x1.c956799110245p-2, 0x1.cfb83acc33deep-2, 0x1.d60e77215274ap-2,
        0x1.dc591b7c4e500p-2, 0x1.e29815c6c164ap-2, 0x1.e8cb54e65b484p-2, 0x1.eef2c8bb1b96bp-2,
        0x1.f50e621d69c49p-2, 0x1.fb1e12dc0b8a8p-2, 0x1.0090e6dcfd8aep-1, 0x1.038cc3360f162p-1,
        0x1.068298cb6fbc6p-1, 0x1.09726265d5983p-1, 0x1.0c5c1b4328246p-1, 0x1.0f3fbf1523ba6p-1,
        0x1.121d49fff08e4p-1, 0x1.14f4b898adc55p-1, 0x1.17c607e3f1404p-1, 0x1.1a9135543cb4bp-1,
        0x1.1d563ec868aecp-1, 0x1.2015228a06141p-1, 0x1.22cddf4bb6be8p-1, 0x1.258074277dc64p-1,
        0x1.282ce09d080e0p-1, 0x1.2ad3248feda59p-1, 0x1.2d734045ec92ap-1, 0x1.300d34651d8f0p-1,
        0x1.32a101f223491p-1, 0x1.352eaa4e54b00p-1, 0x1.37b62f35e2d45p-1, 0x1.3a3792bdfae19p-1,
        0x1.3cb2d752e4b30p-1, 0x1.3f27ffb61e847p-1, 0x1.41970efc763a1p-1, 0x1.4400088c20babp-1,
        0x1.4662f01acfd20p-1, 0x1.48bfc9abc70e7p-1, 0x1.4b16998df00bep-1, 0x1.4d676459ee974p-1,
        0x1.4fb22ef035150p-1, 0x1.51f6fe771991bp-1, 0x1.5435d858ebdebp-1, 0x1.566ec2420d1b9p-1,
        0x1.58a1c21f0907fp-1, 0x1.5acede1ab176fp-1, 0x1.5cf61c9c3c3a1p-1, 0x1.5f17844563d4ap-1,
        0x1.61331bf08b47dp-1, 0x1.6348eaaee5411p-1, 0x1.6558f7c69ef4ap-1, 0x1.67634ab10ee6cp-1,
        0x1.6967eb18e7e6fp-1, 0x1.6b66e0d87079ap-1, 0x1.6d6033f7beec0p-1, 0x1.6f53ecaafa490p-1,
        0x1.71421350a064bp-1, 0x1.732ab06fd12e8p-1, 0x1.750dccb69f78fp-1, 0x1.76eb70f867622p-1,
        0x1.78c3a62c2a860p-1, 0x1.7a96756af21dfp-1, 0x1.7c63e7ee37332p-1, 0x1.7e2c070e5100bp-1,
        0x1.7feedc40e9a52p-1, 0x1.81ac7117793c5p-1, 0x1.8364cf3dc77a5p-1, 0x1.8518007873dd0p-1,
    };

    // the branch of tanh_fast_abs for 0 <= a < 1 (d = a - a0 is exact):
    //   tanh(a0 + d) = t0 + (1 - t0^2) d [1 - t0 d + (t0^2 - 1/3) d^2
    //                  + t0 (2/3 - t0^2) d^3 + (2/15 - t0^2 + t0^4) d^4] + R
    // (tab: kTanhTab or a copy of it, e.g. in a work-group's shared memory)
    MG_TF double tanh_table_abs(double a, const double *tab = kTanhTab)
    {
        const int k = int(a * 128.0);
        const double t = tab[k], u = t * t;
        const double d = a - (k == 0 ? 0.0 : (double(k) + 0.5) * 0x1p-7); // interval 0: about 0
        double e = __builtin_fma(u, u - 1.0, 2.0 / 15.0);
        e = __builtin_fma(d, e, t * (2.0 / 3.0 - u));
        e = __builtin_fma(d, e, u - 1.0 / 3.0);
        e = __builtin_fma(d, e, -t);
        e = __builtin_fma(d, e, 1.0);
        return __builtin_fma((1.0 - u) * d, e, t);
    }

    // the interval t (1 -+ m) that a caller rounds at both ends, one rounding each
    MG_TF void tanh_interval(double t, double &lo, double &hi, double m = kTanhFastMargin)
    {
        lo = __builtin_fma(-t, m, t);
        hi = __builtin_fma(t, m, t);
    }

    MG_TF double tanh_fast_abs(double a)
    {
        if (a < 1.0) return tanh_table_abs(a); // the table index stays in range for every a < 1
        if (a >= 22.0) return 1.0;
        const double y = a + a;
        constexpr double kLog2e = 1.4426950408889634;     // 1 / ln 2
        constexpr double kLn2Hi = 0.6931471805599453;     // ln 2 rounded to double
        constexpr double kLn2Lo = 2.3190468138462996e-17; // ln 2 - kLn2Hi
        const double n = __builtin_rint(y * kLog2e);
        double r = __builtin_fma(-n, kLn2Hi, y);
        r = __builtin_fma(-n, kLn2Lo, r);
        // e^r = sum r^k / k!, k = 0..12
        double p = 1.0 / 479001600.0;
        p = __builtin_fma(p, r, 1.0 / 39916800.0);
        p = __builtin_fma(p, r, 1.0 / 3628800.0);
        p = __builtin_fma(p, r, 1.0 / 362880.0);
        p = __builtin_fma(p, r, 1.0 / 40320.0);
        p = __builtin_fma(p, r, 1.0 / 5040.0);
        p = __builtin_fma(p, r, 1.0 / 720.0);
        p = __builtin_fma(p, r, 1.0 / 120.0);
        p = __builtin_fma(p, r, 1.0 / 24.0);
        p = __builtin_fma(p, r, 1.0 / 6.0);
        p = __builtin_fma(p, r, 0.5);
        p = __builtin_fma(p, r, 1.0);
        p = __builtin_fma(p, r, 1.0);
        // 2^n through the exponent field (0 <= n <= 64)
        const uint64_t sbits = uint64_t(1023 + int(n)) << 52;
        const double e = p * __builtin_bit_cast(double, sbits);
        return 1.0 - 2.0 / (e + 1.0);
    }
} // namespace mgm
