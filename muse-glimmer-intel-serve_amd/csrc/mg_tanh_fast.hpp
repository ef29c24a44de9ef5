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
//   a < 2^-5:  tanh a = a + a^3 P(a^2), P the series to a^11 (truncation
//              below 1e-18 relative);
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

    // the branch of tanh_fast_abs for 0 <= a < 2^-5
    MG_TF double tanh_series_abs(double a)
    {
        const double u = a * a;
        // tanh x / x - 1 = u (-1/3 + u (2/15 + u (-17/315 + u (62/2835 + u (-1382/155925)))))
        double p = -1382.0 / 155925.0;
        p = __builtin_fma(p, u, 62.0 / 2835.0);
        p = __builtin_fma(p, u, -17.0 / 315.0);
        p = __builtin_fma(p, u, 2.0 / 15.0);
        p = __builtin_fma(p, u, -1.0 / 3.0);
        return __builtin_fma(a * u, p, a);
    }

    MG_TF double tanh_fast_abs(double a)
    {
        if (a < 0x1p-5) return tanh_series_abs(a);
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
