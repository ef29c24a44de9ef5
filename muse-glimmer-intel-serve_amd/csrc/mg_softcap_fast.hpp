// The softcapped attention score of one f32 score without a division or a
// per-key branch: the value of rnd(cap * rnd(tanh(rnd(rnd(x * scale) / cap))))
// in f32 (apply_output_tail's op order, src/muse_glimmer.hpp:920-943, as the
// twin rounds each step), for the keys where two cheap steps are certain:
//
//   s / cap  Markstein's correction of q0 = s * rcap with rcap = RN(1 / cap):
//            q = RN(q0 + (s - q0 cap) rcap), the remainder exact by fma, is
//            the correctly rounded quotient when operands and quotient are
//            normal (P. Markstein, IBM J. Res. Dev. 34(1), 1990); the host
//            test checks it against the IEEE quotient for every f32 s with
//            2^-100 < |s| < 2^100 at several caps, negative ones included.
//            With 1 <= |cap| <= 2^20 (the caller's condition) a result with
//            2^-99 <= |q| < 2^-5 implies s in that range: |s| < 2^-100 gives
//            |q| <= 2 |s| < 2^-99, and |s| >= 2^100 gives |q| >= 2^80.
//   tanh     tanh a = a + a^3 (-1/3 + 2/15 a^2 - 17/315 a^4) in f64 for
//            a = |q| < 2^-5: the dropped terms are below 0.022 a^9, a
//            relative error under 2^-45.5. Its f32 rounding equals that of
//            FDLIBM's tanh (itself within an f64 ulp) whenever the 29
//            mantissa bits below the f32 ones stay more than 2^13 units from
//            the midpoint 2^28: 2^13 units of t's binade are at least 2^-40 |t|.
//            For a >= 2^-99 the result is a normal f32, where that test holds.
//
// `ok` is false where either step is not certain (|q| >= 2^-5 included);
// the caller then evaluates the plain chain (IEEE quotient, FDLIBM tanh).
// Plain C++ with fma: the host test and the device evaluate the same bits.
#pragma once

#include <stdint.h>

#include "mg_tanh_fast.hpp"

#if defined(__HIPCC__)
#define MG_SF __host__ __device__ __forceinline__
#else
#define MG_SF inline
#endif

namespace mgm
{
    // RN(1 / c) in f32 for a finite nonzero f32 c, the rcap the kernels take
    // (computed on the host): the f64 quotient rounded to f32, then corrected
    // to the neighbour whose residual 1 - r c (exact in f64: r c has at most
    // 48 significant bits) is smallest. Host code; the exhaustive checker
    // calls this same function.
    inline float recip_rn(float c)
    {
        const float r = float(1.0 / double(c));
        const float nb[2] = {__builtin_nextafterf(r, 0.0f), __builtin_nextafterf(r, 2.0f * r)};
        float best = r;
        double err = __builtin_fabs(1.0 - double(r) * double(c));
        for (int i = 0; i < 2; ++i) {
            const double e = __builtin_fabs(1.0 - double(nb[i]) * double(c));
            if (e < err) {
                err = e;
                best = nb[i];
            }
        }
        return best;
    }

    MG_SF float softcap_quotient(float s, float cap, float rcap)
    {
        const float q0 = s * rcap;
        const float r = __builtin_fmaf(-q0, cap, s);
        return __builtin_fmaf(r, rcap, q0);
    }

    // t's f32 rounding cannot change within `units` f64 ulps of t (the test
    // uses 2^13: 2^-40 |t| at least); t a positive normal in f32 range
    MG_SF bool f32_rounding_certain(double t, uint32_t units = 0x2000u)
    {
        const uint32_t low = uint32_t(__builtin_bit_cast(uint64_t, t)) & 0x1fffffffu;
        return uint32_t(int32_t(low) - 0x10000000 + int32_t(units)) > 2u * units;
    }

    // tanh a for 0 <= a < 2^-5, relative error below 2^-45
    MG_SF double tanh_small_abs(double a)
    {
        const double v = a * a;
        const double p = __builtin_fma(__builtin_fma(-17.0 / 315.0, v, 2.0 / 15.0), v, -1.0 / 3.0);
        return __builtin_fma(a * v, p, a);
    }

    // the capped score; valid for 1 <= |cap| <= 2^20 (the range the host checks
    // exhaustively and the callers use it for), rcap = recip_rn(cap)
    MG_SF float softcap_score_fast(float x, float scale, float cap, float rcap, bool &ok)
    {
        const float q = softcap_quotient(x * scale, cap, rcap);
        const float aq = __builtin_fabsf(q);
        const double t = tanh_small_abs(double(aq));
        ok = aq >= 0x1p-99f && aq < 0x1p-5f && f32_rounding_certain(t);
        return __builtin_copysignf(float(t), q) * cap;
    }
} // namespace mgm
