// Exhaustive host checks of mg_softcap_fast.hpp, the softmax kernel's capped
// score without a division, against the IEEE quotient and the oracle's FDLIBM
// tanh (fmath.hpp:389-415 restated):
//
//   quot CAP             every positive f32 s with 2^-100 < s < 2^100 (and a
//                        strided sample of negative ones): Markstein's
//                        quotient equals RN32(s / CAP) (the f64 quotient
//                        rounded to f32, an innocuous double rounding).
//                        prints "mismatches count"
//   tanh UNITS [REL]     every float a in [2^-100, 2^-5): wherever
//                        f32_rounding_certain(tanh_small_abs(a), UNITS)
//                        holds, its f32 rounding equals FDLIBM's; also the
//                        largest relative error of tanh_small_abs. REL (default
//                        0) plants a relative error in the series value, to
//                        show that the check sees errors beyond the margin.
//                        prints "accepted_bad fallbacks count maxrel"
//   score SCALE CAP STRIDE   every STRIDE-th f32 x: wherever the fast score
//                        reports ok, it equals the twin's chain
//                        rnd(cap rnd(tanh(rnd(rnd(x scale) / cap)))) bitwise.
//                        prints "accepted_bad fallbacks count"
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "mg_softcap_fast.hpp"
#include "oracle.cpp"

static float bits_f(uint32_t u)
{
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

int main(int argc, char **argv)
{
    if (argc < 2) return 2;
    long long bad = 0, fb = 0, count = 0;
    if (!std::strcmp(argv[1], "quot") && argc > 2) {
        const float cap = float(std::atof(argv[2]));
        const float rcap = mgm::recip_rn(cap); // what the kernels are given
        const int64_t lo = 0x0d800000; // 2^-100
        const int64_t hi = 0x71800000; // 2^100
#pragma omp parallel for schedule(static, 1 << 16) reduction(+ : bad, count)
        for (int64_t i = lo + 1; i < hi; ++i) {
            const float s = bits_f(uint32_t(i));
            if (mgm::softcap_quotient(s, cap, rcap) != float(double(s) / double(cap))) ++bad;
            if ((i & 255) == 0 && mgm::softcap_quotient(-s, cap, rcap) != float(double(-s) / double(cap))) ++bad;
            ++count;
        }
        std::printf("%lld %lld\n", bad, count);
        return 0;
    }
    if (!std::strcmp(argv[1], "tanh") && argc > 2) {
        const uint32_t units = uint32_t(std::atoll(argv[2]));
        const double rel = argc > 3 ? std::atof(argv[3]) : 0.0;
        const int64_t lo = 0x0d800000; // 2^-100
        const int64_t hi = 0x3d000000; // 2^-5
        double maxrel = 0.0;
#pragma omp parallel for schedule(static, 1 << 16) reduction(+ : bad, fb, count) reduction(max : maxrel)
        for (int64_t i = lo; i < hi; ++i) {
            const double a = bits_f(uint32_t(i));
            const double t = mgm::tanh_small_abs(a) * (1.0 + rel), r = orc::tanh(a);
            const double e = std::fabs(t - r) / r;
            if (e > maxrel) maxrel = e;
            if (mgm::f32_rounding_certain(t, units)) {
                if (float(t) != float(r)) ++bad;
            } else {
                ++fb;
            }
            ++count;
        }
        std::printf("%lld %lld %lld %.6e\n", bad, fb, count, maxrel);
        return 0;
    }
    if (!std::strcmp(argv[1], "score") && argc > 4) {
        const float scale = float(std::atof(argv[2])), cap = float(std::atof(argv[3]));
        const float rcap = mgm::recip_rn(cap);
        const int64_t stride = std::atoll(argv[4]);
#pragma omp parallel for schedule(static, 1 << 12) reduction(+ : bad, fb, count)
        for (int64_t i = 0; i < (int64_t(1) << 32); i += stride) {
            const float x = bits_f(uint32_t(i));
            if (x != x) continue;
            bool ok = false;
            const float got = mgm::softcap_score_fast(x, scale, cap, rcap, ok);
            // the twin: each step exact in f64, rounded to f32 (rounding.hpp)
            const float s = float(double(x) * double(scale));
            const float u = float(double(s) / double(cap));
            const float t = float(orc::tanh(double(u)));
            const float want = float(double(t) * double(cap));
            if (ok) {
                if (std::memcmp(&got, &want, 4) != 0) ++bad;
            } else {
                ++fb;
            }
            ++count;
        }
        std::printf("%lld %lld %lld\n", bad, fb, count);
        return 0;
    }
    return 2;
}
