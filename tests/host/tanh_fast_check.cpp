// Exhaustive host check of mgm::tanh_fast_abs (the output tail's fast tanh)
// against the oracle's FDLIBM tanh (fmath.hpp:389-415 restated), over every
// float input a in [0, 22) (the tail only ever applies tanh to stored values,
// and every f32, bf16 and f16 value is a float), plus values >= 22 and inf.
// For each input: the relative error of the fast value, and, for f32, bf16
// and f16 storage, that whenever t(1 -+ margin) round to one stored value,
// FDLIBM's result rounds to it too.
//
// usage: tanh_fast_check [stride [margin [perturb]]]   prints "maxrel accepted_bad fb_f32 fb_bf16 fb_f16 count"
// (perturb: a relative error planted in the fast value, to show the check catches one)
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "mg_tanh_fast.hpp"
#include "oracle.cpp"

int main(int argc, char **argv)
{
    const int64_t stride = argc > 1 ? std::atoll(argv[1]) : 1;
    const int64_t end = 0x41B00000; // 22.0f
    const double m = argc > 2 ? std::atof(argv[2]) : mgm::kTanhFastMargin;
    const double perturb = argc > 3 ? std::atof(argv[3]) : 0.0;
    long long bad = 0, fb32 = 0, fbb = 0, fbh = 0, count = 0;
    double maxrel = 0.0;
#pragma omp parallel for schedule(static, 1 << 16) reduction(+ : bad, fb32, fbb, fbh, count) reduction(max : maxrel)
    for (int64_t i = 0; i < end; i += stride) {
        const uint32_t u = uint32_t(i);
        float f;
        std::memcpy(&f, &u, 4);
        const double a = f;
        const double t = mgm::tanh_fast_abs(a) * (1.0 + perturb), r = orc::tanh(a);
        const double rel = r == 0.0 ? std::fabs(t - r) : std::fabs(t - r) / r;
        if (rel > maxrel) maxrel = rel;
        double lo, hi;
        mgm::tanh_interval(t, lo, hi, m);
        if (float(lo) == float(hi)) {
            if (float(lo) != float(r)) ++bad;
        } else {
            ++fb32;
        }
        if (orc::bf16_bits(lo) == orc::bf16_bits(hi)) {
            if (orc::bf16_bits(lo) != orc::bf16_bits(r)) ++bad;
        } else {
            ++fbb;
        }
        if (orc::f16_bits(lo) == orc::f16_bits(hi)) {
            if (orc::f16_bits(lo) != orc::f16_bits(r)) ++bad;
        } else {
            ++fbh;
        }
        ++count;
    }
    const double big[] = {22.0, 22.5, 100.0, 65504.0, 3.0e38, INFINITY};
    for (double a : big)
        if (mgm::tanh_fast_abs(a) != orc::tanh(a)) ++bad;
    std::printf("%.6e %lld %lld %lld %lld %lld\n", maxrel, bad, fb32, fbb, fbh, count);
    return 0;
}
