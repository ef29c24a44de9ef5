// Q8_0 block dequantization for gfx950.
//
// Layout is the reference's QW (src/gpu/gpu_engine.cpp:120-141): int8 quants
// [rows, in] row-major and f16 scales [rows, in/32] in a separate array. Each
// output is rnd(f32(q) * f32(d)) (k_dequant_q8, src/gpu/gpu_engine.cpp:1117-1171):
// an int8 times an f16 is exact in f32 (8 + 11 significant bits), so the one
// RNE to the output format equals the twin's f64 -> f32 -> storage chain, and
// f16 subnormal scales decode exactly (v_cvt_f32_f16 keeps them,
// gpu_engine.cpp:145-151 explains why that matters).
//
// One thread owns 16 quants (one 16-byte load; the 16 never straddle a 32-block)
// and writes them as 32 bytes of bf16; four such groups are in flight per
// thread; the scale read is 2 bytes per thread, coalesced across the wave.
#include "mg_device.hpp"
#include "mg_internal.hpp"

namespace mg
{
    template <class SO>
    __global__ __launch_bounds__(256) void k_dequant_q8_0(const int8_t *__restrict__ qs,
                                                          const uint16_t *__restrict__ d,
                                                          typename SO::raw *__restrict__ out,
                                                          int64_t ngroups)
    {
        using raw = typename SO::raw;
        constexpr int U = 4;
        const int64_t stride = int64_t(gridDim.x) * blockDim.x;
        for (int64_t base = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; base < ngroups; base += stride * U) {
            Vec<int8_t, 16> q[U];
            float sc[U];
#pragma unroll
            for (int k = 0; k < U; ++k) {
                const int64_t g = base + k * stride;
                if (g < ngroups) {
                    q[k] = ld16_stream<int8_t, 16>(qs + 16 * g);
                    // `in` is a multiple of 32, so group g's 32-block is g / 2 in
                    // the row-major [rows, in/32] scale array
                    sc[k] = f16_f32(d[g >> 1]);
                }
            }
#pragma unroll
            for (int k = 0; k < U; ++k) {
                const int64_t g = base + k * stride;
                if (g < ngroups) {
                    raw o[16];
                    if (__builtin_isfinite(sc[k])) {
                        // int8 x finite scale: finite products, no NaN to canonicalize
#pragma unroll
                        for (int e = 0; e < 16; ++e) o[e] = SO::enc_finite(float(q[k].v[e]) * sc[k]);
                    } else {
#pragma unroll
                        for (int e = 0; e < 16; ++e) o[e] = SO::enc32(float(q[k].v[e]) * sc[k]);
                    }
                    constexpr int V = 16 / sizeof(raw);
#pragma unroll
                    for (int p = 0; p < 16 / V; ++p) {
                        Vec<raw, V> w;
#pragma unroll
                        for (int e = 0; e < V; ++e) w.v[e] = o[p * V + e];
                        st16_stream<raw, V>(out + 16 * g + p * V, w);
                    }
                }
            }
        }
    }

    void launch_dequant_q8_0(mg_ctx *c, const int8_t *qs, const uint16_t *d, void *out,
                             int64_t rows, int64_t in, int dt_out)
    {
        need(rows >= 0 && in >= 0, "dequant_q8_0: bad shape");
        need(in % 32 == 0, "dequant_q8_0: input dim must be a multiple of 32 (got " + std::to_string(in) + ")");
        need(qs && d && out, "dequant_q8_0: NULL tensor");
        need(aligned16(qs) && aligned16(out), "dequant_q8_0: quants and output must be 16-byte aligned");
        if (rows == 0 || in == 0) return;
        const int64_t ngroups = rows * (in / 16);
        const unsigned blocks = unsigned(std::min<int64_t>((ngroups + 1023) / 1024, int64_t(c->num_cus) * 32));
        switch (dt_out) {
        case BF16: hipLaunchKernelGGL(k_dequant_q8_0<SBf16>, dim3(blocks), dim3(256), 0, c->stream, qs, d, static_cast<uint16_t *>(out), ngroups); break;
        case F16: hipLaunchKernelGGL(k_dequant_q8_0<SF16>, dim3(blocks), dim3(256), 0, c->stream, qs, d, static_cast<uint16_t *>(out), ngroups); break;
        case F32: hipLaunchKernelGGL(k_dequant_q8_0<SF32>, dim3(blocks), dim3(256), 0, c->stream, qs, d, static_cast<float *>(out), ngroups); break;
        default: fail("dequant_q8_0: output dtype must be bf16, f16 or f32");
        }
        check_launch("k_dequant_q8_0");
    }
} // namespace mg
