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
// A lane owns Q = 16 / sizeof(out) consecutive quants (8 for bf16/f16, 4 for
// f32): one Q-byte load and one 16-byte store, so every load and store
// instruction of a wave covers one contiguous span (512 B in, 1 KiB out for
// bf16) and no cache line is written in parts. A work-group of 256 lanes
// takes U = 4 such spans per lane in flight; the grid covers the tensor
// exactly. The scale read is 2 bytes per lane, shared by the 32/Q lanes of
// its block and coalesced across the wave.
#include "mg_device.hpp"
#include "mg_internal.hpp"

namespace mg
{
    template <int Q>
    MG_DEV Vec<int8_t, Q> ld_quants(const int8_t *p)
    {
        if constexpr (Q == 8) {
            const uint64_t u = __builtin_nontemporal_load(reinterpret_cast<const uint64_t *>(p));
            return __builtin_bit_cast(Vec<int8_t, 8>, u);
        } else {
            const uint32_t u = __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(p));
            return __builtin_bit_cast(Vec<int8_t, 4>, u);
        }
    }

    template <class SO>
    __global__ __launch_bounds__(256) void k_dequant_q8_0(const int8_t *__restrict__ qs,
                                                          const uint16_t *__restrict__ d,
                                                          typename SO::raw *__restrict__ out,
                                                          int64_t nspans)
    {
        using raw = typename SO::raw;
        constexpr int Q = 16 / sizeof(raw), U = 4;
        const int64_t base = int64_t(blockIdx.x) * (256 * U) + threadIdx.x;
        Vec<int8_t, Q> q[U];
        float sc[U];
#pragma unroll
        for (int k = 0; k < U; ++k) {
            const int64_t g = base + 256 * k;
            if (g < nspans) {
                q[k] = ld_quants<Q>(qs + Q * g);
                // `in` is a multiple of 32, so span g lies in the row-major
                // [rows, in/32] scale array's block g*Q/32
                sc[k] = f16_f32(d[(g * Q) >> 5]);
            }
        }
#pragma unroll
        for (int k = 0; k < U; ++k) {
            const int64_t g = base + 256 * k;
            if (g < nspans) {
                Vec<raw, Q> o;
                if (__builtin_isfinite(sc[k])) {
                    // int8 x finite scale: finite products, no NaN to canonicalize
#pragma unroll
                    for (int e = 0; e < Q; ++e) o.v[e] = SO::enc_finite(float(q[k].v[e]) * sc[k]);
                } else {
#pragma unroll
                    for (int e = 0; e < Q; ++e) o.v[e] = SO::enc32(float(q[k].v[e]) * sc[k]);
                }
                st16_stream<raw, Q>(out + Q * g, o);
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
        const int64_t n = rows * in;
        const int Q = dt_out == F32 ? 4 : 8;
        const int64_t nspans = n / Q, blocks = (nspans + 1023) / 1024;
        need(blocks < (int64_t(1) << 31), "dequant_q8_0: tensor too large");
        const dim3 g{unsigned(blocks), 1u, 1u};
        switch (dt_out) {
        case BF16: hipLaunchKernelGGL(k_dequant_q8_0<SBf16>, g, dim3(256), 0, c->stream, qs, d, static_cast<uint16_t *>(out), nspans); break;
        case F16: hipLaunchKernelGGL(k_dequant_q8_0<SF16>, g, dim3(256), 0, c->stream, qs, d, static_cast<uint16_t *>(out), nspans); break;
        case F32: hipLaunchKernelGGL(k_dequant_q8_0<SF32>, g, dim3(256), 0, c->stream, qs, d, static_cast<float *>(out), nspans); break;
        default: fail("dequant_q8_0: output dtype must be bf16, f16 or f32");
        }
        check_launch("k_dequant_q8_0");
    }
} // namespace mg
