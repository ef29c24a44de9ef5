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
// bf16) and no cache line is written in parts. A work-group is one wave
// (measured faster than four) with U = 2 such spans per lane in flight; the
// grid covers the tensor exactly. The scale read is 2 bytes per lane, shared by the 32/Q lanes of
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

    constexpr int kDequantSpans = 2; // spans per lane (measured: 1 and 2 beat 4 and 8)

    template <class SO>
    __global__ __launch_bounds__(64) void k_dequant_q8_0(const int8_t *__restrict__ qs,
                                                          const uint16_t *__restrict__ d,
                                                          typename SO::raw *__restrict__ out,
                                                          int64_t nspans)
    {
        using raw = typename SO::raw;
        constexpr int Q = 16 / sizeof(raw), U = kDequantSpans;
        const int64_t base = int64_t(blockIdx.x) * (64 * U) + threadIdx.x;
        Vec<int8_t, Q> q[U];
        float sc[U];
#pragma unroll
        for (int k = 0; k < U; ++k) {
            const int64_t g = base + 64 * k;
            if (g < nspans) {
                q[k] = ld_quants<Q>(qs + Q * g);
                // `in` is a multiple of 32, so span g lies in the row-major
                // [rows, in/32] scale array's block g*Q/32
                sc[k] = f16_f32(d[(g * Q) >> 5]);
            }
        }
#pragma unroll
        for (int k = 0; k < U; ++k) {
            const int64_t g = base + 64 * k;
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

    // 16-bit outputs over whole 1 KiB chunks of quants, one chunk a wave: lane L
    // loads quants 16L..16L+15 (one 16-byte load, so each load instruction
    // reads 1 KiB where the 8-quant lanes above read 512 B), then takes the 8
    // quants of outputs 8L.. and 512 + 8L.. from lanes L/2 and 32 + L/2
    // (ds_bpermute, no LDS storage), so each of the two 16-byte stores still
    // writes 1 KiB contiguously. The scale of outputs 8L.. is block L/4 of the
    // chunk's 32, that of 512 + 8L.. block 16 + L/4: loaded by the lane itself.
    template <class SO>
    __global__ __launch_bounds__(64) void k_dequant_q8_0_wide(const int8_t *__restrict__ qs,
                                                               const uint16_t *__restrict__ d,
                                                               uint16_t *__restrict__ out)
    {
        const int lane = threadIdx.x;
        const int64_t ch = blockIdx.x;
        const Vec<uint32_t, 4> qv = ld16_stream<uint32_t, 4>(reinterpret_cast<const uint32_t *>(qs + 1024 * ch + 16 * lane));
        const float sa = f16_f32(d[ch * 32 + (lane >> 2)]);
        const float sb = f16_f32(d[ch * 32 + 16 + (lane >> 2)]);
        // source lanes' words j, then the half (h) this lane's outputs take
        const int h = lane & 1, srcA = (lane >> 1) * 4, srcB = (32 + (lane >> 1)) * 4;
        uint32_t wa[4], wb[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            wa[j] = uint32_t(__builtin_amdgcn_ds_bpermute(srcA, int(qv.v[j])));
            wb[j] = uint32_t(__builtin_amdgcn_ds_bpermute(srcB, int(qv.v[j])));
        }
        const Vec<int8_t, 8> qa = __builtin_bit_cast(Vec<int8_t, 8>, Vec<uint32_t, 2>{{h ? wa[2] : wa[0], h ? wa[3] : wa[1]}});
        const Vec<int8_t, 8> qb = __builtin_bit_cast(Vec<int8_t, 8>, Vec<uint32_t, 2>{{h ? wb[2] : wb[0], h ? wb[3] : wb[1]}});
        Vec<uint16_t, 8> oa, ob;
        if (__builtin_isfinite(sa) && __builtin_isfinite(sb)) {
            // int8 x finite scale: finite products, no NaN to canonicalize
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                oa.v[e] = SO::enc_finite(float(qa.v[e]) * sa);
                ob.v[e] = SO::enc_finite(float(qb.v[e]) * sb);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                oa.v[e] = SO::enc32(float(qa.v[e]) * sa);
                ob.v[e] = SO::enc32(float(qb.v[e]) * sb);
            }
        }
        uint16_t *o = out + 1024 * ch;
        st16_stream<uint16_t, 8>(o + 8 * lane, oa);
        st16_stream<uint16_t, 8>(o + 512 + 8 * lane, ob);
    }

    // ------------------------------------------------------------ quantizer
    // up_w (src/gpu/gpu_engine.cpp:2722-2755), the llama.cpp quantize_row_q8_0
    // rule: per 32-block, amax = max |x| over the bf16 values, d = amax / 127
    // (f32), id = d ? 1/d : 0, the scale stored as f16 (RNE, subnormals kept,
    // f32_to_f16 at 152-158), q = lround(x * id) (half away from zero).
    // A wave takes 64 consecutive blocks (2048 weights): in step k, lane L
    // holds weights 512k + 8L .. +7, so the four lanes of a quad hold one
    // block and amax is a quad reduction; every load instruction reads 1 KiB
    // and every store instruction writes 512 contiguous bytes of quants, and
    // the wave's 64 scales go out in one 128-byte store.
    MG_DEV float quad_max(float v)
    {
        v = __builtin_fmaxf(v, dpp_mov<0xB1, 0xf>(v, v)); // quad_perm [1,0,3,2]
        v = __builtin_fmaxf(v, dpp_mov<0x4E, 0xf>(v, v)); // quad_perm [2,3,0,1]
        return v;
    }

    __global__ __launch_bounds__(64) void k_quantize_q8_0(const uint16_t *__restrict__ w, int8_t *__restrict__ qs,
                                                           uint16_t *__restrict__ d, int64_t nblk)
    {
        const int lane = threadIdx.x & 63;
        const int64_t b0 = int64_t(blockIdx.x) * 64; // the wave's (= work-group's) first block
        if (b0 >= nblk) return;
        Vec<uint16_t, 8> v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            v[k] = Vec<uint16_t, 8>{};
            if (b0 + 16 * k + (lane >> 2) < nblk) v[k] = ld16_stream<uint16_t, 8>(w + b0 * 32 + 512 * k + 8 * lane);
        }
        uint16_t my_scale = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int64_t b = b0 + 16 * k + (lane >> 2);
            float x[8], amax = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                x[e] = bf16_f32(v[k].v[e]);
                amax = __builtin_fmaxf(amax, __builtin_fabsf(x[e]));
            }
            amax = quad_max(amax);
            const float dd = amax / 127.0f;
            const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
            const uint16_t dh = __builtin_bit_cast(uint16_t, static_cast<_Float16>(dd));
            // gather the scales so that lane j holds block b0 + j's
            const uint16_t s = uint16_t(__shfl(int(dh), 4 * (lane & 15), 64));
            if ((lane >> 4) == k) my_scale = s;
            if (b < nblk) {
                uint64_t q = 0;
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    q |= uint64_t(uint8_t(int8_t(int(__builtin_roundf(x[e] * id))))) << (8 * e);
                __builtin_nontemporal_store(q, reinterpret_cast<uint64_t *>(qs + b0 * 32 + 512 * k + 8 * lane));
            }
        }
        if (b0 + lane < nblk) d[b0 + lane] = my_scale;
    }

    void launch_quantize_q8_0(mg_ctx *c, const uint16_t *w, int64_t rows, int64_t in, int8_t *qs, uint16_t *d)
    {
        need(rows >= 0 && in >= 0, "quantize_q8_0: bad shape");
        need(in % 32 == 0, "quantize_q8_0: input dim must be a multiple of 32 (got " + std::to_string(in) + ")");
        need(w && qs && d, "quantize_q8_0: NULL tensor");
        need(aligned16(w) && aligned16(qs), "quantize_q8_0: weights and quants must be 16-byte aligned");
        const int64_t nblk = rows * (in / 32);
        if (nblk == 0) return;
        const int64_t waves = (nblk + 63) / 64;
        need(waves <= int64_t(0x7fffffff), "quantize_q8_0: tensor too large");
        hipLaunchKernelGGL(k_quantize_q8_0, dim3(unsigned(waves)), dim3(64), 0, c->stream, w, qs, d, nblk);
        check_launch("k_quantize_q8_0");
    }

    // ----------------------------------------------------------- Q8_0 GEMV
    // y[b, o] = sum_i w[o, i] * x[b, i] over a Q8_0 weight, as k_gemv_q8
    // (src/gpu/gpu_engine.cpp:815-889) defines it: by default every weight is
    // first materialized as bf16(q * d) (so decode agrees with a prefill that
    // dequantizes), with the BLOCKDOT form sum_blocks d * sum(q * x) behind a
    // flag (llama.cpp's Q8_0 dot). f32 accumulation in both.
    // One wave per output row, 16 quants (one 16-byte load) per lane and step.
    // q * d is formed as fma(u, d, -128 d) on the biased byte u = q + 128
    // (exact, the same rounding as the product), rounded to bf16 in pairs, and
    // dotted with the bf16 activations by v_dot2_f32_bf16.
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

    template <int B, bool BLOCKDOT>
    __global__ __launch_bounds__(256) void k_gemv_q8_0(const int8_t *__restrict__ W, const uint16_t *__restrict__ D,
                                                       const uint16_t *__restrict__ X, float *__restrict__ Y,
                                                       int64_t in, int64_t out, int64_t ldx, int64_t ldy)
    {
        const int64_t o = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
        const int lane = threadIdx.x & 63;
        if (o >= out) return;
        const int8_t *w = W + o * in;
        const uint16_t *dd = D + o * (in / 32);
        float part[B];
#pragma unroll
        for (int bb = 0; bb < B; ++bb) part[bb] = 0.0f;
        const int64_t nc = in / 16;
        for (int64_t c = lane; c < nc; c += 64) {
            const Vec<uint32_t, 4> qv = ld16_stream<uint32_t, 4>(reinterpret_cast<const uint32_t *>(w + 16 * c));
            const float sc = f16_f32(dd[c >> 1]);
            if constexpr (!BLOCKDOT) {
                const float nsc = -128.0f * sc;
                uint32_t wb[8]; // bf16(q * d) in pairs
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const uint32_t u = qv.v[k] ^ 0x80808080u; // q + 128 in each byte
                    const float f0 = __builtin_fmaf(float(u & 0xffu), sc, nsc);
                    const float f1 = __builtin_fmaf(float((u >> 8) & 0xffu), sc, nsc);
                    const float f2 = __builtin_fmaf(float((u >> 16) & 0xffu), sc, nsc);
                    const float f3 = __builtin_fmaf(float(u >> 24), sc, nsc);
                    wb[2 * k] = uint32_t(__builtin_bit_cast(uint16_t, static_cast<__bf16>(f0))) |
                                (uint32_t(__builtin_bit_cast(uint16_t, static_cast<__bf16>(f1))) << 16);
                    wb[2 * k + 1] = uint32_t(__builtin_bit_cast(uint16_t, static_cast<__bf16>(f2))) |
                                    (uint32_t(__builtin_bit_cast(uint16_t, static_cast<__bf16>(f3))) << 16);
                }
#pragma unroll
                for (int bb = 0; bb < B; ++bb) {
                    const uint32_t *xr = reinterpret_cast<const uint32_t *>(X + bb * ldx + 16 * c);
                    const Vec<uint32_t, 4> x0 = *reinterpret_cast<const Vec<uint32_t, 4> *>(xr);
                    const Vec<uint32_t, 4> x1 = *reinterpret_cast<const Vec<uint32_t, 4> *>(xr + 4);
                    float acc = part[bb];
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, wb[k]),
                                                              __builtin_bit_cast(bf16x2, x0.v[k]), acc, false);
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, wb[4 + k]),
                                                              __builtin_bit_cast(bf16x2, x1.v[k]), acc, false);
                    part[bb] = acc;
                }
            } else {
                const Vec<int8_t, 16> q = __builtin_bit_cast(Vec<int8_t, 16>, qv);
#pragma unroll
                for (int bb = 0; bb < B; ++bb) {
                    const Vec<uint16_t, 8> x0 = *reinterpret_cast<const Vec<uint16_t, 8> *>(X + bb * ldx + 16 * c);
                    const Vec<uint16_t, 8> x1 = *reinterpret_cast<const Vec<uint16_t, 8> *>(X + bb * ldx + 16 * c + 8);
                    float acc = 0.0f;
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc = __builtin_fmaf(float(q.v[e]), bf16_f32(x0.v[e]), acc);
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc = __builtin_fmaf(float(q.v[8 + e]), bf16_f32(x1.v[e]), acc);
                    part[bb] = __builtin_fmaf(acc, sc, part[bb]);
                }
            }
        }
#pragma unroll
        for (int bb = 0; bb < B; ++bb) {
            const float s = dpp_sum_f32(part[bb]);
            if (lane == 0) Y[bb * ldy + o] = s;
        }
    }

    void launch_gemv_q8_0(mg_ctx *c, const int8_t *qs, const uint16_t *d, const uint16_t *x, int64_t batch,
                          int64_t rows, int64_t in, int64_t ldx, float *y, int64_t ldy, bool blockdot)
    {
        need(rows >= 0 && in >= 0 && batch >= 1 && batch <= 8, "gemv_q8_0: batch must be in [1, 8]");
        need(in % 32 == 0, "gemv_q8_0: input dim must be a multiple of 32 (got " + std::to_string(in) + ")");
        need(qs && d && x && y, "gemv_q8_0: NULL tensor");
        if (ldx == 0) ldx = in;
        if (ldy == 0) ldy = rows;
        need(ldx >= in && ldy >= rows, "gemv_q8_0: leading dimension too small");
        need(aligned16(qs) && aligned16(x) && ldx % 8 == 0, "gemv_q8_0: quants and activations must be 16-byte aligned");
        if (rows == 0) return;
        need(rows < (int64_t(1) << 33), "gemv_q8_0: too many rows");
        const dim3 g{unsigned((rows + 3) / 4), 1u, 1u};
        // up to four activation rows per pass over the weights
        for (int64_t b0 = 0; b0 < batch; b0 += 4) {
            const int nb = int(batch - b0 < 4 ? batch - b0 : 4);
            const uint16_t *xb = x + b0 * ldx;
            float *yb = y + b0 * ldy;
            auto go = [&](auto kern) {
                hipLaunchKernelGGL(kern, g, dim3(256), 0, c->stream, qs, d, xb, yb, in, rows, ldx, ldy);
            };
            switch (nb * 2 + (blockdot ? 1 : 0)) {
            case 2: go(k_gemv_q8_0<1, false>); break;
            case 3: go(k_gemv_q8_0<1, true>); break;
            case 4: go(k_gemv_q8_0<2, false>); break;
            case 5: go(k_gemv_q8_0<2, true>); break;
            case 6: go(k_gemv_q8_0<3, false>); break;
            case 7: go(k_gemv_q8_0<3, true>); break;
            case 8: go(k_gemv_q8_0<4, false>); break;
            default: go(k_gemv_q8_0<4, true>); break;
            }
        }
        check_launch("k_gemv_q8_0");
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
        const int64_t nspans = n / Q, blocks = (nspans + 64 * kDequantSpans - 1) / (64 * kDequantSpans);
        need(blocks < (int64_t(1) << 31), "dequant_q8_0: tensor too large");
        const dim3 g{unsigned(blocks), 1u, 1u};
        if ((dt_out == BF16 || dt_out == F16) && n % 1024 == 0 && n / 1024 < (int64_t(1) << 31)) {
            const dim3 gw{unsigned(n / 1024), 1u, 1u};
            uint16_t *o = static_cast<uint16_t *>(out);
            if (dt_out == BF16)
                hipLaunchKernelGGL(k_dequant_q8_0_wide<SBf16>, gw, dim3(64), 0, c->stream, qs, d, o);
            else
                hipLaunchKernelGGL(k_dequant_q8_0_wide<SF16>, gw, dim3(64), 0, c->stream, qs, d, o);
            check_launch("k_dequant_q8_0_wide");
            return;
        }
        switch (dt_out) {
        case BF16: hipLaunchKernelGGL(k_dequant_q8_0<SBf16>, g, dim3(64), 0, c->stream, qs, d, static_cast<uint16_t *>(out), nspans); break;
        case F16: hipLaunchKernelGGL(k_dequant_q8_0<SF16>, g, dim3(64), 0, c->stream, qs, d, static_cast<uint16_t *>(out), nspans); break;
        case F32: hipLaunchKernelGGL(k_dequant_q8_0<SF32>, g, dim3(64), 0, c->stream, qs, d, static_cast<float *>(out), nspans); break;
        default: fail("dequant_q8_0: output dtype must be bf16, f16 or f32");
        }
        check_launch("k_dequant_q8_0");
    }
} // namespace mg
