// Fused QK-norm + qk-scale + RoPE + KV-cache append for gfx950: the caller
// sequence around RoPE, one pass over q and k.
//
// Reference sequence (src/muse_glimmer.hpp:799-819; GPU engine
// src/gpu/gpu_engine.cpp:4339-4350 and k_kv_append 481-492):
//   q[t,h,:] = rnd(q * rs)            weight-less rmsnorm_rows over head_dim
//   k[t,g,:] = rnd(k * rs)            (rs = 1/sqrt(mean_sq + eps) per head row)
//   q        = rnd(q * qk_scale)      q only; qk_scale an f32 value outside f64
//   q, k     = apply_rope(., table row pos)   when a table is given
//   k_cache[pos % slots, g, :] = k,  v_cache[pos % slots, g, :] = v
// Each step materializes at storage exactly as the separate primitives do, so
// the result is bit-identical to running mg_rmsnorm_rows, mg_scale, mg_rope and
// the two cache copies one after the other.
//
// Each wave takes 8 head rows (of q and k alike) on its own, with no
// work-group barrier: the rows are staged in the wave's part of LDS with
// 16-byte loads; eight lanes per row run mean_sq's eight interleaved f64
// accumulators in the reference order and its fixed tree (bit-identical rs);
// then every lane takes (lo, hi) pairs of a row: normalize, scale, rotate,
// store back and append to the caches. With the f32-compat flag (f64 storage)
// the norm takes the f32 chain of rmsnorm_rows (src/muse_glimmer.hpp:530-556,
// 581-594): f32 accumulators in the same order and tree, rs = 1.0f/sqrtf(ms),
// x = double(float(x) * rs); the scale and the rotation stay f64.
#include <type_traits>

#include "mg_device.hpp"
#include "mg_internal.hpp"

namespace mg
{
    constexpr int kQkRows = 32;    // head rows per work-group
    constexpr int kQkWaveRows = 8; // head rows per wave (eight lanes per row for mean_sq)
    constexpr int kQkPieces = 1;   // k_qk_pairs: 8-element pieces per lane in each half of a row

    struct QkArgs
    {
        int64_t nq, nkv, ldq, ldk, ldv, T, table_rows, pos0, slots;
        int D;
        double eps;
    };

    template <class S, int VEC, bool C>
    __global__ __launch_bounds__(256) void k_qk_norm_rope(typename S::raw *q, typename S::raw *k,
                                                          const typename S::raw *__restrict__ v, QkArgs a,
                                                          typename S::comp qs,
                                                          const typename S::raw *__restrict__ co,
                                                          const typename S::raw *__restrict__ si,
                                                          const int64_t *__restrict__ pos,
                                                          typename S::raw *kc, typename S::raw *vc)
    {
        using raw = typename S::raw;
        extern __shared__ double smem_d[];
        double *rsq = smem_d;                                 // [kQkRows]
        raw *st = reinterpret_cast<raw *>(smem_d + kQkRows); // [kQkRows][SD]
        const int D = a.D, half = D / 2;
        const int SD = D + 16 / int(sizeof(raw)); // row stride: 16 bytes of padding against bank conflicts
        const int64_t heads = a.nq + a.nkv, rows = a.T * heads;
        // each wave owns kQkWaveRows rows of the group's kQkRows and works on
        // them alone: no work-group barrier anywhere
        const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
        const int64_t r0 = int64_t(blockIdx.x) * kQkRows + wv * kQkWaveRows;
        if (r0 >= rows) return; // the whole wave
        const int nr = int(rows - r0 < kQkWaveRows ? rows - r0 : kQkWaveRows);
        const int w0 = wv * kQkWaveRows; // the wave's slots in the per-row arrays
        // per row, once: its address, table position, and the cache row it
        // appends to (k rows with a cache and a position >= 0), or -1
        __shared__ raw *rptr[kQkRows];
        __shared__ const raw *vptr[kQkRows];
        __shared__ int64_t rpos[kQkRows], rcache[kQkRows];
        __shared__ int risq[kQkRows];
        if (lane < nr) {
            const int64_t r = r0 + lane, t = r / heads, hh = r - t * heads;
            const int64_t p = pos ? pos[t] : a.pos0 + t;
            const bool isq = hh < a.nq;
            rptr[w0 + lane] = isq ? q + t * a.ldq + hh * D : k + t * a.ldk + (hh - a.nq) * D;
            vptr[w0 + lane] = isq || !v ? nullptr : v + t * a.ldv + (hh - a.nq) * D;
            rpos[w0 + lane] = p;
            risq[w0 + lane] = isq;
            rcache[w0 + lane] = !isq && kc && p >= 0 ? (p % a.slots) * (a.nkv * D) + (hh - a.nq) * D : -1;
        }
        wave_lds_sync();

        // stage the head rows
        const int vpr = D / VEC;
        for (int idx = lane; idx < nr * vpr; idx += 64) {
            const int rr = w0 + idx / vpr, i = (idx - (rr - w0) * vpr) * VEC;
            *reinterpret_cast<Vec<raw, VEC> *>(st + rr * SD + i) = *reinterpret_cast<const Vec<raw, VEC> *>(rptr[rr] + i);
        }
        wave_lds_sync();

        // mean_sq (src/muse_glimmer.hpp:509-527): lane l of a row's 8-lane
        // group owns accumulator a_l
        {
            const int rr = w0 + (lane >> 3), l = lane & 7;
            const int full = D & ~7;
            // the accumulator type: f64 (mean_sq), f32 for the compat chain (mean_sq_f32)
            using acc_t = std::conditional_t<C, float, double>;
            acc_t acc = 0;
            if (rr < w0 + nr)
                for (int i = l; i < full; i += 8) {
                    const acc_t x = acc_t(S::dec(st[rr * SD + i]));
                    acc = acc + x * x;
                }
            const acc_t s1 = acc + __shfl_xor(acc, 1, 64);
            const acc_t s2 = s1 + __shfl_xor(s1, 2, 64);
            const acc_t s3 = s2 + __shfl_xor(s2, 4, 64);
            if (rr < w0 + nr && l == 0) {
                acc_t tail = 0;
                for (int i = full; i < D; ++i) {
                    const acc_t x = acc_t(S::dec(st[rr * SD + i]));
                    tail = tail + x * x;
                }
                if constexpr (C) {
                    // f32 quotient, sum, sqrt and reciprocal, each correctly
                    // rounded (the f64 operation rounded to f32: 53 >= 2*24 + 2)
                    const float ms = float(double(s3 + tail) / double(D)) + float(a.eps);
                    const float sq = float(__builtin_sqrt(double(ms)));
                    rsq[rr] = double(float(1.0 / double(sq)));
                } else {
                    rsq[rr] = 1.0 / __builtin_sqrt((s3 + tail) / double(D) + a.eps);
                }
            }
        }
        // x * rs: f64 (or at the storage format), f32 in the compat chain
        auto nrm = [](typename S::raw x, double rs) -> typename S::raw {
            if constexpr (C)
                return S::enc64(double(float(S::dec(x)) * float(rs)));
            else
                return S::enc64(double(S::dec(x)) * rs);
        };
        wave_lds_sync();

        // (lo, hi) pairs, VEC at a time when the halves allow 16-byte
        // accesses: normalize, scale q, rotate, store, append
        constexpr int PV = VEC;
        const int npv = half % PV == 0 ? half / PV : 0;
        if (npv) {
            for (int idx = lane; idx < nr * npv; idx += 64) {
                const int rr = w0 + idx / npv, j = (idx - (rr - w0) * npv) * PV;
                const bool isq = risq[rr] != 0;
                const double rs = rsq[rr];
                Vec<raw, PV> lo = *reinterpret_cast<const Vec<raw, PV> *>(st + rr * SD + j);
                Vec<raw, PV> hi = *reinterpret_cast<const Vec<raw, PV> *>(st + rr * SD + j + half);
                const int64_t p = rpos[rr];
                const bool rot = co && p >= 0 && p < a.table_rows;
                Vec<raw, PV> cv, sv;
                if (rot) {
                    cv = *reinterpret_cast<const Vec<raw, PV> *>(co + p * half + j);
                    sv = *reinterpret_cast<const Vec<raw, PV> *>(si + p * half + j);
                }
                if constexpr (S::dt == BF16) {
                    // bf16: NaN propagates through every step and the twin's NaN
                    // is the single pattern 0x7FC0, so the steps round without
                    // NaN checks and the outputs are made canonical once
                    auto rn = [](float f) { return SBf16::enc_finite(f); };
#pragma unroll
                    for (int e = 0; e < PV; ++e) {
                        raw l = rn(float(double(S::dec(lo.v[e])) * rs));
                        raw h = rn(float(double(S::dec(hi.v[e])) * rs));
                        if (isq) {
                            l = rn(S::dec(l) * qs);
                            h = rn(S::dec(h) * qs);
                        }
                        if (rot) {
                            const float fl = S::dec(l), fh = S::dec(h), cc = S::dec(cv.v[e]), ss = S::dec(sv.v[e]);
                            l = rn(S::dec(rn(fl * cc)) + S::dec(rn(-(fh * ss))));
                            h = rn(S::dec(rn(fh * cc)) + S::dec(rn(fl * ss)));
                        }
                        lo.v[e] = S::dec(l) != S::dec(l) ? raw(0x7fc0) : l;
                        hi.v[e] = S::dec(h) != S::dec(h) ? raw(0x7fc0) : h;
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < PV; ++e) {
                        raw l = nrm(lo.v[e], rs);
                        raw h = nrm(hi.v[e], rs);
                        if (isq) {
                            l = S::enc(S::dec(l) * qs);
                            h = S::enc(S::dec(h) * qs);
                        }
                        if (rot) rope_pair<S>(l, h, cv.v[e], sv.v[e]);
                        lo.v[e] = l;
                        hi.v[e] = h;
                    }
                }
                raw *dst = rptr[rr];
                stv<raw, PV>(dst + j, lo);
                stv<raw, PV>(dst + j + half, hi);
                const int64_t o = rcache[rr];
                if (o >= 0) {
                    stv<raw, PV>(kc + o + j, lo);
                    stv<raw, PV>(kc + o + j + half, hi);
                    if (vc) {
                        const raw *vr = vptr[rr];
                        stv<raw, PV>(vc + o + j, ldv<raw, PV>(vr + j));
                        stv<raw, PV>(vc + o + j + half, ldv<raw, PV>(vr + j + half));
                    }
                }
            }
            return;
        }
        for (int idx = lane; idx < nr * half; idx += 64) {
            const int rr = w0 + idx / half, j = idx - (rr - w0) * half;
            const bool isq = risq[rr] != 0;
            const double rs = rsq[rr];
            raw lo = nrm(st[rr * SD + j], rs);
            raw hi = nrm(st[rr * SD + j + half], rs);
            if (isq) {
                lo = S::enc(S::dec(lo) * qs);
                hi = S::enc(S::dec(hi) * qs);
            }
            const int64_t p = rpos[rr];
            if (co && p >= 0 && p < a.table_rows) rope_pair<S>(lo, hi, co[p * half + j], si[p * half + j]);
            raw *dst = rptr[rr];
            dst[j] = lo;
            dst[j + half] = hi;
            const int64_t o = rcache[rr];
            if (o >= 0) {
                kc[o + j] = lo;
                kc[o + j + half] = hi;
                if (vc) {
                    const raw *vr = vptr[rr];
                    vc[o + j] = vr[j];
                    vc[o + j + half] = vr[j + half];
                }
            }
        }
    }

    // 16-bit storage with head_dim 64, 128 or 256: RoPE's layout, each lane
    // holding NV 8-element pieces of the first half and the matching pieces of
    // the second (TPR = head_dim / (16 NV) lanes per head row), no LDS on the
    // common path; more elements per lane spread the per-row work (the
    // reduction, rs, addresses) over more of them.
    // Sum of squares: the square of a stored value is exact in f64 and a
    // multiple of the smallest nonzero square's last bit u; when the sum stays
    // below 2^53 u every partial sum in any order is exact, so a butterfly over
    // the row's lanes gives mean_sq's bits. A wave with a row outside that
    // bound (or holding inf or NaN) stages its rows in LDS and runs mean_sq's
    // own order (eight interleaved accumulators, fixed tree).
    template <class S, int D, int NV>
    __global__ __launch_bounds__(256) void k_qk_pairs(typename S::raw *q, typename S::raw *k,
                                                      const typename S::raw *__restrict__ v, QkArgs a,
                                                      typename S::comp qs,
                                                      const typename S::raw *__restrict__ co,
                                                      const typename S::raw *__restrict__ si,
                                                      const int64_t *__restrict__ pos, typename S::raw *kc,
                                                      typename S::raw *vc)
    {
        using raw = typename S::raw;
        using W4 = Vec<uint32_t, 4>;
        constexpr int VEC = 8, TPR = D / (16 * NV), half = D / 2, RPW = 64 / TPR, NH = NV * VEC;
        constexpr int MB = S::dt == BF16 ? 7 : 10;              // stored mantissa bits
        constexpr int BIAS = S::dt == BF16 ? 127 : 15;          // exponent bias
        static_assert(TPR >= 2 && TPR <= 16 && TPR * 16 * NV == D, "lanes per row");
        __shared__ __align__(16) raw st[4][RPW][D + 8];
        __shared__ double rsf[4][RPW];
        const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
        const int64_t heads = a.nq + a.nkv, rows = a.T * heads;
        const int64_t wrow0 = (int64_t(blockIdx.x) * 256 + wv * 64) / TPR; // the wave's first row
        if (wrow0 >= rows) return; // the whole wave
        const int64_t r = wrow0 + lane / TPR;
        const int j = lane & (TPR - 1);
        const bool live = r < rows;
        const int64_t rc = live ? r : rows - 1; // addresses of a dead lane stay in bounds
        const int64_t t = rows <= int64_t(0xffffffff) ? int64_t(uint32_t(rc) / uint32_t(heads)) : rc / heads;
        const int hh = int(rc - t * heads);
        const bool isq = hh < a.nq;
        raw *x = isq ? q + t * a.ldq + int64_t(hh) * D : k + t * a.ldk + int64_t(hh - a.nq) * D;
        const int c0 = NH * j; // the lane's first column of each half
        Vec<raw, VEC> lo[NV], hi[NV];
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            lo[i] = ldv<raw, VEC>(x + c0 + VEC * i);
            hi[i] = ldv<raw, VEC>(x + half + c0 + VEC * i);
        }
        const int64_t p = pos ? pos[t] : a.pos0 + t;
        Vec<raw, VEC> vlo[NV], vhi[NV];
        if (!isq && vc && p >= 0) {
            const raw *vr = v + t * a.ldv + int64_t(hh - a.nq) * D + c0;
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                vlo[i] = ldv<raw, VEC>(vr + VEC * i);
                vhi[i] = ldv<raw, VEC>(vr + half + VEC * i);
            }
        }
        const bool rot = co && p >= 0 && p < a.table_rows;
        Vec<raw, VEC> cv[NV], sv[NV];
        if (rot) {
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                cv[i] = *reinterpret_cast<const Vec<raw, VEC> *>(co + p * half + c0 + VEC * i);
                sv[i] = *reinterpret_cast<const Vec<raw, VEC> *>(si + p * half + c0 + VEC * i);
            }
        }

        double ss = 0.0;
#pragma unroll
        for (int e = 0; e < 2 * NH; ++e) {
            const double d = double(S::dec(e < NH ? lo[e / VEC].v[e % VEC] : hi[(e - NH) / VEC].v[e % VEC]));
            ss = __builtin_fma(d, d, ss); // d * d is exact: the same sum as ss + d * d
        }
        // smallest nonzero magnitude over the lane's values, two halves per
        // packed step (zero wraps to 0xFFFF; an all-zero lane ends at
        // 0x10000 >> MB, above every exponent field)
        uint32_t umin = 0xffffffffu;
#pragma unroll
        for (int w = 0; w < 8 * NV; ++w) {
            const uint32_t m =
                (w < 4 * NV ? __builtin_bit_cast(W4, lo[w / 4]).v[w % 4] : __builtin_bit_cast(W4, hi[w / 4 - NV]).v[w % 4]) &
                0x7fff7fffu;
            umin = pk_min_u16(umin, pk_dec_u16(m));
        }
        int emin = max(int((min(umin & 0xffffu, umin >> 16) + 1) >> MB), 1);
        // over the row's TPR lanes (a lane pair, quad, half-row or row of the
        // DPP network); the sum is exact in any order when it is used
        auto step = [&](auto mov) {
            ss += mov(ss);
            emin = min(emin, mov(emin));
        };
        step([](auto v) { return dpp_mov<0xB1, 0xf>(v, v); }); // quad_perm [1,0,3,2]
        if constexpr (TPR >= 4) step([](auto v) { return dpp_mov<0x4E, 0xf>(v, v); }); // quad_perm [2,3,0,1]
        if constexpr (TPR >= 8) step([](auto v) { return dpp_mov<0x141, 0xf>(v, v); }); // row_half_mirror
        if constexpr (TPR >= 16) step([](auto v) { return dpp_mov<0x140, 0xf>(v, v); }); // row_mirror
        // every square is a multiple of u = 2^(2 (emin - bias - MB)), and so is
        // every partial sum, which is then exact while below 2^53 u. A sum of
        // at most 256 squares computed with any roundings is more than half
        // the exact one, so ss <= 2^52 u bounds the exact sum below 2^53 u;
        // inf and NaN fail the comparison
        const bool exact = ss <= __builtin_ldexp(1.0, 52 + 2 * (emin - BIAS - MB));
        double rs;
        if (__builtin_amdgcn_ballot_w64(!exact) == 0) {
            rs = 1.0 / __builtin_sqrt(ss / double(D) + a.eps);
        } else {
            // mean_sq's order (src/muse_glimmer.hpp:509-527) over the wave's rows
            raw *sr = st[wv][lane / TPR];
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                *reinterpret_cast<Vec<raw, VEC> *>(sr + c0 + VEC * i) = lo[i];
                *reinterpret_cast<Vec<raw, VEC> *>(sr + half + c0 + VEC * i) = hi[i];
            }
            wave_lds_sync();
            for (int rw = lane >> 3; rw < RPW; rw += 8) {
                const int l = lane & 7;
                double acc = 0.0;
                for (int i = l; i < D; i += 8) {
                    const double d = double(S::dec(st[wv][rw][i]));
                    acc += d * d;
                }
                const double s1 = acc + __shfl_xor(acc, 1, 64);
                const double s2 = s1 + __shfl_xor(s1, 2, 64);
                const double s3 = s2 + __shfl_xor(s2, 4, 64);
                if (l == 0) rsf[wv][rw] = 1.0 / __builtin_sqrt(s3 / double(D) + a.eps);
            }
            wave_lds_sync();
            rs = rsf[wv][lane / TPR];
        }

        if constexpr (S::dt == BF16) {
            // every intermediate is held as the f32 of its bf16 value (one
            // conversion per rounding) and the last rounding packs two
            // elements per word. NaN propagates through every step and the
            // twin's NaN is the one pattern 0x7FC0: the steps round without
            // NaN checks and a lane whose outputs hold a NaN makes them
            // canonical once
            float fl[NH], fh[NH];
#pragma unroll
            for (int e = 0; e < NH; ++e) {
                fl[e] = bf_round(float(double(S::dec(lo[e / VEC].v[e % VEC])) * rs));
                fh[e] = bf_round(float(double(S::dec(hi[e / VEC].v[e % VEC])) * rs));
                if (isq) {
                    fl[e] = bf_round(fl[e] * qs);
                    fh[e] = bf_round(fh[e] * qs);
                }
            }
            if (rot) {
#pragma unroll
                for (int e = 0; e < NH; ++e) {
                    const uint32_t cw = __builtin_bit_cast(W4, cv[e / VEC]).v[(e % VEC) / 2];
                    const uint32_t sw = __builtin_bit_cast(W4, sv[e / VEC]).v[(e % VEC) / 2];
                    const float cc = e & 1 ? bf_hi(cw) : bf_lo(cw), sn = e & 1 ? bf_hi(sw) : bf_lo(sw);
                    const float l = fl[e], h = fh[e];
                    fl[e] = bf_round(l * cc) + bf_round(-(h * sn)); // rounded by the packing below
                    fh[e] = bf_round(h * cc) + bf_round(l * sn);
                }
            }
            W4 l4[NV], h4[NV];
            uint32_t mag = 0;
#pragma unroll
            for (int w = 0; w < 4 * NV; ++w) {
                const uint32_t lw = bf_pack(fl[2 * w], fl[2 * w + 1]), hw = bf_pack(fh[2 * w], fh[2 * w + 1]);
                l4[w / 4].v[w % 4] = lw;
                h4[w / 4].v[w % 4] = hw;
                mag = pk_max_u16(mag, pk_max_u16(lw & 0x7fff7fffu, hw & 0x7fff7fffu));
            }
            if (max(mag & 0xffffu, mag >> 16) > 0x7f80u) {
#pragma unroll
                for (int w = 0; w < 4 * NV; ++w) {
                    l4[w / 4].v[w % 4] = bf_canon(l4[w / 4].v[w % 4]);
                    h4[w / 4].v[w % 4] = bf_canon(h4[w / 4].v[w % 4]);
                }
            }
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                lo[i] = __builtin_bit_cast(Vec<raw, VEC>, l4[i]);
                hi[i] = __builtin_bit_cast(Vec<raw, VEC>, h4[i]);
            }
        } else {
#pragma unroll
            for (int e = 0; e < NH; ++e) {
                raw &lr = lo[e / VEC].v[e % VEC], &hr = hi[e / VEC].v[e % VEC];
                raw l = S::enc64(double(S::dec(lr)) * rs);
                raw h = S::enc64(double(S::dec(hr)) * rs);
                if (isq) {
                    l = S::enc(S::dec(l) * qs);
                    h = S::enc(S::dec(h) * qs);
                }
                if (rot) rope_pair<S>(l, h, cv[e / VEC].v[e % VEC], sv[e / VEC].v[e % VEC]);
                lr = l;
                hr = h;
            }
        }
        if (!live) return;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            stv<raw, VEC>(x + c0 + VEC * i, lo[i]);
            stv<raw, VEC>(x + half + c0 + VEC * i, hi[i]);
        }
        if (!isq && kc && p >= 0) {
            const int64_t slot = p < a.slots ? p : p % a.slots;
            const int64_t o = slot * (a.nkv * D) + int64_t(hh - a.nq) * D + c0;
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                stv<raw, VEC>(kc + o + VEC * i, lo[i]);
                stv<raw, VEC>(kc + o + half + VEC * i, hi[i]);
                if (vc) {
                    stv<raw, VEC>(vc + o + VEC * i, vlo[i]);
                    stv<raw, VEC>(vc + o + half + VEC * i, vhi[i]);
                }
            }
        }
    }

    template <class S, bool C = false>
    void launch_qk_t(mg_ctx *c, void *q, void *k, const void *v, const QkArgs &a, double qk_scale, const void *co,
                     const void *si, const int64_t *pos, void *kc, void *vc)
    {
        using raw = typename S::raw;
        using comp = typename S::comp;
        constexpr int V16 = 16 / sizeof(raw);
        const bool vec = a.D % V16 == 0 && a.ldq % V16 == 0 && (a.nkv == 0 || a.ldk % V16 == 0) &&
                         aligned16(q) && (a.nkv == 0 || aligned16(k)) && (!co || (aligned16(co) && aligned16(si))) &&
                         (!kc || aligned16(kc)) && (!vc || (aligned16(vc) && aligned16(v) && a.ldv % V16 == 0));
        const int64_t rows = a.T * (a.nq + a.nkv);
        const unsigned blocks = unsigned((rows + kQkRows - 1) / kQkRows);
        const size_t smem = kQkRows * sizeof(double) + size_t(kQkRows) * (a.D * sizeof(raw) + 16);
        // python-float scalar: an f32 value outside f64 (src/muse_glimmer.hpp:772)
        const comp qs = comp(S::dt == F64 ? qk_scale : double(float(qk_scale)));
        auto go = [&](auto kern) {
            hipLaunchKernelGGL(kern, dim3(blocks), dim3(256), smem, c->stream, static_cast<raw *>(q),
                               static_cast<raw *>(k), static_cast<const raw *>(v), a, qs,
                               static_cast<const raw *>(co), static_cast<const raw *>(si), pos,
                               static_cast<raw *>(kc), static_cast<raw *>(vc));
        };
        if constexpr (sizeof(raw) == 2) {
            if (vec && (a.D == 64 || a.D == 128 || a.D == 256)) {
                const int tpr = a.D / (16 * kQkPieces);
                need(rows * tpr / 256 < (int64_t(1) << 31), "qk_norm_rope: too many rows");
                const unsigned pblocks = unsigned((rows * tpr + 255) / 256);
                auto gp = [&](auto kern) {
                    hipLaunchKernelGGL(kern, dim3(pblocks), dim3(256), 0, c->stream, static_cast<raw *>(q),
                                       static_cast<raw *>(k), static_cast<const raw *>(v), a, qs,
                                       static_cast<const raw *>(co), static_cast<const raw *>(si), pos,
                                       static_cast<raw *>(kc), static_cast<raw *>(vc));
                };
                if (a.D == 64)
                    gp(k_qk_pairs<S, 64, kQkPieces>);
                else if (a.D == 128)
                    gp(k_qk_pairs<S, 128, kQkPieces>);
                else
                    gp(k_qk_pairs<S, 256, kQkPieces>);
                check_launch("k_qk_pairs");
                return;
            }
        }
        if (vec)
            go(k_qk_norm_rope<S, V16, C>);
        else
            go(k_qk_norm_rope<S, 1, C>);
        check_launch("k_qk_norm_rope");
    }

    void launch_qk_norm_rope(mg_ctx *c, void *q, int64_t nq, int64_t ldq, void *k, int64_t nkv, int64_t ldk,
                             int64_t T, int64_t D, double eps, double qk_scale, const void *co, const void *si,
                             int64_t table_rows, const int64_t *pos, int64_t pos0, const void *v, int64_t ldv,
                             void *kc, void *vc, int64_t slots, int dt)
    {
        need(D > 0 && D % 2 == 0 && D <= 512, "qk_norm_rope: head_dim must be even and <= 512");
        need(T >= 0 && nq >= 0 && nkv >= 0, "qk_norm_rope: bad shape");
        need(q != nullptr || nq == 0, "qk_norm_rope: q is NULL");
        need(k != nullptr || nkv == 0, "qk_norm_rope: k is NULL");
        need((co == nullptr) == (si == nullptr), "qk_norm_rope: give both cos and sin, or neither");
        need(co == nullptr || table_rows > 0, "qk_norm_rope: empty rope table");
        need(vc == nullptr || (kc != nullptr && v != nullptr), "qk_norm_rope: v_cache needs k_cache and v");
        need(kc == nullptr || slots > 0, "qk_norm_rope: cache_slots must be > 0");
        if (ldq == 0) ldq = nq * D;
        if (ldk == 0) ldk = nkv * D;
        if (ldv == 0) ldv = nkv * D;
        need(ldq >= nq * D && ldk >= nkv * D && (v == nullptr || ldv >= nkv * D),
             "qk_norm_rope: token stride smaller than heads*head_dim");
        if (T == 0 || nq + nkv == 0) return;
        QkArgs a{nq, nkv, ldq, ldk, ldv, T, table_rows, pos0, slots > 0 ? slots : 1, int(D), eps};
        switch (dt) {
        case BF16: launch_qk_t<SBf16>(c, q, k, v, a, qk_scale, co, si, pos, kc, vc); break;
        case F16: launch_qk_t<SF16>(c, q, k, v, a, qk_scale, co, si, pos, kc, vc); break;
        case F32: launch_qk_t<SF32>(c, q, k, v, a, qk_scale, co, si, pos, kc, vc); break;
        case F64: launch_qk_t<SF64>(c, q, k, v, a, qk_scale, co, si, pos, kc, vc); break;
        case F64 | kF32Compat: launch_qk_t<SF64, true>(c, q, k, v, a, qk_scale, co, si, pos, kc, vc); break;
        default: fail("qk_norm_rope: unknown dtype " + std::to_string(dt));
        }
    }
} // namespace mg
