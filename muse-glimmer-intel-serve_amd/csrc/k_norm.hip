// RMSNorm rows and fused residual-add + RMSNorm for gfx950.
//
// Semantics: the reference's rmsnorm_rows pure/twin branch
// (src/muse_glimmer.hpp:572-608): rs = 1/sqrt(mean(x^2) + eps) and
// y = x*rs*(1+w) | x*rs*w | x*rs in f64, one rounding to storage. With a
// residual operand the stream is first updated h = rnd(h + x)
// (src/muse_glimmer.hpp:1023-1024); rnd(a + b) of two stored values is computed
// in f32 for the 16-bit formats, which equals the twin's f64 add followed by
// f64 -> f32 -> storage (an f32 add of f32-representable operands is the f32
// rounding of the exact sum, and rounding to f64 first cannot change that:
// 53 >= 2*24 + 2).
//
// Two kernels, chosen by shape only (never by a measurement, the rule of
// k_rmsnorm_auto, src/gpu/gpu_engine.cpp:379-390):
//   dim <= 128  k_norm_ordered: 32 rows per work-group; eight lanes per row run
//               mean_sq's eight interleaved f64 accumulators in its exact order
//               and combine them with its tree (src/muse_glimmer.hpp:509-527),
//               so the result is bit-identical to the twin in every dtype.
//   dim  > 128  k_norm_row (rows of 16-byte multiples, 16-byte aligned) or
//               k_norm_tree (others): one work-group per row, the row held in
//               registers, f64 sum of squares reduced in a fixed lane/wave
//               order (deterministic, within 1e-16 relative of the twin's
//               order; the bf16 output equals the twin's except where x*rs*w
//               lies within that distance of a rounding boundary).
// f64 storage with the f32-compat flag takes k_norm_f32compat, the
// reference's --hf-f32-compat branch bit for bit (see the kernel).
#include "mg_device.hpp"
#include "mg_internal.hpp"

#include <type_traits>

namespace mg
{
    constexpr int kOrderedMaxDim = 128;
    constexpr int kOrderedRows = 32; // 8 lanes per row, 256 threads
    constexpr int64_t kPrefetchRows = 256; // k_norm_tree requests w up front for at most this many rows

    MG_DEV double norm_out(int kind, double v, double rs, double w)
    {
        double t = v * rs;
        if (kind == 0)
            t = t * (1.0 + w);
        else if (kind == 1)
            t = t * w;
        return t;
    }

    template <class S>
    __global__ __launch_bounds__(256) void k_norm_ordered(int kind, typename S::raw *h,
                                                          const typename S::raw *__restrict__ x,
                                                          int64_t ldh, int64_t ldx,
                                                          const typename S::raw *__restrict__ w,
                                                          double eps, typename S::raw *y,
                                                          int64_t ldy, int64_t rows, int dim)
    {
        using raw = typename S::raw;
        extern __shared__ double smem_d[];
        double *rsq = smem_d;                                    // [kOrderedRows]
        raw *st = reinterpret_cast<raw *>(smem_d + kOrderedRows); // [kOrderedRows][dim]
        const int64_t r0 = int64_t(blockIdx.x) * kOrderedRows;
        const int nr = int(rows - r0 < kOrderedRows ? rows - r0 : kOrderedRows);

        // stage the rows (after the residual update) in LDS
        for (int idx = threadIdx.x; idx < nr * dim; idx += blockDim.x) {
            const int rr = idx / dim, i = idx - rr * dim;
            raw v = h[(r0 + rr) * ldh + i];
            if (x) {
                v = S::enc(S::dec(v) + S::dec(x[(r0 + rr) * ldx + i]));
                h[(r0 + rr) * ldh + i] = v;
            }
            st[rr * dim + i] = v;
        }
        __syncthreads();

        // mean_sq: lane l of a row's 8-lane group owns accumulator a_l
        const int rr = threadIdx.x >> 3, l = threadIdx.x & 7;
        const int full = dim & ~7;
        double a = 0.0;
        if (rr < nr)
            for (int i = l; i < full; i += 8) {
                const double v = double(S::dec(st[rr * dim + i]));
                a += v * v;
            }
        const double s1 = a + __shfl_xor(a, 1, 64);   // a0+a1, a2+a3, ...
        const double s2 = s1 + __shfl_xor(s1, 2, 64);  // (a0+a1)+(a2+a3), (a4+a5)+(a6+a7)
        const double s3 = s2 + __shfl_xor(s2, 4, 64);  // the fixed tree
        if (rr < nr && l == 0) {
            double tail = 0.0;
            for (int i = full; i < dim; ++i) {
                const double v = double(S::dec(st[rr * dim + i]));
                tail += v * v;
            }
            const double ms = (s3 + tail) / double(dim);
            rsq[rr] = 1.0 / __builtin_sqrt(ms + eps);
        }
        __syncthreads();

        for (int idx = threadIdx.x; idx < nr * dim; idx += blockDim.x) {
            const int r = idx / dim, i = idx - r * dim;
            const double wv = kind == 2 ? 0.0 : double(S::dec(w[i]));
            y[(r0 + r) * ldy + i] = S::enc64(norm_out(kind, double(S::dec(st[r * dim + i])), rsq[r], wv));
        }
    }

    // Sum over the work-group in a fixed order: the DPP reduction inside each
    // wave, then the wave partials in wave order. Every thread returns the
    // same value.
    MG_DEV double block_sum(double v, double *part)
    {
        v = dpp_sum(v);
        const int wid = threadIdx.x >> 6;
        if ((threadIdx.x & 63) == 0) part[wid] = v;
        __syncthreads();
        const int nw = (blockDim.x + 63) >> 6;
        double t = 0.0;
        for (int i = 0; i < nw; ++i) t += part[i];
        return t;
    }

    // WPRE (few rows, where latency rules): w is requested with h and x, so
    // the row costs one trip to memory instead of two
    template <class S, int VEC, int CPT, bool WPRE>
    __global__ __launch_bounds__(1024) void k_norm_tree(int kind, typename S::raw *h,
                                                        const typename S::raw *__restrict__ x,
                                                        int64_t ldh, int64_t ldx,
                                                        const typename S::raw *__restrict__ w,
                                                        double eps, typename S::raw *y, int64_t ldy,
                                                        int dim)
    {
        using raw = typename S::raw;
        using comp = typename S::comp;
        __shared__ double part[16];
        const int64_t row = blockIdx.x;
        raw *hr = h + row * ldh;
        const raw *xr = x ? x + row * ldx : nullptr;
        raw *yr = y + row * ldy;
        const int nchunk = dim / VEC;

        comp v[CPT][VEC];
        Vec<raw, VEC> wv[CPT], hv[CPT], xv[CPT];
        // every load of the row is issued before the first store: a store
        // between two loads would make each chunk its own round trip
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
            const int ch = threadIdx.x + c * blockDim.x;
            if (ch < nchunk) {
                hv[c] = ldv<raw, VEC>(hr + ch * VEC);
                if (xr) xv[c] = ldv<raw, VEC>(xr + ch * VEC);
                if (WPRE && kind != 2) wv[c] = *reinterpret_cast<const Vec<raw, VEC> *>(w + ch * VEC);
            }
        }
        double ss = 0.0;
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
            const int ch = threadIdx.x + c * blockDim.x;
            if (ch < nchunk) {
                Vec<raw, VEC> a = hv[c];
                if (xr) {
#pragma unroll
                    for (int e = 0; e < VEC; ++e) a.v[e] = S::enc(S::dec(a.v[e]) + S::dec(xv[c].v[e]));
                    stv<raw, VEC>(hr + ch * VEC, a);
                }
#pragma unroll
                for (int e = 0; e < VEC; ++e) {
                    v[c][e] = S::dec(a.v[e]);
                    const double d = double(v[c][e]);
                    ss += d * d;
                }
            }
        }
        const double tot = block_sum(ss, part);
        const double rs = 1.0 / __builtin_sqrt(tot / double(dim) + eps);

        if constexpr (!WPRE) {
#pragma unroll
            for (int c = 0; c < CPT; ++c) {
                const int ch = threadIdx.x + c * blockDim.x;
                if (ch < nchunk && kind != 2) wv[c] = *reinterpret_cast<const Vec<raw, VEC> *>(w + ch * VEC);
            }
        }
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
            const int ch = threadIdx.x + c * blockDim.x;
            if (ch < nchunk) {
                Vec<raw, VEC> o;
#pragma unroll
                for (int e = 0; e < VEC; ++e)
                    o.v[e] = S::enc64(norm_out(kind, double(v[c][e]), rs, kind != 2 ? double(S::dec(wv[c].v[e])) : 0.0));
                stv<raw, VEC>(yr + ch * VEC, o);
            }
        }
    }

    // The 16-byte path of k_norm_tree (rows of a multiple of 16 bytes, 16-byte
    // aligned): the same arithmetic, every access a raw buffer access over the
    // row, so threads past the row read zeros (adding nothing to the sum) and
    // store nothing, and no memory access sits behind a branch. All of a row's
    // loads (h, x and, with WPRE, w) are issued before its first store; w is
    // otherwise requested right after the sum, all chunks at once. RES: x
    // given (the fused residual add); WGT: a weighted kind.
    template <class S, int CPT, bool RES, bool WGT, bool WPRE>
    __global__ __launch_bounds__(1024) void k_norm_row(int kind, typename S::raw *h,
                                                       const typename S::raw *__restrict__ x, int64_t ldh,
                                                       int64_t ldx, const typename S::raw *__restrict__ w,
                                                       double eps, typename S::raw *y, int64_t ldy, int dim)
    {
        using raw = typename S::raw;
        using comp = typename S::comp;
        constexpr int VEC = 16 / sizeof(raw);
        __shared__ double part[16];
        const int64_t row = blockIdx.x;
        const int bytes = dim * int(sizeof(raw));
        const auto rh = buf_rsrc(h + row * ldh, bytes);
        const auto rx = buf_rsrc(RES ? x + row * ldx : h, bytes);
        const auto rw = buf_rsrc(WGT ? w : h, bytes);
        const auto ry = buf_rsrc(y + row * ldy, bytes);

        Vec<raw, VEC> hv[CPT], xv[CPT], wv[CPT];
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
            const int off = (int(threadIdx.x) + c * int(blockDim.x)) * 16;
            hv[c] = buf_ld16<raw, VEC, kAuxNT>(rh, off);
            if constexpr (RES) xv[c] = buf_ld16<raw, VEC, kAuxNT>(rx, off);
            if constexpr (WGT && WPRE) wv[c] = buf_ld16<raw, VEC, 0>(rw, off);
        }
        comp v[CPT][VEC];
        double ss = 0.0;
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
            const int off = (int(threadIdx.x) + c * int(blockDim.x)) * 16;
            if constexpr (RES) {
#pragma unroll
                for (int e = 0; e < VEC; ++e) hv[c].v[e] = S::enc(S::dec(hv[c].v[e]) + S::dec(xv[c].v[e]));
                buf_st16<raw, VEC, kAuxNT>(rh, off, hv[c]);
            }
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                v[c][e] = S::dec(hv[c].v[e]);
                const double d = double(v[c][e]);
                ss += d * d;
            }
        }
        const double tot = block_sum(ss, part);
        const double rs = 1.0 / __builtin_sqrt(tot / double(dim) + eps);
        if constexpr (WGT && !WPRE) {
#pragma unroll
            for (int c = 0; c < CPT; ++c)
                wv[c] = buf_ld16<raw, VEC, 0>(rw, (int(threadIdx.x) + c * int(blockDim.x)) * 16);
        }
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
            Vec<raw, VEC> o;
#pragma unroll
            for (int e = 0; e < VEC; ++e)
                o.v[e] = S::enc64(norm_out(kind, double(v[c][e]), rs, WGT ? double(S::dec(wv[c].v[e])) : 0.0));
            buf_st16<raw, VEC, kAuxNT>(ry, (int(threadIdx.x) + c * int(blockDim.x)) * 16, o);
        }
    }

    // f32 division and square root, correctly rounded: the f64 operation
    // rounded to f32 (53 >= 2*24 + 2, so the double rounding cannot differ)
    MG_DEV float div_f32(float a, float b) { return float(double(a) / double(b)); }
    MG_DEV float sqrt_f32(float a) { return float(__builtin_sqrt(double(a))); }

    // The f32-compat branch of rmsnorm_rows over f64 storage
    // (src/muse_glimmer.hpp:530-556, 581-594):
    //   ms = mean_sq_f32(x) + float(eps)   eight f32 accumulators a_l over
    //                                      i = l mod 8, the tree
    //                                      ((a0+a1)+(a2+a3))+((a4+a5)+(a6+a7)),
    //                                      the n mod 8 tail in order, / float(n)
    //   rs = 1.0f / sqrtf(ms)
    //   y  = double(float(x)*rs [* (1.0f + float(w)) | * float(w)])
    // every sum and product an f32 operation. Eight lanes per row, each
    // touching only its own elements (i = l mod 8; lane 0 also the tail), so a
    // residual update it stores is the value it reads back.
    __global__ __launch_bounds__(256) void k_norm_f32compat(int kind, double *h, const double *__restrict__ x,
                                                            int64_t ldh, int64_t ldx, const double *__restrict__ w,
                                                            float eps, double *y, int64_t ldy, int64_t rows,
                                                            int dim)
    {
        const int64_t r = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) >> 3;
        const int l = threadIdx.x & 7;
        const bool live = r < rows;
        double *hr = h + (live ? r : 0) * ldh;
        const double *xr = x ? x + (live ? r : 0) * ldx : nullptr;
        const int full = dim & ~7;
        // the row's value at i, after the residual update h = h + x (f64: the
        // twin's round_act at f64 is the identity)
        auto val = [&](int i) {
            double v = hr[i];
            if (xr) {
                v = v + xr[i];
                hr[i] = v;
            }
            return float(v);
        };
        float a = 0.0f;
        if (live) {
#pragma unroll 8
            for (int i = l; i < full; i += 8) {
                const float f = val(i);
                a = a + f * f;
            }
        }
        const float s1 = a + __shfl_xor(a, 1, 64);   // a0+a1, a2+a3, ...
        const float s2 = s1 + __shfl_xor(s1, 2, 64);  // (a0+a1)+(a2+a3), (a4+a5)+(a6+a7)
        const float s3 = s2 + __shfl_xor(s2, 4, 64);  // the fixed tree
        float rs = 0.0f;
        if (live && l == 0) {
            float tail = 0.0f;
            for (int i = full; i < dim; ++i) {
                const float f = val(i);
                tail = tail + f * f;
            }
            rs = div_f32(1.0f, sqrt_f32(div_f32(s3 + tail, float(dim)) + eps));
        }
        rs = __shfl(rs, int(threadIdx.x & 56), 64);
        if (!live) return;
        double *yr = y + r * ldy;
        auto out = [&](int i) {
            const float v = float(hr[i]) * rs;
            float o = v;
            if (kind == 0)
                o = v * (1.0f + float(w[i]));
            else if (kind == 1)
                o = v * float(w[i]);
            yr[i] = double(o);
        };
        for (int i = l; i < full; i += 8) out(i);
        if (l == 0)
            for (int i = full; i < dim; ++i) out(i);
    }

    template <class S, int VEC>
    void launch_tree(mg_ctx *c, int kind, void *h, const void *x, int64_t ldh, int64_t ldx,
                     const void *w, double eps, void *y, int64_t ldy, int64_t rows, int dim)
    {
        using raw = typename S::raw;
        const int nchunk = dim / VEC;
        // threads per row <= 512 where possible, <= 1024 for the few rows of a
        // decode step (each row's latency is the op's: the shortest per-thread
        // chain wins there); up to 16 chunks per thread
        int cpt = 1;
        const int lim = rows <= kPrefetchRows ? 1024 : 512;
        while ((nchunk + cpt - 1) / cpt > lim && cpt < 16) cpt *= 2;
        int nt = (nchunk + cpt - 1) / cpt;
        need(nt <= 1024, "rmsnorm: dim " + std::to_string(dim) + " too large");
        nt = (nt + 63) / 64 * 64;
        auto args = [&](auto kern) {
            hipLaunchKernelGGL(kern, dim3(unsigned(rows)), dim3(unsigned(nt)), 0, c->stream, kind,
                               static_cast<raw *>(h), static_cast<const raw *>(x), ldh, ldx,
                               static_cast<const raw *>(w), eps, static_cast<raw *>(y), ldy, dim);
        };
        if constexpr (VEC * sizeof(raw) == 16) {
            // the branch-free buffer form; <= 2^31 bytes a row (dim <= 2^20 is checked)
            auto row = [&](auto res, auto wgt, auto wpre) {
                constexpr bool R = decltype(res)::value, G = decltype(wgt)::value, P = decltype(wpre)::value;
                switch (cpt) {
                case 1: args(k_norm_row<S, 1, R, G, P>); break;
                case 2: args(k_norm_row<S, 2, R, G, P>); break;
                case 4: args(k_norm_row<S, 4, R, G, P>); break;
                case 8: args(k_norm_row<S, 8, R, G, P>); break;
                default: args(k_norm_row<S, 16, R, G, P>); break;
                }
            };
            // w requested with h and x at every row count (30.0 against 30.5 us
            // at [4096, 5120] with w after the sum)
            auto pre = [&](auto res, auto wgt) { row(res, wgt, std::true_type{}); };
            auto wgt = [&](auto res) {
                if (kind != 2)
                    pre(res, std::true_type{});
                else
                    pre(res, std::false_type{});
            };
            if (x)
                wgt(std::true_type{});
            else
                wgt(std::false_type{});
            check_launch("k_norm_row");
        } else {
        auto pick = [&](auto wpre) {
            constexpr bool P = decltype(wpre)::value;
            switch (cpt) {
            case 1: args(k_norm_tree<S, VEC, 1, P>); break;
            case 2: args(k_norm_tree<S, VEC, 2, P>); break;
            case 4: args(k_norm_tree<S, VEC, 4, P>); break;
            case 8: args(k_norm_tree<S, VEC, 8, P>); break;
            default: args(k_norm_tree<S, VEC, 16, P>); break;
            }
        };
        if (rows <= kPrefetchRows)
            pick(std::true_type{});
        else
            pick(std::false_type{});
        check_launch("k_norm_tree");
        }
    }

    template <class S>
    void launch_norm_t(mg_ctx *c, int kind, void *h, const void *x, int64_t ldh, int64_t ldx,
                       const void *w, double eps, void *y, int64_t ldy, int64_t rows, int dim)
    {
        using raw = typename S::raw;
        if (dim <= kOrderedMaxDim) {
            const size_t smem = kOrderedRows * sizeof(double) + size_t(kOrderedRows) * dim * sizeof(raw);
            const unsigned blocks = unsigned((rows + kOrderedRows - 1) / kOrderedRows);
            hipLaunchKernelGGL(k_norm_ordered<S>, dim3(blocks), dim3(256), smem, c->stream, kind,
                               static_cast<raw *>(h), static_cast<const raw *>(x), ldh, ldx,
                               static_cast<const raw *>(w), eps, static_cast<raw *>(y), ldy, rows, dim);
            check_launch("k_norm_ordered");
            return;
        }
        constexpr int V = 16 / sizeof(raw);
        const bool vec = dim % V == 0 && ldh % V == 0 && ldy % V == 0 && (!x || ldx % V == 0) &&
                         aligned16(h) && aligned16(y) && (!x || aligned16(x)) && (kind == 2 || aligned16(w));
        if (vec)
            launch_tree<S, V>(c, kind, h, x, ldh, ldx, w, eps, y, ldy, rows, dim);
        else
            launch_tree<S, 1>(c, kind, h, x, ldh, ldx, w, eps, y, ldy, rows, dim);
    }

    // Mixed storage formats — the bf16exec candidate's norm_rows
    // (src/bf16exec.hpp:398-421): rows x at one format (f32 there), weights at
    // another (bf16), the output at a third (bf16), f64 internals
    // (rs = 1/sqrt(sum x^2 / dim + eps), y = x*rs*(1+w) | x*rs*w | x*rs) and one
    // rounding of the f64 value to y's format (f64 -> f32 -> bf16 there). The
    // sum runs in a fixed order over the work-group instead of bf16exec's
    // sequential one (within 1e-16 relative). One 256-thread work-group per
    // row; the formats are uniform branches.
    MG_DEV double ld_any(const void *p, int64_t i, int dt)
    {
        switch (dt) {
        case BF16: return double(bf16_f32(static_cast<const uint16_t *>(p)[i]));
        case F16: return double(f16_f32(static_cast<const uint16_t *>(p)[i]));
        case F32: return double(static_cast<const float *>(p)[i]);
        default: return static_cast<const double *>(p)[i];
        }
    }
    MG_DEV void st_any(void *p, int64_t i, double v, int dt)
    {
        switch (dt) {
        case BF16: static_cast<uint16_t *>(p)[i] = SBf16::enc64(v); break;
        case F16: static_cast<uint16_t *>(p)[i] = SF16::enc64(v); break;
        case F32: static_cast<float *>(p)[i] = float(v); break;
        case kBf16AsF32: static_cast<float *>(p)[i] = bf16_f32(SBf16::enc64(v)); break;
        default: static_cast<double *>(p)[i] = v; break;
        }
    }
    __global__ __launch_bounds__(256) void k_norm_mixed(int kind, const void *x, int64_t ldx, int dtx, const void *w,
                                                        int dtw, double eps, void *y, int64_t ldy, int dty, int dim)
    {
        __shared__ double part[16];
        const int64_t row = blockIdx.x;
        double ss = 0.0;
        for (int i = threadIdx.x; i < dim; i += blockDim.x) {
            const double v = ld_any(x, row * ldx + i, dtx);
            ss += v * v;
        }
        const double rs = 1.0 / __builtin_sqrt(block_sum(ss, part) / double(dim) + eps);
        for (int i = threadIdx.x; i < dim; i += blockDim.x)
            st_any(y, row * ldy + i,
                   norm_out(kind, ld_any(x, row * ldx + i, dtx), rs, kind == 2 ? 0.0 : ld_any(w, i, dtw)), dty);
    }

    // f32 rows, bf16 weights (or none), y as bf16, f32 or bf16 values in f32 —
    // bf16exec's norm_rows and norm_rows_f32 (src/bf16exec.hpp:398-442) on
    // 16-byte-aligned rows of a multiple of 4: k_norm_row's form (one
    // work-group per row, every access a raw buffer access, every load before
    // the first store, so y may be x), four values a 16-byte chunk.
    template <int CPT, int DTY, bool WGT>
    __global__ __launch_bounds__(1024) void k_norm_f32rows(int kind, const float *x, int64_t ldx,
                                                           const uint16_t *__restrict__ w, double eps, void *y,
                                                           int64_t ldy, int dim)
    {
        __shared__ double part[16];
        const int64_t row = blockIdx.x;
        const auto rx = buf_rsrc(x + row * ldx, dim * 4);
        const auto rw = buf_rsrc(WGT ? static_cast<const void *>(w) : static_cast<const void *>(x), WGT ? dim * 2 : 0);
        Vec<float, 4> xv[CPT];
        uint32_t wv[CPT][2];
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
            const int ch = int(threadIdx.x) + c * int(blockDim.x);
            xv[c] = buf_ld16<float, 4, kAuxNT>(rx, ch * 16);
            if constexpr (WGT) {
                typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
                const u32x2 u = __builtin_amdgcn_raw_buffer_load_b64(rw, ch * 8, 0, 0);
                wv[c][0] = u[0];
                wv[c][1] = u[1];
            }
        }
        double ss = 0.0;
#pragma unroll
        for (int c = 0; c < CPT; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e) ss += double(xv[c].v[e]) * double(xv[c].v[e]);
        const double rs = 1.0 / __builtin_sqrt(block_sum(ss, part) / double(dim) + eps);
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
            const int ch = int(threadIdx.x) + c * int(blockDim.x);
            double o[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const double wt = WGT ? double(bf16_f32((e & 1) ? wv[c][e >> 1] >> 16 : wv[c][e >> 1] & 0xffffu)) : 0.0;
                o[e] = norm_out(kind, double(xv[c].v[e]), rs, wt);
            }
            if constexpr (DTY == BF16) {
                typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
                u32x2 u;
                u[0] = uint32_t(SBf16::enc64(o[0])) | uint32_t(SBf16::enc64(o[1])) << 16;
                u[1] = uint32_t(SBf16::enc64(o[2])) | uint32_t(SBf16::enc64(o[3])) << 16;
                __builtin_amdgcn_raw_buffer_store_b64(u, buf_rsrc(static_cast<uint16_t *>(y) + row * ldy, dim * 2),
                                                      ch * 8, 0, kAuxNT);
            } else {
                Vec<float, 4> v;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    v.v[e] = DTY == F32 ? float(o[e]) : bf16_f32(SBf16::enc64(o[e]));
                buf_st16<float, 4, kAuxNT>(buf_rsrc(static_cast<float *>(y) + row * ldy, dim * 4), ch * 16, v);
            }
        }
    }

    void launch_norm_mixed(mg_ctx *c, int kind, const void *x, int64_t ldx, int dtx, const void *w, int dtw,
                           double eps, void *y, int64_t ldy, int dty, int64_t rows, int64_t dim)
    {
        need(kind >= 0 && kind <= 2, "norm_rows_mixed: unknown norm kind " + std::to_string(kind));
        for (const int dt : {dtx, dtw})
            need(dt >= F64 && dt <= F32, "norm_rows_mixed: unknown dtype " + std::to_string(dt));
        need((dty >= F64 && dty <= F32) || dty == kBf16AsF32, "norm_rows_mixed: unknown dtype " + std::to_string(dty));
        // bf16 values kept in f32: bf16exec's norm_rows_f32 (src/bf16exec.hpp:422-442),
        // which applies the weight for Plain only (437-438): a Centered call there
        // is weight-less
        if (dty == kBf16AsF32 && kind == 0) kind = 2;
        need(rows >= 0 && dim > 0 && dim <= (int64_t(1) << 24), "norm_rows_mixed: bad shape");
        need(rows < (int64_t(1) << 31), "norm_rows_mixed: too many rows");
        need(x != nullptr && y != nullptr && (kind == 2 || w != nullptr), "norm_rows_mixed: NULL tensor");
        if (ldx == 0) ldx = dim;
        if (ldy == 0) ldy = dim;
        need(ldx >= dim && ldy >= dim, "norm_rows_mixed: leading dimension < dim");
        const int sx = dtx == F64 ? 8 : dtx == F32 ? 4 : 2, sy = dty == F64 ? 8 : (dty == F32 || dty == kBf16AsF32) ? 4 : 2;
        need(x != y || (sx == sy && ldx == ldy), "norm_rows_mixed: in place needs one element size and stride");
        if (rows == 0) return;
        const bool wgt = kind != 2;
        if (dtx == F32 && (!wgt || dtw == BF16) && (dty == BF16 || dty == F32 || dty == kBf16AsF32) && dim % 4 == 0 &&
            ldx % 4 == 0 && ldy % (dty == BF16 ? 8 : 4) == 0 && aligned16(x) && aligned16(y) &&
            (!wgt || (reinterpret_cast<uintptr_t>(w) & 7u) == 0) && dim <= (int64_t(1) << 20)) {
            const int nchunk = int(dim / 4);
            int cpt = 1;
            while ((nchunk + cpt - 1) / cpt > (rows <= 256 ? 1024 : 512) && cpt < 16) cpt *= 2;
            const int nt = ((nchunk + cpt - 1) / cpt + 63) / 64 * 64;
            if (nt <= 1024) {
                auto go = [&](auto kern) {
                    hipLaunchKernelGGL(kern, dim3(unsigned(rows)), dim3(unsigned(nt)), 0, c->stream, kind,
                                       static_cast<const float *>(x), ldx, static_cast<const uint16_t *>(w), eps, y,
                                       ldy, int(dim));
                };
                auto pick = [&](auto dtyc, auto wgtc) {
                    constexpr int D = decltype(dtyc)::value;
                    constexpr bool G = decltype(wgtc)::value;
                    switch (cpt) {
                    case 1: go(k_norm_f32rows<1, D, G>); break;
                    case 2: go(k_norm_f32rows<2, D, G>); break;
                    case 4: go(k_norm_f32rows<4, D, G>); break;
                    case 8: go(k_norm_f32rows<8, D, G>); break;
                    default: go(k_norm_f32rows<16, D, G>); break;
                    }
                };
                auto bywgt = [&](auto dtyc) {
                    if (wgt)
                        pick(dtyc, std::true_type{});
                    else
                        pick(dtyc, std::false_type{});
                };
                if (dty == BF16)
                    bywgt(std::integral_constant<int, BF16>{});
                else if (dty == F32)
                    bywgt(std::integral_constant<int, F32>{});
                else
                    bywgt(std::integral_constant<int, kBf16AsF32>{});
                check_launch("k_norm_f32rows");
                return;
            }
        }
        hipLaunchKernelGGL(k_norm_mixed, dim3(unsigned(rows)), dim3(256), 0, c->stream, kind, x, ldx, dtx, w, dtw, eps,
                           y, ldy, dty, int(dim));
        check_launch("k_norm_mixed");
    }

    void launch_norm(mg_ctx *c, int kind, void *h, const void *x, int64_t ldh, int64_t ldx,
                     const void *w, double eps, void *y, int64_t ldy, int64_t rows, int64_t dim,
                     int dt)
    {
        need(kind >= 0 && kind <= 2, "rmsnorm: unknown norm kind " + std::to_string(kind));
        need(rows >= 0 && dim > 0, "rmsnorm: bad shape");
        need(dim <= (int64_t(1) << 20), "rmsnorm: dim too large");
        need(rows <= int64_t(0x7fffffff), "rmsnorm: too many rows");
        need(kind == 2 || w != nullptr, "rmsnorm: weight is NULL for a weighted norm");
        need(h != nullptr && y != nullptr, "rmsnorm: NULL tensor");
        need(ldh >= dim && ldy >= dim && (!x || ldx >= dim), "rmsnorm: leading dimension < dim");
        if (rows == 0) return;
        if (dt & kF32Compat) {
            need(dt == (F64 | kF32Compat), "rmsnorm: the f32-compat chain takes f64 storage only");
            need(rows <= (int64_t(1) << 28), "rmsnorm: too many rows");
            const unsigned blocks = unsigned((rows + 31) / 32); // 8 lanes per row
            hipLaunchKernelGGL(k_norm_f32compat, dim3(blocks), dim3(256), 0, c->stream, kind, static_cast<double *>(h),
                               static_cast<const double *>(x), ldh, ldx, static_cast<const double *>(w),
                               float(eps), static_cast<double *>(y), ldy, rows, int(dim));
            check_launch("k_norm_f32compat");
            return;
        }
        switch (dt) {
        case BF16: launch_norm_t<SBf16>(c, kind, h, x, ldh, ldx, w, eps, y, ldy, rows, int(dim)); break;
        case F16: launch_norm_t<SF16>(c, kind, h, x, ldh, ldx, w, eps, y, ldy, rows, int(dim)); break;
        case F32: launch_norm_t<SF32>(c, kind, h, x, ldh, ldx, w, eps, y, ldy, rows, int(dim)); break;
        case F64: launch_norm_t<SF64>(c, kind, h, x, ldh, ldx, w, eps, y, ldy, rows, int(dim)); break;
        default: fail("rmsnorm: unknown dtype " + std::to_string(dt));
        }
    }
} // namespace mg
