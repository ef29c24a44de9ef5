// RoPE table and rotate-half application for gfx950.
//
// Table: muse::build_rope_table (src/muse_glimmer.hpp:625-674), evaluated on the
// device with the FDLIBM pow/cos/sin that the twin uses, so every entry is
// bit-identical to the reference's host table. bf16/f16/f32 follow the f32
// inverse-frequency chain (f32 exponent, f32 reciprocal, f32 angle), f64 the
// pure f64 chain, f64 with the f32-compat flag the f32 chain with entries
// stored as double(float(v)) (src/muse_glimmer.hpp:654-657).
//
// Application: muse::apply_rope (src/muse_glimmer.hpp:681-705) over (token, head)
// as muse_glimmer.hpp:809-819 drives it:
//   x[j]        = rnd(rnd(lo*c) + rnd(-hi*s))
//   x[j+half]   = rnd(rnd(hi*c) + rnd(lo*s))
// with the products and the sum of stored values taken in f32 (exact products
// for 16-bit operands, correctly rounded sums; see k_elementwise.hip) and the
// pure f64 expression for f64. One thread owns 16 bytes of `lo` and the
// matching 16 bytes of `hi`; cos/sin rows are shared by all heads of a token
// and stay in L2.
#include "mg_device.hpp"
#include "mg_internal.hpp"

namespace mg
{
    template <class S, bool C>
    __global__ __launch_bounds__(256) void k_rope_table(double theta, int dim, int64_t T,
                                                        typename S::raw *__restrict__ co,
                                                        typename S::raw *__restrict__ si)
    {
        const int half = dim / 2;
        const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
        if (idx >= T * half) return;
        const int64_t t = idx / half;
        const int j = int(idx - t * half);
        double cv, sv;
        if (S::dt != F64 || C) {
            const float e = float(2 * j) / float(dim);
            const float pw = float(mgm::pow(double(float(theta)), double(e)));
            const float inv = 1.0f / pw;
            const float ang = float(t) * inv;
            cv = mgm::cos(double(ang));
            sv = mgm::sin(double(ang));
        } else {
            const double inv = 1.0 / mgm::pow(theta, double(2 * j) / double(dim));
            const double ang = double(t) * inv;
            cv = mgm::cos(ang);
            sv = mgm::sin(ang);
        }
        if (C) {
            cv = double(float(cv));
            sv = double(float(sv));
        }
        co[idx] = S::enc64(cv);
        si[idx] = S::enc64(sv);
    }

    void launch_rope_table(mg_ctx *c, double theta, int64_t dim, int64_t T, int dt, void *co, void *si)
    {
        need(dim > 0 && dim % 2 == 0 && dim <= 65536, "rope_table: head_dim must be even");
        need(T > 0 && T < 1600000, "rope_table: positions must be in [1, 1.6e6)"); // FDLIBM medium-path range
        need(theta > 0.0 && theta < 1e300, "rope_table: theta must be finite and > 0");
        need(co && si, "rope_table: NULL output");
        const int64_t n = T * (dim / 2);
        const unsigned blocks = unsigned((n + 255) / 256);
        switch (dt) {
        case BF16: hipLaunchKernelGGL((k_rope_table<SBf16, false>), dim3(blocks), dim3(256), 0, c->stream, theta, int(dim), T, static_cast<uint16_t *>(co), static_cast<uint16_t *>(si)); break;
        case F16: hipLaunchKernelGGL((k_rope_table<SF16, false>), dim3(blocks), dim3(256), 0, c->stream, theta, int(dim), T, static_cast<uint16_t *>(co), static_cast<uint16_t *>(si)); break;
        case F32: hipLaunchKernelGGL((k_rope_table<SF32, false>), dim3(blocks), dim3(256), 0, c->stream, theta, int(dim), T, static_cast<float *>(co), static_cast<float *>(si)); break;
        case F64: hipLaunchKernelGGL((k_rope_table<SF64, false>), dim3(blocks), dim3(256), 0, c->stream, theta, int(dim), T, static_cast<double *>(co), static_cast<double *>(si)); break;
        case F64 | kF32Compat: hipLaunchKernelGGL((k_rope_table<SF64, true>), dim3(blocks), dim3(256), 0, c->stream, theta, int(dim), T, static_cast<double *>(co), static_cast<double *>(si)); break;
        default: fail("rope_table: unknown dtype " + std::to_string(dt));
        }
        check_launch("k_rope_table");
    }

    // One thread per VEC consecutive j of one (token, head). Positions outside
    // [0, table_rows) leave that head unchanged (no out-of-table read).
    template <class S, int VEC>
    __global__ __launch_bounds__(256) void k_rope(typename S::raw *q, int qh, int64_t ldq,
                                                  typename S::raw *k, int kh, int64_t ldk,
                                                  int64_t tokens, int dim,
                                                  const typename S::raw *__restrict__ co,
                                                  const typename S::raw *__restrict__ si,
                                                  int64_t table_rows, const int64_t *__restrict__ pos,
                                                  int64_t pos0)
    {
        using raw = typename S::raw;
        const int half = dim / 2, vph = half / VEC;
        const int64_t per_tok = int64_t(qh + kh) * vph;
        const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
        if (idx >= tokens * per_tok) return;
        const int64_t t = tokens * per_tok <= int64_t(0xffffffff) ? int64_t(uint32_t(idx) / uint32_t(per_tok))
                                                                    : idx / per_tok;
        const int rem = int(idx - t * per_tok);
        const int hh = rem / vph, jv = rem - hh * vph;
        const int64_t p = pos ? pos[t] : pos0 + t;
        if (p < 0 || p >= table_rows) return;
        raw *x = hh < qh ? q + t * ldq + int64_t(hh) * dim : k + t * ldk + int64_t(hh - qh) * dim;
        x += jv * VEC;
        Vec<raw, VEC> lo = ldv<raw, VEC>(x);
        Vec<raw, VEC> hi = ldv<raw, VEC>(x + half);
        const Vec<raw, VEC> c = *reinterpret_cast<const Vec<raw, VEC> *>(co + p * half + jv * VEC);
        const Vec<raw, VEC> s = *reinterpret_cast<const Vec<raw, VEC> *>(si + p * half + jv * VEC);
        if constexpr (S::dt == BF16) {
            // bf16: NaN propagates and the twin's NaN is the one pattern
            // 0x7FC0, so the steps round without NaN checks and the outputs
            // are made canonical once
            auto rn = [](float f) { return SBf16::enc_finite(f); };
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                const float fl = S::dec(lo.v[e]), fh = S::dec(hi.v[e]), cc = S::dec(c.v[e]), ss = S::dec(s.v[e]);
                const raw l = rn(S::dec(rn(fl * cc)) + S::dec(rn(-(fh * ss))));
                const raw h = rn(S::dec(rn(fh * cc)) + S::dec(rn(fl * ss)));
                lo.v[e] = S::dec(l) != S::dec(l) ? raw(0x7fc0) : l;
                hi.v[e] = S::dec(h) != S::dec(h) ? raw(0x7fc0) : h;
            }
        } else {
#pragma unroll
            for (int e = 0; e < VEC; ++e) rope_pair<S>(lo.v[e], hi.v[e], c.v[e], s.v[e]);
        }
        stv<raw, VEC>(x, lo);
        stv<raw, VEC>(x + half, hi);
    }

    template <class S>
    void launch_rope_t(mg_ctx *c, void *q, int64_t qh, int64_t ldq, void *k, int64_t kh, int64_t ldk,
                       int64_t tokens, int64_t dim, const void *co, const void *si, int64_t table_rows,
                       const int64_t *pos, int64_t pos0)
    {
        using raw = typename S::raw;
        constexpr int V = 16 / sizeof(raw);
        const int64_t half = dim / 2;
        const bool vec = half % V == 0 && ldq % V == 0 && (!k || ldk % V == 0) && aligned16(q) &&
                         (!k || aligned16(k)) && aligned16(co) && aligned16(si);
        const int vw = vec ? V : 1;
        const int64_t n = tokens * (qh + kh) * (half / vw);
        const unsigned blocks = unsigned((n + 255) / 256);
        need((n + 255) / 256 < (int64_t(1) << 31), "rope: too large");
        auto go = [&](auto kern) {
            hipLaunchKernelGGL(kern, dim3(blocks), dim3(256), 0, c->stream, static_cast<raw *>(q), int(qh),
                               ldq, static_cast<raw *>(k), int(kh), ldk, tokens, int(dim),
                               static_cast<const raw *>(co), static_cast<const raw *>(si), table_rows, pos, pos0);
        };
        if (vec)
            go(k_rope<S, V>);
        else
            go(k_rope<S, 1>);
        check_launch("k_rope");
    }

    void launch_rope(mg_ctx *c, void *q, int64_t qh, int64_t ldq, void *k, int64_t kh, int64_t ldk,
                     int64_t tokens, int64_t dim, const void *co, const void *si, int64_t table_rows,
                     const int64_t *pos, int64_t pos0, int dt)
    {
        need(dim > 0 && dim % 2 == 0 && dim <= 65536, "rope: head_dim must be even");
        need(tokens >= 0 && qh >= 0 && kh >= 0, "rope: bad shape");
        need(q != nullptr || qh == 0, "rope: q is NULL");
        if (k == nullptr) kh = 0;
        need(co && si && table_rows > 0, "rope: missing cos/sin table");
        if (ldq == 0) ldq = qh * dim;
        if (ldk == 0) ldk = kh * dim;
        need(ldq >= qh * dim && ldk >= kh * dim, "rope: token stride smaller than heads*head_dim");
        if (tokens == 0 || qh + kh == 0) return;
        switch (dt) {
        case BF16: launch_rope_t<SBf16>(c, q, qh, ldq, k, kh, ldk, tokens, dim, co, si, table_rows, pos, pos0); break;
        case F16: launch_rope_t<SF16>(c, q, qh, ldq, k, kh, ldk, tokens, dim, co, si, table_rows, pos, pos0); break;
        case F32: launch_rope_t<SF32>(c, q, qh, ldq, k, kh, ldk, tokens, dim, co, si, table_rows, pos, pos0); break;
        case F64: launch_rope_t<SF64>(c, q, qh, ldq, k, kh, ldk, tokens, dim, co, si, table_rows, pos, pos0); break;
        default: fail("rope: unknown dtype " + std::to_string(dt));
        }
    }
} // namespace mg
