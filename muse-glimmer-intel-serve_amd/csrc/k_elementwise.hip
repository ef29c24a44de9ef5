// Elementwise primitives for gfx950: SwiGLU, the sigmoid output gate, the
// residual add, the qk scale and the output-tail softcap.
//
// Bit-exactness against the twin (src/rounding.hpp:11-16 states the argument
// the reference relies on): a product of two stored 16-bit values is exact in
// f32, and a sum, or a product with an f32 scalar, is the f32 rounding of the
// exact value, which a prior rounding to f64 cannot change (53 >= 2*24 + 2).
// So "f32 op, then one RNE to storage" equals the twin's
// "exact f64 op, f64 -> f32 -> storage".
//
// silu and sigmoid are the twin's f64 FDLIBM forms (src/muse_glimmer.hpp:493-494).
// For bf16/f16 operands rnd(silu(g)) depends only on the 16 bits of g, so the
// context holds it as a 65536-entry table built on the device at mg_open with
// the same f64 code; the hot kernel stages the 128 KiB table in LDS (gfx950
// has 160 KiB per CU) and gathers from it, turning ~45 f64 operations per
// element into one LDS read. (Evaluating silu in f32 and proving each rounding
// unambiguous, with the table as a fallback, is exact too but measured about
// 1.8x slower here: ALU-bound at ~30 instructions per element.) f32/f64
// operands evaluate the f64 form per element.
#include "mg_device.hpp"
#include "mg_internal.hpp"

namespace mg
{
    constexpr int kLutEntries = 65536;

    // ----------------------------------------------------------------- tables
    // lut[0] silu bf16, lut[1] sigmoid bf16, lut[2] silu f16, lut[3] sigmoid f16:
    // entry i = rnd(f(decode(i))) as storage bits
    __global__ void k_build_luts(uint16_t *lut)
    {
        const int i = blockIdx.x * blockDim.x + threadIdx.x;
        if (i >= kLutEntries) return;
        const double gb = double(bf16_f32(uint32_t(i)));
        const double gh = double(f16_f32(uint16_t(i)));
        lut[0 * kLutEntries + i] = bf16_bits(float(mgm::silu(gb)));
        lut[1 * kLutEntries + i] = bf16_bits(float(mgm::sigmoid(gb)));
        lut[2 * kLutEntries + i] = f16_bits(float(mgm::silu(gh)));
        lut[3 * kLutEntries + i] = f16_bits(float(mgm::sigmoid(gh)));
    }

    void build_luts(mg_ctx *c)
    {
        hipLaunchKernelGGL(k_build_luts, dim3(kLutEntries / 256), dim3(256), 0, c->stream, c->lut);
        check_launch("k_build_luts");
    }

    // ------------------------------------------------------- gated (LUT path)
    // out = rnd(T[a] * b) with T the table of a's 16-bit pattern:
    //   SwiGLU       a = gate, b = up  (src/muse_glimmer.hpp:1036-1039)
    //   output gate  a = gate, b = pv  (src/muse_glimmer.hpp:896-906)
    // One persistent work-group per CU; 8 elements (16 bytes) per vector, one
    // vector pair per thread per pass, the grid sweeping memory contiguously.
    template <class S>
    __global__ __launch_bounds__(1024) void k_gate_lut(const uint16_t *__restrict__ table,
                                                       const uint16_t *__restrict__ a,
                                                       const uint16_t *__restrict__ b,
                                                       uint16_t *__restrict__ out, int64_t n)
    {
        __shared__ uint16_t lut[kLutEntries];
        // pairs per thread per pass: one keeps the whole grid on one contiguous
        // window of memory (4 per thread, a grid stride apart, ran 116 us
        // against 105 at config 3)
        constexpr int U = 1;
        const int64_t nvec = n / 8;
        const int64_t stride = int64_t(gridDim.x) * blockDim.x;
        int64_t base = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
        Vec<uint16_t, 8> av[U], bv[U];
        auto fetch = [&](int64_t b0) {
#pragma unroll
            for (int k = 0; k < U; ++k) {
                const int64_t i = b0 + k * stride;
                if (i < nvec) {
                    av[k] = ld16_stream<uint16_t, 8>(a + 8 * i);
                    bv[k] = ld16_stream<uint16_t, 8>(b + 8 * i);
                }
            }
        };
        // the first operands are requested before the table, whose copy into
        // LDS (all of a thread's pieces in flight at once) overlaps them
        fetch(base);
        {
            static_assert(kLutEntries / 8 == 8 * 1024, "table copy assumes 8 pieces per thread");
            const Vec<uint32_t, 4> *src = reinterpret_cast<const Vec<uint32_t, 4> *>(table);
            Vec<uint32_t, 4> *dst = reinterpret_cast<Vec<uint32_t, 4> *>(lut);
            Vec<uint32_t, 4> tv[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) tv[u] = src[threadIdx.x + 1024 * u];
#pragma unroll
            for (int u = 0; u < 8; ++u) dst[threadIdx.x + 1024 * u] = tv[u];
        }
        __syncthreads();

        for (; base < nvec; base += stride * U) {
            if (base != int64_t(blockIdx.x) * blockDim.x + threadIdx.x) fetch(base);
#pragma unroll
            for (int k = 0; k < U; ++k) {
                const int64_t i = base + k * stride;
                if (i < nvec) {
                    Vec<uint16_t, 8> o;
#pragma unroll
                    for (int e = 0; e < 8; ++e) o.v[e] = S::enc32(S::dec(lut[av[k].v[e]]) * S::dec(bv[k].v[e]));
                    st16_stream<uint16_t, 8>(out + 8 * i, o);
                }
            }
        }
        // the n % 8 tail
        if (blockIdx.x == 0)
            for (int64_t i = nvec * 8 + threadIdx.x; i < n; i += blockDim.x)
                out[i] = S::enc32(S::dec(lut[a[i]]) * S::dec(b[i]));
    }

    // Scalar LUT variant for operands that are not 16-byte aligned.
    template <class S>
    __global__ __launch_bounds__(256) void k_gate_lut_scalar(const uint16_t *__restrict__ table,
                                                             const uint16_t *__restrict__ a,
                                                             const uint16_t *__restrict__ b,
                                                             uint16_t *__restrict__ out, int64_t n)
    {
        for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x)
            out[i] = S::enc32(S::dec(table[a[i]]) * S::dec(b[i]));
    }

    // ------------------------------------------------------ gated (f64 path)
    // f32 / f64 storage: f = silu or sigmoid in f64 per element; f64 keeps the
    // pure form f(a)*b, f32 materializes rnd(rnd(f(a)) * b) at f32.
    template <class S, bool SIG>
    __global__ __launch_bounds__(256) void k_gate_f64(const typename S::raw *__restrict__ a,
                                                      const typename S::raw *__restrict__ b,
                                                      typename S::raw *__restrict__ out, int64_t n)
    {
        for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
            const double g = double(a[i]);
            const double f = SIG ? mgm::sigmoid(g) : mgm::silu(g);
            if (S::dt == F64)
                out[i] = typename S::raw(f * double(b[i]));
            else
                out[i] = typename S::raw(float(f) * float(b[i]));
        }
    }

    void launch_swiglu(mg_ctx *c, const void *g, const void *u, void *out, int64_t n, int dt,
                       bool sigmoid_gate)
    {
        // sigmoid gate: the table operand is the gate, the other the pv product
        need(n >= 0, "swiglu: negative size");
        need(g && u && out, "swiglu: NULL tensor");
        if (n == 0) return;
        const int blocks_f64 = int(std::min<int64_t>((n + 255) / 256, int64_t(c->num_cus) * 16));
        if (dt == BF16 || dt == F16) {
            const uint16_t *table = c->lut + (dt == BF16 ? 0 : 2 * kLutEntries) + (sigmoid_gate ? kLutEntries : 0);
            const auto *a = static_cast<const uint16_t *>(g);
            const auto *b = static_cast<const uint16_t *>(u);
            auto *o = static_cast<uint16_t *>(out);
            if (aligned16(a) && aligned16(b) && aligned16(o)) {
                const int blocks = int(std::min<int64_t>((n / 8 + 1023) / 1024 + 1, int64_t(c->num_cus)));
                if (dt == BF16)
                    hipLaunchKernelGGL(k_gate_lut<SBf16>, dim3(blocks), dim3(1024), 0, c->stream, table, a, b, o, n);
                else
                    hipLaunchKernelGGL(k_gate_lut<SF16>, dim3(blocks), dim3(1024), 0, c->stream, table, a, b, o, n);
            } else {
                if (dt == BF16)
                    hipLaunchKernelGGL(k_gate_lut_scalar<SBf16>, dim3(blocks_f64), dim3(256), 0, c->stream, table, a, b, o, n);
                else
                    hipLaunchKernelGGL(k_gate_lut_scalar<SF16>, dim3(blocks_f64), dim3(256), 0, c->stream, table, a, b, o, n);
            }
        } else if (dt == F32) {
            auto *a = static_cast<const float *>(g);
            auto *b = static_cast<const float *>(u);
            auto *o = static_cast<float *>(out);
            if (sigmoid_gate)
                hipLaunchKernelGGL((k_gate_f64<SF32, true>), dim3(blocks_f64), dim3(256), 0, c->stream, a, b, o, n);
            else
                hipLaunchKernelGGL((k_gate_f64<SF32, false>), dim3(blocks_f64), dim3(256), 0, c->stream, a, b, o, n);
        } else if (dt == F64) {
            auto *a = static_cast<const double *>(g);
            auto *b = static_cast<const double *>(u);
            auto *o = static_cast<double *>(out);
            if (sigmoid_gate)
                hipLaunchKernelGGL((k_gate_f64<SF64, true>), dim3(blocks_f64), dim3(256), 0, c->stream, a, b, o, n);
            else
                hipLaunchKernelGGL((k_gate_f64<SF64, false>), dim3(blocks_f64), dim3(256), 0, c->stream, a, b, o, n);
        } else {
            fail("swiglu: unknown dtype " + std::to_string(dt));
        }
        check_launch(sigmoid_gate ? "k_gate(sigmoid)" : "k_gate(silu)");
    }

    // ------------------------------------------------------- residual / scale
    // OP 0: h = rnd(h + x)   (src/muse_glimmer.hpp:1023-1024)
    // OP 1: h = rnd(h * s)   (src/muse_glimmer.hpp:803-807, s an f32 opmath value
    //                         for stored formats other than f64)
    template <class S, int OP>
    __global__ __launch_bounds__(256) void k_binary(typename S::raw *__restrict__ h,
                                                    const typename S::raw *__restrict__ x,
                                                    typename S::comp s, int64_t n)
    {
        using raw = typename S::raw;
        constexpr int V = 16 / sizeof(raw);
        const int64_t nvec = n / V;
        const int64_t stride = int64_t(gridDim.x) * blockDim.x;
        const int64_t t0 = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
        for (int64_t i = t0; i < nvec; i += stride) {
            Vec<raw, V> a = ldv<raw, V>(h + V * i);
            Vec<raw, V> b;
            if (OP == 0) b = ldv<raw, V>(x + V * i);
#pragma unroll
            for (int e = 0; e < V; ++e)
                a.v[e] = OP == 0 ? S::enc(S::dec(a.v[e]) + S::dec(b.v[e])) : S::enc(S::dec(a.v[e]) * s);
            stv<raw, V>(h + V * i, a);
        }
        for (int64_t i = nvec * V + t0; i < n; i += stride)
            h[i] = OP == 0 ? S::enc(S::dec(h[i]) + S::dec(x[i])) : S::enc(S::dec(h[i]) * s);
    }

    template <class S, int OP>
    void launch_binary_t(mg_ctx *c, void *h, const void *x, double s, int64_t n)
    {
        using raw = typename S::raw;
        using comp = typename S::comp;
        need(aligned16(h) && (OP == 1 || aligned16(x)), "elementwise: tensors must be 16-byte aligned");
        const int blocks = int(std::min<int64_t>((n / (16 / sizeof(raw)) + 255) / 256 + 1, int64_t(c->num_cus) * 8));
        hipLaunchKernelGGL((k_binary<S, OP>), dim3(blocks), dim3(256), 0, c->stream, static_cast<raw *>(h),
                           static_cast<const raw *>(x), comp(S::dt == F64 ? s : double(float(s))), n);
        check_launch("k_binary");
    }

    template <int OP>
    void launch_binary(mg_ctx *c, void *h, const void *x, double s, int64_t n, int dt)
    {
        need(n >= 0, "elementwise: negative size");
        need(h && (OP == 1 || x), "elementwise: NULL tensor");
        if (n == 0) return;
        switch (dt) {
        case BF16: launch_binary_t<SBf16, OP>(c, h, x, s, n); break;
        case F16: launch_binary_t<SF16, OP>(c, h, x, s, n); break;
        case F32: launch_binary_t<SF32, OP>(c, h, x, s, n); break;
        case F64: launch_binary_t<SF64, OP>(c, h, x, s, n); break;
        default: fail("elementwise: unknown dtype " + std::to_string(dt));
        }
    }

    void launch_residual_add(mg_ctx *c, void *h, const void *x, int64_t n, int dt)
    {
        launch_binary<0>(c, h, x, 0.0, n, dt);
    }
    void launch_scale(mg_ctx *c, void *x, int64_t n, double s, int dt)
    {
        launch_binary<1>(c, x, nullptr, s, n, dt);
    }

    // ---------------------------------------------------------------- softcap
    // apply_output_tail (src/muse_glimmer.hpp:920-943): z*mult, z/cap, tanh, z*cap,
    // each materialized at storage; FDLIBM tanh in f64 per element.
    template <class S>
    __global__ __launch_bounds__(256) void k_softcap(typename S::raw *__restrict__ z, int64_t n,
                                                     double mult, double cap)
    {
        for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
            double v = double(S::dec(z[i]));
            if (mult != 1.0) v = double(S::dec(S::enc64(v * mult)));
            if (cap != 0.0) {
                v = double(S::dec(S::enc64(v / cap)));
                v = double(S::dec(S::enc64(mgm::tanh(v))));
                v = double(S::dec(S::enc64(v * cap)));
            }
            z[i] = S::enc64(v);
        }
    }

    void launch_softcap(mg_ctx *c, void *z, int64_t n, double mult, double cap, int dt)
    {
        need(n >= 0 && z, "softcap: bad arguments");
        if (n == 0) return;
        const int blocks = int(std::min<int64_t>((n + 255) / 256, int64_t(c->num_cus) * 16));
        // python-float scalars are f32 opmath values outside f64 (src/muse_glimmer.hpp:929-931)
        const double m = dt == F64 ? mult : double(float(mult));
        const double k = dt == F64 ? cap : double(float(cap));
        switch (dt) {
        case BF16: hipLaunchKernelGGL(k_softcap<SBf16>, dim3(blocks), dim3(256), 0, c->stream, static_cast<uint16_t *>(z), n, m, k); break;
        case F16: hipLaunchKernelGGL(k_softcap<SF16>, dim3(blocks), dim3(256), 0, c->stream, static_cast<uint16_t *>(z), n, m, k); break;
        case F32: hipLaunchKernelGGL(k_softcap<SF32>, dim3(blocks), dim3(256), 0, c->stream, static_cast<float *>(z), n, m, k); break;
        case F64: hipLaunchKernelGGL(k_softcap<SF64>, dim3(blocks), dim3(256), 0, c->stream, static_cast<double *>(z), n, m, k); break;
        default: fail("softcap: unknown dtype " + std::to_string(dt));
        }
        check_launch("k_softcap");
    }
} // namespace mg
