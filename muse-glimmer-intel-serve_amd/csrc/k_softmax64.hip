// Scaled, masked row softmax over f64 scores for gfx950: the twin's f64 runs.
//
// pure (dtype_in = dtype_out = f64): attention_forward's f64 softmax
// (src/muse_glimmer.hpp:845-848, 871-880):
//   s = x * scale in f64 (with a softcap, s = cap * tanh(s / cap) in
//   apply_output_tail's op order, 920-943, FDLIBM tanh), m = max over the
//   visible keys, e = exp(s - m) (FDLIBM), p = e / sum.
//   The sum is taken in a fixed order over the work-group instead of the
//   ascending loop: the same bits on every run, within 2e-15 relative of the
//   reference's sum.
// f32-compat (dtype_in = f64 | compat, the --hf-f32-compat chain, 856-870),
// bit for bit:
//   m32 = max float(s)   (std::max(m32, v): a NaN score is never taken)
//   e   = float(exp(double(float(s) - m32)))
//   sum32 = e_lo + ... + e_hi, one f32 chain in ascending key order
//   p   = double(float(e) / sum32)
// The ascending chain is one wave's job: it reads 64 e values at a time and
// adds them in lane order, each addition an f32 operation on wave-uniform
// values; the other waves wait at the barrier. The max, by contrast, is exact
// in any order.
// Masked keys get exactly 0; a row with no visible key is all zeros.
// One work-group of 256 threads per row; e is parked in y between the passes
// and every thread reads back only what it wrote (the chain's wave aside, after
// a barrier), so y may alias x.
#include "mg_device.hpp"
#include "mg_internal.hpp"

namespace mg
{
    struct Sm64Args
    {
        int64_t q, kc, window, q_pos0;
        int64_t ldx, ldy; // row strides, in elements
        double scale, cap;
        int mask;
    };

    template <typename T>
    MG_DEV T max_keep(T m, T v) { return m < v ? v : m; } // std::max(m, v)

    // max over the work-group of values that are never NaN: exact in any order
    template <typename T>
    MG_DEV T block_max(T v, T *red)
    {
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) v = max_keep(v, __shfl_xor(v, m, 64));
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
        __syncthreads();
        T r = red[0];
        for (int i = 1; i < 4; ++i) r = max_keep(r, red[i]);
        return r;
    }

    template <bool COMPAT, bool CAP>
    __global__ __launch_bounds__(256) void k_softmax_f64(const double *x, double *y, Sm64Args a)
    {
        __shared__ double red[4];
        __shared__ float redf[4];
        __shared__ float sum32_sh;
        const int64_t row = blockIdx.x;
        const double *xr = x + row * a.ldx;
        double *yr = y + row * a.ldy;
        int64_t lo, hi;
        mask_range(a.mask, a.q_pos0 + row % a.q, a.kc, a.window, lo, hi);
        const int tid = threadIdx.x;
        for (int64_t j = tid; j < a.kc; j += 256)
            if (j < lo || j > hi) yr[j] = 0.0;
        if (hi < lo) return; // uniform over the work-group

        auto score = [&](int64_t j) {
            double s = xr[j] * a.scale;
            if (CAP) {
                s = s / a.cap;
                s = mgm::tanh(s);
                s = s * a.cap;
            }
            return s;
        };

        if constexpr (COMPAT) {
            float m = -__builtin_huge_valf();
            for (int64_t j = lo + tid; j <= hi; j += 256) m = max_keep(m, float(score(j)));
            const float m32 = block_max(m, redf);
            for (int64_t j = lo + tid; j <= hi; j += 256)
                yr[j] = double(float(mgm::exp(double(float(score(j)) - m32))));
            __syncthreads();
            if (tid < 64) {
                // the ascending f32 chain; lanes past hi add +0, which leaves
                // every partial sum (>= +0 or NaN) unchanged
                float acc = 0.0f;
                for (int64_t b = lo; b <= hi; b += 64) {
                    const int64_t j = b + tid;
                    const float e = j <= hi ? float(yr[j]) : 0.0f;
                    const int eb = __builtin_bit_cast(int, e);
#pragma unroll
                    for (int l = 0; l < 64; ++l) acc = acc + __builtin_bit_cast(float, __builtin_amdgcn_readlane(eb, l));
                }
                if (tid == 0) sum32_sh = acc;
            }
            __syncthreads();
            const float sum32 = sum32_sh;
            for (int64_t j = lo + tid; j <= hi; j += 256)
                yr[j] = double(float(double(float(yr[j])) / double(sum32))); // f32 quotient (53 >= 2*24 + 2)
        } else {
            double m = -__builtin_huge_val();
            for (int64_t j = lo + tid; j <= hi; j += 256) m = max_keep(m, score(j));
            const double mx = block_max(m, red);
            double s = 0.0;
            for (int64_t j = lo + tid; j <= hi; j += 256) {
                const double e = mgm::exp(score(j) - mx);
                yr[j] = e;
                s += e;
            }
            // fixed order: butterfly in each wave, then the waves in order
            s = wave_sum(s);
            __syncthreads(); // red is reused
            if ((tid & 63) == 0) red[tid >> 6] = s;
            __syncthreads();
            const double sum = ((red[0] + red[1]) + red[2]) + red[3];
            for (int64_t j = lo + tid; j <= hi; j += 256) yr[j] = yr[j] / sum;
        }
    }

    void launch_softmax_f64(mg_ctx *c, const void *x, int64_t ldx, void *y, int64_t ldy, int64_t rows, int64_t q,
                            int64_t kc, double scale, int mask, int64_t window, int64_t q_pos0, double softcap,
                            bool compat)
    {
        need(rows < (int64_t(1) << 31), "softmax: too many rows");
        need(!compat || softcap == 0.0, "softmax: the f32-compat chain has no softcap");
        const Sm64Args a{q, kc, window, q_pos0, ldx, ldy, scale, softcap, mask};
        const double *xi = static_cast<const double *>(x);
        double *yo = static_cast<double *>(y);
        const dim3 grid{unsigned(rows)};
        if (compat)
            hipLaunchKernelGGL((k_softmax_f64<true, false>), grid, dim3(256), 0, c->stream, xi, yo, a);
        else if (softcap != 0.0)
            hipLaunchKernelGGL((k_softmax_f64<false, true>), grid, dim3(256), 0, c->stream, xi, yo, a);
        else
            hipLaunchKernelGGL((k_softmax_f64<false, false>), grid, dim3(256), 0, c->stream, xi, yo, a);
        check_launch("k_softmax_f64");
    }
} // namespace mg
