// The sampler's candidate distribution on the device, from the vocab pass's
// sorted top-K (serve/sampler.py:43-112, Sampler._transformed after the
// logit edits): with top_k = K candidates in value order,
//   drop -inf candidates; none left -> point mass on the row's argmax
//   temperature <= 0 -> point mass on the argmax (greedy, first maximum)
//   probs = softmax(cl); top_p < 1 keeps the first searchsorted(cumsum, top_p)+1
//   min_p > 0 keeps probs >= min_p * max(probs)
//   final = softmax(cl / temperature), renormalized
// The reference runs these steps in numpy float32; here exp is the accurate
// f32 exp and the sums are f64, so probabilities agree to a few f32 ulp (the
// reference pins no bits here: its numpy order of summation is its own).
//
// One wave per row, candidate i in lane i / 4, slot i % 4 (K <= 256).
#include "mg_device.hpp"
#include "mg_internal.hpp"

namespace mg
{
    MG_DEV double wave_incl_scan(double v)
    {
        const int lane = threadIdx.x & 63;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const double o = __shfl_up(v, d, 64);
            v += lane >= d ? o : 0.0;
        }
        return v;
    }

    __global__ __launch_bounds__(256) void k_sample_dist(const int64_t *__restrict__ top_idx,
                                                         const float *__restrict__ top_val,
                                                         const int64_t *__restrict__ amax, int64_t rows, int K,
                                                         float temperature, float top_p, float min_p,
                                                         int64_t *__restrict__ out_ids, float *__restrict__ out_p,
                                                         int64_t *__restrict__ out_n)
    {
        const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
        const int lane = threadIdx.x & 63;
        if (row >= rows) return;
        const int64_t *ir = top_idx + row * K;
        const float *vr = top_val + row * K;
        int64_t *oi = out_ids + row * K;
        float *op = out_p + row * K;
        float cl[4];
        int64_t id[4];
        int nvalid = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int i = 4 * lane + q;
            cl[q] = i < K ? vr[i] : -__builtin_huge_valf();
            id[q] = i < K ? ir[i] : -1;
            nvalid += wave_count(cl[q] > -__builtin_huge_valf());
        }
        // candidates are sorted, so the valid ones are the first nvalid
        if (nvalid == 0 || !(temperature > 0.0f)) {
            if (lane == 0) {
                oi[0] = amax[row];
                op[0] = 1.0f;
                out_n[row] = 1;
            }
            return;
        }
        const float m = __shfl(cl[0], 0, 64); // the largest candidate
        // probs = softmax(cl) over the valid candidates
        double e[4], loc = 0.0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int i = 4 * lane + q;
            e[q] = i < nvalid ? double(exp_diff(cl[q], m)) : 0.0;
            loc += e[q];
        }
        const double S = dpp_sum(loc);
        float pr[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) pr[q] = float(e[q] / S);
        // top_p: n = first i with cumsum[i] >= top_p, plus one
        int n = nvalid;
        if (top_p < 1.0f) {
            const double base = wave_incl_scan(double(pr[0]) + pr[1] + pr[2] + pr[3]) - (double(pr[0]) + pr[1] + pr[2] + pr[3]);
            double run = base;
            int first = 0x7fffffff;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int i = 4 * lane + q;
                run += pr[q];
                if (i < nvalid && run >= double(top_p) && i < first) first = i;
            }
            int fm = first;
#pragma unroll
            for (int d = 32; d >= 1; d >>= 1) {
                const int o = __shfl_xor(fm, d, 64);
                fm = o < fm ? o : fm;
            }
            if (fm != 0x7fffffff) n = fm + 1 < nvalid ? fm + 1 : nvalid;
        }
        // min_p: probs >= min_p * max(probs) among the first n
        const float pmax = __shfl(pr[0], 0, 64);
        bool keep[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int i = 4 * lane + q;
            keep[q] = i < n && (i == 0 || !(min_p > 0.0f) || pr[q] >= min_p * pmax);
        }
        // final = softmax(cl / T) over the kept candidates, renormalized
        const float y0 = __shfl(cl[0], 0, 64) / temperature; // the largest kept (first is always kept)
        double f[4], fl = 0.0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            f[q] = keep[q] ? double(exp_diff(cl[q] / temperature, y0)) : 0.0;
            fl += f[q];
        }
        const double F = dpp_sum(fl);
        // compact the kept candidates in order
        int cnt = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) cnt += keep[q] ? 1 : 0;
        const int incl = wave_prefix_sum(cnt);
        int w = incl - cnt;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (keep[q]) {
                oi[w] = id[q];
                op[w] = float(f[q] / F);
                ++w;
            }
        if (lane == 63) out_n[row] = incl;
    }

    void launch_sample_dist(mg_ctx *c, const int64_t *top_idx, const float *top_val, const int64_t *amax,
                            int64_t rows, int64_t K, double temperature, double top_p, double min_p,
                            int64_t *out_ids, float *out_p, int64_t *out_n)
    {
        need(rows >= 0 && K >= 1 && K <= 256, "sample_dist: K must be in [1, 256]");
        need(top_idx && top_val && amax && out_ids && out_p && out_n, "sample_dist: NULL tensor");
        need(rows <= int64_t(0x7fffffff) * 4, "sample_dist: too many rows");
        if (rows == 0) return;
        hipLaunchKernelGGL(k_sample_dist, dim3(unsigned((rows + 3) / 4)), dim3(256), 0, c->stream, top_idx, top_val,
                           amax, rows, int(K), float(temperature), float(top_p), float(min_p), out_ids, out_p, out_n);
        check_launch("k_sample_dist");
    }
} // namespace mg
