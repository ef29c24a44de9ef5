// Vocab-wide logsumexp, argmax and top-K over logits [rows, V] for gfx950,
// in one read of the logits.
//
// Semantics:
//   lse     serve/sampler.py:168-171: m = max of the finite entries,
//           m + log(sum exp(x - m)) over them; -inf for a row with none
//   argmax  src/main.cpp:475-483: the strict '>' scan from index 0, i.e. the
//           first maximum; NaN never wins except at index 0, where the scan
//           starts and nothing compares greater
//   top-K   src/main.cpp:604-615 (partial_sort by value, a > b) with the tie
//           order the reference leaves unspecified made total: value
//           descending, then index ascending. NaN entries rank below -inf.
//
// Every (value, index) is packed into one 64-bit key — an order-preserving
// image of the f32 value above the complement of the index — so keys are
// unique, "K largest keys" is exactly the tie rule above, and every selection
// below is deterministic however the work is split.
//
// Pass 1, one work-group per 8192-key chunk of a row (1600 groups at the
// 64 x 201088 shape): the chunk's finite max and the f64 sum of f32 exp(x - max)
// (in a fixed order), its argmax, and its own top-K. The top-K
// uses a threshold that cannot miss: the K-th largest of the 256 per-thread
// maximum keys bounds the chunk's K-th largest from below, so every key at
// or above it is a candidate (about K + K/8 of them for random logits); the
// candidates are compacted to LDS and bitonic-sorted. If a pathological chunk
// (mass ties) yields more than kCap candidates, a bisection over the key space
// finds the exact K-th key first.
// Pass 2, one work-group per row: merge the chunk partials in a fixed order
// (max, rescaled f64 sum, FDLIBM log), fold the argmaxes, and select the
// row's top-K from the chunks' lists with the same threshold argument (the
// largest chunk K-th key bounds the row's K-th key from below).
#include "mg_device.hpp"
#include "mg_internal.hpp"

namespace mg
{
    constexpr int kVT = 256;             // threads per work-group
    constexpr int kVEPT = 32;            // keys per thread in pass 1
    constexpr int kVChunk = kVT * kVEPT; // 8192 keys per chunk
    constexpr int kCap = 2048;           // LDS candidate capacity
    constexpr int kMaxK = 256;

    struct VPart
    {
        double l;     // sum over the chunk's finite x of exp(x - m)
        float m;      // max of the chunk's finite x (-inf if none)
        float bv;     // argmax value
        int32_t bi;   // argmax index (-1: the chunk holds only NaN)
        int32_t nfin; // finite entries in the chunk
        int32_t ncand;
        int32_t pad;
    };

    MG_DEV uint64_t vkey(float v, uint32_t j)
    {
        const uint32_t hi = (v != v) ? 0u : f32_key(v);
        return (uint64_t(hi) << 32) | uint64_t(0xffffffffu - j);
    }

    MG_DEV int block_sum_i(int v, int *red)
    {
        v = wave_sum(v);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
        __syncthreads();
        int t = 0;
        for (int i = 0; i < int(blockDim.x >> 6); ++i) t += red[i];
        __syncthreads();
        return t;
    }
    MG_DEV double block_sum_d(double v, double *red)
    {
        v = wave_sum(v);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
        __syncthreads();
        double t = 0.0;
        for (int i = 0; i < int(blockDim.x >> 6); ++i) t += red[i];
        __syncthreads();
        return t;
    }
    MG_DEV float block_max_f(float v, float *red)
    {
        v = wave_max(v);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
        __syncthreads();
        float t = red[0];
        for (int i = 1; i < int(blockDim.x >> 6); ++i) t = red[i] > t ? red[i] : t;
        __syncthreads();
        return t;
    }

    MG_DEV uint64_t block_max_u64(uint64_t v, uint64_t *red)
    {
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
            const uint64_t o = __shfl_xor(v, m, 64);
            v = o > v ? o : v;
        }
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
        __syncthreads();
        uint64_t t = red[0];
        for (int i = 1; i < int(blockDim.x >> 6); ++i) t = red[i] > t ? red[i] : t;
        __syncthreads();
        return t;
    }

    // (value, index) argmax rule of the '>' scan: a beats b
    MG_DEV bool beats(float av, int ai, float bv, int bi)
    {
        if (ai < 0) return false;
        if (bi < 0) return true;
        return av > bv || (av == bv && ai < bi);
    }
    MG_DEV void block_argmax(float &v, int &i, float *redv, int *redi)
    {
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
            const float ov = __shfl_xor(v, m, 64);
            const int oi = __shfl_xor(i, m, 64);
            if (beats(ov, oi, v, i)) {
                v = ov;
                i = oi;
            }
        }
        if ((threadIdx.x & 63) == 0) {
            redv[threadIdx.x >> 6] = v;
            redi[threadIdx.x >> 6] = i;
        }
        __syncthreads();
        v = redv[0];
        i = redi[0];
        for (int w = 1; w < int(blockDim.x >> 6); ++w)
            if (beats(redv[w], redi[w], v, i)) {
                v = redv[w];
                i = redi[w];
            }
        __syncthreads();
    }

    // descending bitonic sort of a[0..n) in LDS, n a power of two
    MG_DEV void bitonic_desc(uint64_t *a, int n)
    {
        __syncthreads();
        for (int k = 2; k <= n; k <<= 1)
            for (int j = k >> 1; j > 0; j >>= 1) {
                for (int i = threadIdx.x; i < n; i += blockDim.x) {
                    const int ixj = i ^ j;
                    if (ixj > i) {
                        const uint64_t x = a[i], y = a[ixj];
                        const bool desc = (i & k) == 0;
                        if (desc ? (x < y) : (x > y)) {
                            a[i] = y;
                            a[ixj] = x;
                        }
                    }
                }
                __syncthreads();
            }
    }

    MG_DEV int pow2_at_least(int n)
    {
        int p = 1;
        while (p < n) p <<= 1;
        return p;
    }

    // ------------------------------------------------------------------ pass 1
    template <class SI>
    __global__ __launch_bounds__(kVT) void k_vocab_chunk(const typename SI::raw *__restrict__ L, int64_t V,
                                                         int K, VPart *__restrict__ part,
                                                         uint64_t *__restrict__ cand)
    {
        __shared__ uint64_t sk[kCap];
        __shared__ double redd[4];
        __shared__ float redf[4];
        __shared__ int redi[4];
        __shared__ unsigned slot;
        const int64_t row = blockIdx.y;
        const int ch = blockIdx.x, nch = gridDim.x;
        const int64_t base = int64_t(ch) * kVChunk;
        const typename SI::raw *xr = L + row * V;
        const int tid = threadIdx.x;
        const int64_t left = V - base - tid; // keys of this thread: base + tid + 256*i < V
        int nv = 0;
        if (left > 0) {
            const int64_t q = (left + kVT - 1) / kVT;
            nv = q < kVEPT ? int(q) : kVEPT;
        }

        float v[kVEPT];
#pragma unroll
        for (int i = 0; i < kVEPT; ++i)
            v[i] = i < nv ? float(SI::dec(xr[base + tid + int64_t(kVT) * i])) : 0.0f;

        // finite max, count, argmax, max key
        float m = -__builtin_huge_valf(), bv = 0.0f;
        int nfin = 0, bi = -1;
        uint64_t kmax = 0;
#pragma unroll
        for (int i = 0; i < kVEPT; ++i)
            if (i < nv) {
                const float x = v[i];
                const int j = int(base) + tid + kVT * i;
                if (__builtin_isfinite(x)) {
                    m = x > m ? x : m;
                    ++nfin;
                }
                if (x == x && (bi < 0 || x > bv)) {
                    bv = x;
                    bi = j;
                }
                const uint64_t k = vkey(x, uint32_t(j));
                kmax = k > kmax ? k : kmax;
            }
        m = block_max_f(m, redf);
        nfin = block_sum_i(nfin, redi);
        block_argmax(bv, bi, redf, redi);

        double ls = 0.0;
        if (nfin > 0)
#pragma unroll
            for (int i = 0; i < kVEPT; ++i)
                if (i < nv && __builtin_isfinite(v[i])) ls += double(exp_diff(v[i], m));
        const double l = block_sum_d(ls, redd);

        // threshold: K-th largest per-thread max key
        sk[tid] = kmax;
        bitonic_desc(sk, kVT);
        const uint64_t kmx = sk[0];
        uint64_t kappa = sk[K - 1];
        __syncthreads();
        int cnt = 0;
#pragma unroll
        for (int i = 0; i < kVEPT; ++i)
            if (i < nv && vkey(v[i], uint32_t(base + tid + kVT * i)) >= kappa) ++cnt;
        int total = block_sum_i(cnt, redi);
        if (total > kCap) {
            // exact K-th key by bisection: count(>= lo) >= K > count(>= hi)
            uint64_t lo = kappa, hi = kmx + 1;
            while (hi - lo > 1) {
                const uint64_t mid = lo + (hi - lo) / 2;
                int c = 0;
#pragma unroll
                for (int i = 0; i < kVEPT; ++i)
                    if (i < nv && vkey(v[i], uint32_t(base + tid + kVT * i)) >= mid) ++c;
                c = block_sum_i(c, redi);
                if (c >= K)
                    lo = mid;
                else
                    hi = mid;
            }
            kappa = lo;
            total = K;
        }
        if (tid == 0) slot = 0;
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kVEPT; ++i)
            if (i < nv) {
                const uint64_t k = vkey(v[i], uint32_t(base + tid + kVT * i));
                if (k >= kappa) sk[atomicAdd(&slot, 1u)] = k;
            }
        __syncthreads();
        const int n2 = pow2_at_least(total < 1 ? 1 : total);
        for (int i = total + tid; i < n2; i += kVT) sk[i] = 0;
        bitonic_desc(sk, n2);
        const int keep = total < K ? total : K;
        uint64_t *cr = cand + (row * nch + ch) * int64_t(K);
        for (int i = tid; i < K; i += kVT) cr[i] = i < keep ? sk[i] : 0;
        if (tid == 0) {
            VPart p;
            p.l = l;
            p.m = m;
            p.bv = bv;
            p.bi = bi;
            p.nfin = nfin;
            p.ncand = keep;
            p.pad = 0;
            part[row * nch + ch] = p;
        }
    }

    // ------------------------------------------------------------------ pass 2
    template <class SI>
    __global__ __launch_bounds__(kVT) void k_vocab_merge(const typename SI::raw *__restrict__ L, int64_t V,
                                                         int K, int nch, const VPart *__restrict__ part,
                                                         const uint64_t *__restrict__ cand,
                                                         double *lse, int64_t *amax, int64_t *top_idx,
                                                         float *top_val)
    {
        __shared__ uint64_t sk[kCap];
        __shared__ int redi[4];
        __shared__ float redf[4];
        __shared__ double redd[4];
        __shared__ uint64_t redu[4];
        __shared__ unsigned slot;
        __shared__ uint64_t thr;
        const int64_t row = blockIdx.x;
        const int tid = threadIdx.x;
        const VPart *pr = part + row * nch;
        const uint64_t *cr = cand + row * nch * int64_t(K);

        // merge the chunk partials: every thread folds chunks tid, tid+256, ...
        // (in order), then the threads fold in a fixed tree
        float M = -__builtin_huge_valf();
        int nfin = 0;
        float bv = 0.0f;
        int bi = -1;
        uint64_t t = 0;
        for (int c = tid; c < nch; c += kVT) {
            const VPart p = pr[c];
            if (p.nfin > 0) {
                M = p.m > M ? p.m : M;
                nfin += p.nfin;
            }
            if (beats(p.bv, p.bi, bv, bi)) {
                bv = p.bv;
                bi = p.bi;
            }
            // lower bound on the row's K-th key: the largest full chunk's K-th key
            if (p.ncand == K) {
                const uint64_t kk = cr[c * int64_t(K) + K - 1];
                t = kk > t ? kk : t;
            }
        }
        M = block_max_f(M, redf);
        nfin = block_sum_i(nfin, redi);
        block_argmax(bv, bi, redf, redi);
        t = block_max_u64(t, redu);
        double S = 0.0;
        if (nfin > 0)
            for (int c = tid; c < nch; c += kVT)
                if (pr[c].nfin > 0) S += pr[c].l * mgm::exp(double(pr[c].m) - double(M));
        S = block_sum_d(S, redd);
        if (tid == 0) {
            if (lse) lse[row] = nfin > 0 ? double(M) + mgm::log(S) : -__builtin_huge_val();
            // the scan starts at index 0: a NaN there is never beaten
            const float x0 = float(SI::dec(L[row * V]));
            if (amax) amax[row] = (x0 != x0 || bi < 0) ? 0 : bi;
            thr = t;
            slot = 0;
        }
        __syncthreads();
        if (!top_idx && !top_val) return;
        const int ncand = nch * K;
        uint64_t kappa = thr;
        int cnt = 0;
        for (int i = tid; i < ncand; i += kVT) cnt += (cr[i] != 0 && cr[i] >= kappa) ? 1 : 0;
        int total = block_sum_i(cnt, redi);
        if (total > kCap) {
            uint64_t lo = kappa, hi = ~uint64_t(0);
            while (hi - lo > 1) {
                const uint64_t mid = lo + (hi - lo) / 2;
                int c = 0;
                for (int i = tid; i < ncand; i += kVT) c += (cr[i] != 0 && cr[i] >= mid) ? 1 : 0;
                c = block_sum_i(c, redi);
                if (c >= K)
                    lo = mid;
                else
                    hi = mid;
            }
            kappa = lo;
            total = K;
        }
        for (int i = tid; i < ncand; i += kVT)
            if (cr[i] != 0 && cr[i] >= kappa) sk[atomicAdd(&slot, 1u)] = cr[i];
        __syncthreads();
        const int n2 = pow2_at_least(total < 1 ? 1 : total);
        for (int i = total + tid; i < n2; i += kVT) sk[i] = 0;
        bitonic_desc(sk, n2);
        for (int i = tid; i < K; i += kVT) {
            const uint64_t k = i < total ? sk[i] : 0;
            const uint32_t hi32 = uint32_t(k >> 32);
            const int64_t idx = k ? int64_t(0xffffffffu - uint32_t(k)) : -1;
            if (top_idx) top_idx[row * K + i] = idx;
            if (top_val) top_val[row * K + i] = k == 0 ? -__builtin_huge_valf() : (hi32 == 0 ? __builtin_nanf("") : key_f32(hi32));
        }
    }

    void launch_vocab(mg_ctx *c, const void *logits, int64_t rows, int64_t V, int dt_in, int64_t K,
                      double *lse, int64_t *amax, int64_t *top_idx, float *top_val)
    {
        need(rows >= 0 && V > 0, "vocab_reduce: bad shape");
        need(V < (int64_t(1) << 31), "vocab_reduce: V must be < 2^31");
        need(logits != nullptr, "vocab_reduce: NULL logits");
        const bool want_top = top_idx || top_val;
        if (!want_top) K = 1;
        need(K >= 1 && K <= kMaxK, "vocab_reduce: K must be in [1, 256]");
        need(K <= V, "vocab_reduce: K larger than the vocabulary");
        need(rows <= 65535, "vocab_reduce: at most 65535 rows per call");
        if (rows == 0) return;
        const int nch = int((V + kVChunk - 1) / kVChunk);
        const int64_t need_bytes = rows * nch * int64_t(sizeof(VPart)) + rows * nch * K * int64_t(sizeof(uint64_t));
        need(need_bytes <= c->work_bytes, "vocab_reduce: partials exceed the context workspace (raise workspace_bytes at mg_open)");
        VPart *part = static_cast<VPart *>(c->work);
        uint64_t *cand = reinterpret_cast<uint64_t *>(static_cast<char *>(c->work) + rows * nch * int64_t(sizeof(VPart)));
        const dim3 g1{unsigned(nch), unsigned(rows), 1u};
        if (dt_in == F32) {
            const float *x = static_cast<const float *>(logits);
            hipLaunchKernelGGL(k_vocab_chunk<SF32>, g1, dim3(kVT), 0, c->stream, x, V, int(K), part, cand);
            check_launch("k_vocab_chunk");
            hipLaunchKernelGGL(k_vocab_merge<SF32>, dim3(unsigned(rows)), dim3(kVT), 0, c->stream, x, V, int(K), nch, part, cand, lse, amax, top_idx, top_val);
        } else if (dt_in == BF16) {
            const uint16_t *x = static_cast<const uint16_t *>(logits);
            hipLaunchKernelGGL(k_vocab_chunk<SBf16>, g1, dim3(kVT), 0, c->stream, x, V, int(K), part, cand);
            check_launch("k_vocab_chunk");
            hipLaunchKernelGGL(k_vocab_merge<SBf16>, dim3(unsigned(rows)), dim3(kVT), 0, c->stream, x, V, int(K), nch, part, cand, lse, amax, top_idx, top_val);
        } else {
            fail("vocab_reduce: input dtype must be f32 or bf16");
        }
        check_launch("k_vocab_merge");
    }
} // namespace mg
