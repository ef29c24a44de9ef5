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
#include "mg_wave_sort.hpp"

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
                                                         const int64_t *__restrict__ amax,
                                                         const int64_t *__restrict__ raw_amax, int64_t rows, int K,
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
        int nvalid = 0, nfinite = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int i = 4 * lane + q;
            cl[q] = i < K ? vr[i] : -__builtin_huge_valf();
            id[q] = i < K ? ir[i] : -1;
            nvalid += wave_count(cl[q] > -__builtin_huge_valf());
            nfinite += wave_count(__builtin_isfinite(cl[q]));
        }
        // candidates are sorted, so the valid ones are the first nvalid. No
        // finite value among them: the row has none (sorted keys put every
        // finite value ahead of -inf and NaN), the reference's "masked"
        // fallback, a point mass on the argmax of the raw logits (70-74);
        // otherwise temperature <= 0 is greedy on the edited logits (76-78)
        if (nfinite == 0 || !(temperature > 0.0f)) {
            if (lane == 0) {
                oi[0] = nfinite == 0 && raw_amax ? raw_amax[row] : amax[row];
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
                            const int64_t *raw_amax, int64_t rows, int64_t K, double temperature, double top_p,
                            double min_p, int64_t *out_ids, float *out_p, int64_t *out_n)
    {
        need(rows >= 0 && K >= 1 && K <= 256, "sample_dist: K must be in [1, 256] (other top_k: mg_sample_rows)");
        need(top_idx && top_val && amax && out_ids && out_p && out_n, "sample_dist: NULL tensor");
        need(rows <= int64_t(0x7fffffff) * 4, "sample_dist: too many rows");
        if (rows == 0) return;
        hipLaunchKernelGGL(k_sample_dist, dim3(unsigned((rows + 3) / 4)), dim3(256), 0, c->stream, top_idx, top_val,
                           amax, raw_amax, rows, int(K), float(temperature), float(top_p), float(min_p), out_ids,
                           out_p, out_n);
        check_launch("k_sample_dist");
    }

    // ------------------------------------------------------------------
    // The whole filter chain on full logit rows, for any top_k
    // (serve/sampler.py:43-112, Sampler._transformed after the logit edits):
    // one 1024-thread work-group per row of lg (f32, the edited logits).
    //   no finite lg            point mass on raw_amax[row] (the raw logits'
    //                           argmax, 70-74; the row's own argmax if NULL)
    //   temperature <= 0        point mass on np.argmax(lg): the first
    //                           maximum, NaN counting as the largest (76-78)
    //   candidates C            entries > -inf (NaN and -inf dropped, 97-98);
    //                           0 < top_k < |C|: the top_k largest, ties by
    //                           lower index (80-89: argpartition's tie order is
    //                           unspecified, this one is total)
    //   p = softmax(C)          e = exp(x - max) (exp_diff), S = sum e in f64
    //   top_p < 1               the shortest prefix of C in (value desc, index
    //                           asc) order whose e sum reaches top_p * S
    //                           (searchsorted(cumsum, top_p) + 1, 104-106)
    //   min_p > 0               keeps p >= min_p * max(p) (f32 compare, 107-109)
    //   final                   softmax(x / T) over the kept entries (111-112)
    // Output order: value order when top_k > 0 or top_p < 1 (the reference
    // sorts then), else index order. Sorted outputs: the largest (at most
    // kSortMax) candidates are gathered into LDS and sorted, the top_p cut is
    // found by an f64 prefix sum in that order; a row whose kept prefix does
    // not fit, or that holds +inf (whose reference probabilities are NaN, so
    // its draw raises), gets count -1 and is left to the host.
    // The gathering: pass 1 also counts the candidates per 13-bit prefix of
    // their 32-bit order-preserving image (8192 bins); the bin holding the
    // kSortMax-th largest (bstar) fixes a threshold, and the pass that sums S
    // gathers the candidates above it (fewer than kSortMax) and those in it
    // (when at most kSortMax) into two LDS regions (positions from LDS
    // counters, in no particular order: the keys are unique and sorted
    // next); the two are sorted apart and the second's largest appended.
    // Rows whose threshold bin holds more, and the top_k selection, take MSD
    // radix passes over the image (and the index among equal values) with an
    // LDS count histogram instead. Counts are integers, so every result is
    // independent of the order in which threads add, and the f64 sums reduce
    // in a fixed order.
    constexpr int kSortMax = 4096;
    constexpr int kGatherCap = 2 * kSortMax;
    constexpr int kHistBits = 13;
    constexpr int kSfThreads = 1024;

    struct SfLds
    {
        uint32_t cnt[256];
        uint32_t hist[(1 << kHistBits) + 1]; // the last: a spare bin for non-candidates
        uint64_t keys[kGatherCap];
        double red[kSortMax / 4];
        double redd[kSfThreads / 64];
        uint64_t redu[kSfThreads / 64];
        uint32_t bc[4]; // broadcast words
        uint32_t gcount[2]; // keys gathered so far above the threshold bin, in it
    };

    MG_DEV uint32_t sf_img(float x) { return f32_key(x + 0.0f); } // -0 ranks with +0
    MG_DEV bool sf_cand(float x) { return x > -__builtin_huge_valf(); } // NaN and -inf fail

    // work-group sums in a fixed order (every thread returns the total)
    MG_DEV double sf_sum_f64(double v, SfLds &L)
    {
        v = dpp_sum(v);
        if ((threadIdx.x & 63) == 0) L.redd[threadIdx.x >> 6] = v;
        __syncthreads();
        double t = 0.0;
        for (int i = 0; i < kSfThreads / 64; ++i) t += L.redd[i];
        __syncthreads();
        return t;
    }
    template <class OP>
    MG_DEV uint64_t sf_red_u64(uint64_t v, SfLds &L, OP op)
    {
        const int lane = threadIdx.x & 63;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const uint64_t o = __shfl_xor(v, d, 64);
            v = op(v, o);
        }
        if (lane == 0) L.redu[threadIdx.x >> 6] = v;
        __syncthreads();
        uint64_t t = L.redu[0];
        for (int i = 1; i < kSfThreads / 64; ++i) t = op(t, L.redu[i]);
        __syncthreads();
        return t;
    }
    MG_DEV uint64_t sf_sum_u64(uint64_t v, SfLds &L)
    {
        return sf_red_u64(v, L, [](uint64_t a, uint64_t b) { return a + b; });
    }
    MG_DEV uint64_t sf_max_u64(uint64_t v, SfLds &L)
    {
        return sf_red_u64(v, L, [](uint64_t a, uint64_t b) { return a > b ? a : b; });
    }
    MG_DEV uint64_t sf_min_u64(uint64_t v, SfLds &L)
    {
        return sf_red_u64(v, L, [](uint64_t a, uint64_t b) { return a < b ? a : b; });
    }
    // exclusive prefix over the work-group in thread order; total in *tot
    MG_DEV int sf_scan(int v, SfLds &L, int *tot)
    {
        const int incl = wave_prefix_sum(v);
        if ((threadIdx.x & 63) == 63) L.redu[threadIdx.x >> 6] = uint64_t(incl);
        __syncthreads();
        int base = 0, all = 0;
        for (int i = 0; i < kSfThreads / 64; ++i) {
            const int w = int(L.redu[i]);
            base += i < int(threadIdx.x >> 6) ? w : 0;
            all += w;
        }
        __syncthreads();
        *tot = all;
        return base + incl - v;
    }
    // the same for f64 values: each thread's exclusive prefix, summed in a
    // fixed order (the lanes' values through LDS, then the waves')
    MG_DEV double sf_scan_f64(double v, SfLds &L)
    {
        L.red[threadIdx.x] = v;
        __syncthreads();
        const int w0 = int(threadIdx.x) & ~63, lane = int(threadIdx.x) & 63;
        double in_wave = 0.0;
        for (int i = 0; i < lane; ++i) in_wave += L.red[w0 + i];
        double wave_tot = in_wave;
        for (int i = lane; i < 64; ++i) wave_tot += L.red[w0 + i];
        if (lane == 63) L.redd[threadIdx.x >> 6] = wave_tot;
        __syncthreads();
        double base = 0.0;
        for (int i = 0; i < int(threadIdx.x >> 6); ++i) base += L.redd[i];
        __syncthreads();
        return base + in_wave;
    }

    // keys[0, n) sorted descending, n a power of two: each wave sorts its n/16
    // contiguous keys in registers (wave_bitonic, direction alternating by
    // wave as the network's runs do), then each merge level takes its strides
    // of n/16 and more through LDS and the rest in registers
    // (wave_bitonic_merge). Callers synchronize before (the keys written).
    template <int R>
    MG_DEV void sf_sort_regs(uint64_t *keys, int n)
    {
        constexpr int SEG = 64 * R;
        const int lane = threadIdx.x & 63;
        const int base = int(threadIdx.x >> 6) * SEG;
        uint64_t a[R];
#pragma unroll
        for (int r = 0; r < R; ++r) a[r] = keys[base + 64 * r + lane];
        if ((base & SEG) == 0)
            wave_bitonic<uint64_t, R, true>(a);
        else
            wave_bitonic<uint64_t, R, false>(a);
        for (int size = 2 * SEG; size <= n; size <<= 1) {
#pragma unroll
            for (int r = 0; r < R; ++r) keys[base + 64 * r + lane] = a[r];
            __syncthreads();
            for (int stride = size >> 1; stride >= SEG; stride >>= 1) {
                for (int i = threadIdx.x; i < n; i += kSfThreads) {
                    const int j = i ^ stride;
                    if (j > i) {
                        const bool desc = (i & size) == 0;
                        const uint64_t x = keys[i], y = keys[j];
                        if (desc ? x < y : x > y) {
                            keys[i] = y;
                            keys[j] = x;
                        }
                    }
                }
                __syncthreads();
            }
#pragma unroll
            for (int r = 0; r < R; ++r) a[r] = keys[base + 64 * r + lane];
            wave_bitonic_merge<uint64_t, R>(a, (base & size) == 0);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) keys[base + 64 * r + lane] = a[r];
        __syncthreads();
    }
    MG_DEV void sf_sort_desc(uint64_t *keys, int n)
    {
        static_assert(kSortMax <= 4 * kSfThreads, "sf_sort_desc: at most four keys a thread");
        switch (n) {
        case kSfThreads: sf_sort_regs<1>(keys, n); return;
        case 2 * kSfThreads: sf_sort_regs<2>(keys, n); return;
        case 4 * kSfThreads: sf_sort_regs<4>(keys, n); return;
        default: break;
        }
        // fewer keys than threads: the network in LDS
        for (int size = 2; size <= n; size <<= 1)
            for (int stride = size >> 1; stride > 0; stride >>= 1) {
                const int i = threadIdx.x;
                const int j = i ^ stride;
                if (i < n && j > i) {
                    const bool desc = (i & size) == 0;
                    const uint64_t x = keys[i], y = keys[j];
                    if (desc ? x < y : x > y) {
                        keys[i] = y;
                        keys[j] = x;
                    }
                }
                __syncthreads();
            }
    }

    // f(i, x) for every entry of the row, in a fixed order per thread; 16-byte
    // loads on 16-byte-aligned rows, entry by entry otherwise. Aligned rows go
    // in groups of 4 x 4096 entries (thread t takes entries 4t..4t+3 of each
    // 4096), the next group's loads in flight while f runs over the current
    // one (two register sets; the last group's successor is re-read in place
    // of a group past the end, so no branch stands between the loads and
    // their waits). Every lane of a wave calls f the same number of times
    // except in the row's last 16 384 entries (lanes past the end idle).
    template <class F>
    MG_DEV void sf_each(const float *lr, int64_t V, bool al16, F f)
    {
        if (al16) {
            const int64_t V4 = V >> 2;
            const Vec<float, 4> *p = reinterpret_cast<const Vec<float, 4> *>(lr);
            constexpr int64_t G = 4 * kSfThreads; // vectors per group
            const int64_t ng = V4 / G;            // whole groups
            auto load = [&](Vec<float, 4>(&r)[4], int64_t grp) {
                const int64_t q = (grp < ng ? grp : ng - 1) * G + threadIdx.x;
#pragma unroll
                for (int u = 0; u < 4; ++u) r[u] = p[q + u * kSfThreads];
            };
            auto run = [&](const Vec<float, 4>(&r)[4], int64_t grp) {
                const int64_t q = grp * G + threadIdx.x;
#pragma unroll
                for (int u = 0; u < 4; ++u)
#pragma unroll
                    for (int e = 0; e < 4; ++e) f(4 * (q + u * kSfThreads) + e, r[u].v[e]);
            };
            if (ng > 0) {
                Vec<float, 4> A[4], B[4];
                load(A, 0);
                for (int64_t grp = 0; grp < ng; grp += 2) {
                    load(B, grp + 1);
                    run(A, grp);
                    load(A, grp + 2);
                    if (grp + 1 < ng) run(B, grp + 1);
                }
            }
            int64_t g = ng * G + threadIdx.x;
            for (; g < V4; g += kSfThreads) {
                const Vec<float, 4> a = p[g];
#pragma unroll
                for (int e = 0; e < 4; ++e) f(4 * g + e, a.v[e]);
            }
            for (int64_t i = (V4 << 2) + threadIdx.x; i < V; i += kSfThreads) f(i, lr[i]);
        } else {
            for (int64_t i = threadIdx.x; i < V; i += kSfThreads) f(i, lr[i]);
        }
    }

    // The entries with keep(i, x), in index order: emit(position, i, x) for
    // each, the positions counted from 0; returns how many. Blocks of 4 x 1024
    // entries (aligned rows) or 1024, each thread's entries consecutive and the
    // threads in order, so positions follow the index.
    template <class KEEP, class EMIT>
    MG_DEV int64_t sf_compact(const float *lr, int64_t V, bool al16, SfLds &L, KEEP keep, EMIT emit)
    {
        const int per = al16 ? 4 : 1;
        int64_t base = 0;
        for (int64_t i0 = 0; i0 < V; i0 += int64_t(kSfThreads) * per) {
            const int64_t j = i0 + int64_t(threadIdx.x) * per;
            float xs[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            if (al16 && j + 3 < V) {
                const Vec<float, 4> a = *reinterpret_cast<const Vec<float, 4> *>(lr + j);
#pragma unroll
                for (int e = 0; e < 4; ++e) xs[e] = a.v[e];
            } else {
                for (int e = 0; e < per; ++e)
                    if (j + e < V) xs[e] = lr[j + e];
            }
            bool ks[4];
            int cnt = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                ks[e] = e < per && j + e < V && keep(j + e, xs[e]);
                cnt += ks[e] ? 1 : 0;
            }
            int tot;
            int pos = sf_scan(cnt, L, &tot);
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (ks[e]) emit(base + pos++, j + e, xs[e]);
            base += tot;
        }
        return base;
    }

    // add one to cnt[bin] for every lane with `valid` (LDS atomics; a wave's
    // lanes on one bin serialize in the LDS, which measured cheaper here than
    // gathering equal bins by ballots first: a wave's 64 values spread over
    // ~16 top-byte bins)
    MG_DEV void sf_hist_add(uint32_t *cnt, uint32_t bin, bool valid)
    {
        if (valid) atomicAdd(&cnt[bin], 1u);
    }

    // The element of rank r (1-based) in (image desc, index asc) order among
    // the entries for which in(i, x) holds (at least r of them): its image in
    // *img and its index in *idx, so that the first r entries are those with
    // a larger image and those with an equal one at index <= *idx. Radix
    // passes over the image from the top byte; when the rank falls inside a
    // run of equal values, passes over the index among them from the top byte.
    template <class IN>
    MG_DEV void sf_select(const float *lr, int64_t V, bool al16, IN in, int64_t r, SfLds &L, uint32_t *img,
                          uint32_t *idx)
    {
        uint32_t pre = 0;
        int64_t rem = r;
        uint32_t ties = 0;
        for (int sh = 24; sh >= 0; sh -= 8) {
            for (int b = threadIdx.x; b < 256; b += kSfThreads) L.cnt[b] = 0;
            __syncthreads();
            const uint32_t hm = sh == 24 ? 0u : (0xffffffffu << (sh + 8));
            sf_each(lr, V, al16, [&](int64_t i, float x) {
                const uint32_t k = sf_img(x);
                sf_hist_add(L.cnt, (k >> sh) & 255u, in(i, x) && (k & hm) == pre);
            });
            __syncthreads();
            if (threadIdx.x == 0) {
                int64_t acc = 0;
                int b = 255;
                for (; b > 0; --b) {
                    if (acc + L.cnt[b] >= rem) break;
                    acc += L.cnt[b];
                }
                L.bc[0] = uint32_t(b);
                L.bc[1] = uint32_t(acc);
                L.bc[2] = L.cnt[b];
            }
            __syncthreads();
            pre |= L.bc[0] << sh;
            rem -= int64_t(L.bc[1]);
            ties = L.bc[2];
            __syncthreads();
        }
        *img = pre;
        if (int64_t(ties) == rem) { // every entry equal to the image is taken: no index cut
            *idx = 0xffffffffu;
            return;
        }
        uint32_t ipre = 0;
        for (int sh = 24; sh >= 0; sh -= 8) {
            for (int b = threadIdx.x; b < 256; b += kSfThreads) L.cnt[b] = 0;
            __syncthreads();
            const uint32_t hm = sh == 24 ? 0u : (0xffffffffu << (sh + 8));
            sf_each(lr, V, al16, [&](int64_t i, float x) {
                const uint32_t k = uint32_t(i);
                sf_hist_add(L.cnt, (k >> sh) & 255u, in(i, x) && sf_img(x) == pre && (k & hm) == ipre);
            });
            __syncthreads();
            if (threadIdx.x == 0) {
                int64_t acc = 0;
                int b = 0;
                for (; b < 255; ++b) {
                    if (acc + L.cnt[b] >= rem) break;
                    acc += L.cnt[b];
                }
                L.bc[0] = uint32_t(b);
                L.bc[1] = uint32_t(acc);
            }
            __syncthreads();
            ipre |= L.bc[0] << sh;
            rem -= int64_t(L.bc[1]);
            __syncthreads();
        }
        *idx = ipre;
    }

    __global__ __launch_bounds__(kSfThreads) void k_sample_rows(const float *__restrict__ lg, int64_t ld, int64_t V,
                                                               const int64_t *__restrict__ raw_amax, int64_t top_k,
                                                               float temperature, float top_p, float min_p,
                                                               int64_t *__restrict__ out_ids,
                                                               float *__restrict__ out_p, int64_t *__restrict__ out_n)
    {
        __shared__ SfLds L;
        const int64_t row = blockIdx.x;
        const float *lr = lg + row * ld;
        int64_t *oi = out_ids + row * V;
        float *op = out_p + row * V;
        const bool al16 = (reinterpret_cast<uintptr_t>(lr) & 15u) == 0;

        // sorted outputs (value order) when top_k > 0 or top_p < 1
        const bool sorted = top_k > 0 || top_p < 1.0f;
        constexpr int kBins = 1 << kHistBits;
        if (sorted) {
            for (int b = threadIdx.x; b < kBins; b += kSfThreads) L.hist[b] = 0;
            __syncthreads();
        }

        // pass 1: finite count, candidate count, the candidates' largest
        // image, np.argmax; for sorted outputs the candidates' image prefixes
        int64_t nfin = 0, nc = 0;
        uint32_t mk = 0; // image of the candidates' maximum (0: none)
        // the thread's first largest entry (image with NaN on top) and its
        // index: a thread visits its entries in index order
        uint32_t bg = 0, bi = 0xffffffffu;
        sf_each(lr, V, al16, [&](int64_t i, float x) {
            nfin += __builtin_isfinite(x) ? 1 : 0;
            const bool cand = sf_cand(x);
            const uint32_t img = sf_img(x);
            nc += cand ? 1 : 0;
            mk = cand && img > mk ? img : mk;
            if (sorted) atomicAdd(&L.hist[cand ? img >> (32 - kHistBits) : uint32_t(kBins)], 1u);
            const uint32_t g = x != x ? 0xffffffffu : img;
            if (g > bg) {
                bg = g;
                bi = uint32_t(i);
            }
        });
        nfin = int64_t(sf_sum_u64(uint64_t(nfin), L));
        nc = int64_t(sf_sum_u64(uint64_t(nc), L));
        // (image, ~index): the largest is np.argmax's entry
        const uint64_t best = sf_max_u64((uint64_t(bg) << 32) | uint64_t(0xffffffffu - bi), L);
        mk = uint32_t(sf_max_u64(mk, L));
        if (nfin == 0 || !(temperature > 0.0f)) {
            if (threadIdx.x == 0) {
                oi[0] = nfin == 0 && raw_amax ? raw_amax[row] : int64_t(0xffffffffu - uint32_t(best));
                op[0] = 1.0f;
                out_n[row] = 1;
            }
            return;
        }
        const float mx = key_f32(uint32_t(mk));
        if (!(mx < __builtin_huge_valf())) { // +inf among the candidates
            if (threadIdx.x == 0) out_n[row] = -1;
            return;
        }

        // the candidate set: the top_k largest when top_k < |C|
        const int64_t k = top_k > 0 ? (top_k < V ? top_k : V) : 0;
        uint32_t kimg = 0, kidx = 0xffffffffu;
        if (k > 0 && k < nc)
            sf_select(lr, V, al16, [](int64_t, float x) { return sf_cand(x); }, k, L, &kimg, &kidx);
        const int64_t ncand = k > 0 && k < nc ? k : nc;
        auto inC = [=](int64_t i, float x) {
            if (!sf_cand(x)) return false;
            const uint32_t g = sf_img(x);
            return g > kimg || (g == kimg && uint32_t(i) <= kidx);
        };

        // sorted outputs: the largest ng = min(|C|, kSortMax) entries of C,
        // which are the candidates' largest (C is a prefix of the candidates
        // in that order). They lie in the bins above bstar, the bin holding
        // the candidates' ng-th largest, and in bstar (every one of C when
        // ng = |C|): gathered when bstar holds at most kSortMax candidates.
        const int64_t ng = ncand < kSortMax ? ncand : kSortMax;
        const bool gall = ng == ncand;
        uint32_t bstar = 0;
        bool gather = false;
        if (sorted) {
            gather = true;
            if (!gall) {
                // thread t holds bins kBins-1-BPT*t-e: its exclusive prefix
                // counts the candidates in higher bins
                constexpr int BPT = kBins / kSfThreads;
                uint32_t c[BPT];
                int own = 0;
#pragma unroll
                for (int e = 0; e < BPT; ++e) {
                    c[e] = L.hist[kBins - 1 - BPT * int(threadIdx.x) - e];
                    own += int(c[e]);
                }
                int tot;
                int64_t acc = sf_scan(own, L, &tot);
#pragma unroll
                for (int e = 0; e < BPT; ++e) {
                    if (acc < ng && acc + c[e] >= ng) {
                        L.bc[0] = uint32_t(kBins - 1 - BPT * int(threadIdx.x) - e);
                        L.bc[1] = c[e];
                    }
                    acc += c[e];
                }
                __syncthreads();
                bstar = L.bc[0];
                gather = L.bc[1] <= uint32_t(kSortMax);
                __syncthreads();
            }
            if (threadIdx.x < 2) L.gcount[threadIdx.x] = 0;
            __syncthreads();
        }

        // S = sum of e over C (f64, fixed order), gathering alongside: region
        // 0 (keys[0, kSortMax)) the entries above bstar, or all of C; region
        // 1 (keys[kSortMax, 2 kSortMax)) those in bstar
        double S = 0.0;
        sf_each(lr, V, al16, [&](int64_t i, float x) {
            const bool in = inC(i, x);
            if (in) S += double(exp_diff(x, mx));
            if (gather) {
                const uint32_t img = sf_img(x), bin = img >> (32 - kHistBits);
                if (in && (gall || bin >= bstar)) {
                    const int reg = gall || bin > bstar ? 0 : 1;
                    const uint32_t at = atomicAdd(&L.gcount[reg], 1u);
                    L.keys[reg * kSortMax + int(at)] = (uint64_t(img) << 32) | uint64_t(0xffffffffu - uint32_t(i));
                }
            }
        });
        S = sf_sum_f64(S, L);
        // min_p: p >= min_p * max(p), p = e / S rounded to f32
        const float pmax = float(1.0 / S), thr = min_p * pmax;
        auto minp_ok = [=](float x) { return !(min_p > 0.0f) || float(double(exp_diff(x, mx)) / S) >= thr; };
        const float y0 = mx / temperature;

        if (!sorted) {
            // every candidate (top_k <= 0) passing min_p, in index order
            auto kept = [=](int64_t, float x) { return sf_cand(x) && minp_ok(x); };
            double F = 0.0;
            sf_each(lr, V, al16, [&](int64_t i, float x) {
                if (kept(i, x)) F += double(exp_diff(x / temperature, y0));
            });
            F = sf_sum_f64(F, L);
            const int64_t cnt = sf_compact(lr, V, al16, L, kept, [&](int64_t pos, int64_t i, float x) {
                oi[pos] = i;
                op[pos] = float(double(exp_diff(x / temperature, y0)) / F);
            });
            if (threadIdx.x == 0) out_n[row] = cnt;
            return;
        }

        // the sorted outputs' keys (value desc, index asc) in LDS, sorted; the
        // first ng are the largest ng of C
        if (gather) {
            // region 0 sorted; region 1 (the rest of the largest ng) sorted and
            // its largest ng - n0 appended (every one of them is below region
            // 0's keys: a lower bin)
            const int n0 = int(L.gcount[0]), n1 = gall ? 0 : int(L.gcount[1]);
            int p0 = 1, p1 = 1;
            while (p0 < n0) p0 <<= 1;
            while (p1 < n1) p1 <<= 1;
            for (int i = n0 + int(threadIdx.x); i < p0; i += kSfThreads) L.keys[i] = 0; // zeros sort last
            for (int i = n1 + int(threadIdx.x); i < p1; i += kSfThreads) L.keys[kSortMax + i] = 0;
            __syncthreads();
            sf_sort_desc(L.keys, p0);
            if (!gall) {
                sf_sort_desc(L.keys + kSortMax, p1);
                for (int i = threadIdx.x; i < int(ng) - n0; i += kSfThreads) L.keys[n0 + i] = L.keys[kSortMax + i];
                __syncthreads();
            }
        } else {
            int np2 = 1;
            // the threshold bin overflows the room: the ng-th largest of C by
            // radix passes, then C's entries up to it in index order
            uint32_t gimg = 0, gidx = 0xffffffffu;
            sf_select(lr, V, al16, inC, ng, L, &gimg, &gidx);
            for (int i = threadIdx.x; i < kSortMax; i += kSfThreads) L.keys[i] = 0;
            __syncthreads();
            sf_compact(
                lr, V, al16, L,
                [=](int64_t i, float x) {
                    if (!inC(i, x)) return false;
                    const uint32_t g = sf_img(x);
                    return g > gimg || (g == gimg && uint32_t(i) <= gidx);
                },
                [&](int64_t pos, int64_t i, float x) {
                    if (pos < kSortMax) L.keys[pos] = (uint64_t(sf_img(x)) << 32) | uint64_t(0xffffffffu - uint32_t(i));
                });
            while (np2 < ng) np2 <<= 1;
            __syncthreads();
            sf_sort_desc(L.keys, np2);
        }
        // the cut: thread t holds sorted entries 4t..4t+3
        const int t0 = 4 * int(threadIdx.x);
        float xv[4];
        double ev[4], own = 0.0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const bool in = t0 + e < ng;
            xv[e] = in ? key_f32(uint32_t(L.keys[t0 + e] >> 32)) : 0.0f;
            ev[e] = in ? double(exp_diff(xv[e], mx)) : 0.0;
            own += ev[e];
        }
        int64_t n = ncand;
        if (top_p < 1.0f) {
            // searchsorted(cumsum(p), top_p) + 1: the first position whose
            // cumulative e reaches top_p * S
            const double target = double(top_p) * S;
            double run = sf_scan_f64(own, L);
            uint64_t first = ~uint64_t(0);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                run += ev[e];
                if (t0 + e < ng && run >= target && first == ~uint64_t(0)) first = uint64_t(t0 + e);
            }
            first = sf_min_u64(first, L);
            if (first != ~uint64_t(0))
                n = int64_t(first) + 1;
            else if (ng < ncand)
                n = kSortMax + 1; // the cut lies beyond the gathered candidates
        }
        if (min_p > 0.0f) {
            // a prefix too: p falls along the sorted order
            int nm = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) nm += t0 + e < ng && minp_ok(xv[e]) ? 1 : 0;
            int64_t nmt = int64_t(sf_sum_u64(uint64_t(nm), L));
            if (nmt == ng && ng < ncand) nmt = kSortMax + 1; // min_p keeps past the gathered ones
            n = nmt < n ? nmt : n;
        }
        if (n > ng) {
            if (threadIdx.x == 0) out_n[row] = -1;
            return;
        }
        double F = 0.0;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (t0 + e < n) F += double(exp_diff(xv[e] / temperature, y0));
        F = sf_sum_f64(F, L);
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (t0 + e < n) {
                oi[t0 + e] = int64_t(0xffffffffu - uint32_t(L.keys[t0 + e]));
                op[t0 + e] = float(double(exp_diff(xv[e] / temperature, y0)) / F);
            }
        if (threadIdx.x == 0) out_n[row] = n;
    }

    void launch_sample_rows(mg_ctx *c, const float *lg, int64_t ld, int64_t rows, int64_t V,
                            const int64_t *raw_amax, int64_t top_k, double temperature, double top_p, double min_p,
                            int64_t *out_ids, float *out_p, int64_t *out_n)
    {
        need(rows >= 0 && V >= 1 && V < (int64_t(1) << 31), "sample_rows: V must be in [1, 2^31)");
        need(rows <= int64_t(0x7fffffff), "sample_rows: too many rows");
        need(lg && out_ids && out_p && out_n, "sample_rows: NULL tensor");
        if (ld == 0) ld = V;
        need(ld >= V, "sample_rows: row stride < V");
        if (rows == 0) return;
        hipLaunchKernelGGL(k_sample_rows, dim3(unsigned(rows)), dim3(kSfThreads), 0, c->stream, lg, ld, V, raw_amax,
                           top_k, float(temperature), float(top_p), float(min_p), out_ids, out_p, out_n);
        check_launch("k_sample_rows");
    }
} // namespace mg
