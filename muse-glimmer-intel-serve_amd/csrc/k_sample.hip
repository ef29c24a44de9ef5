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
    // one 1024-thread work-group per row of lg (f32, the edited logits), or,
    // for the rows the split section below takes, several per row.
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

    // work-group reduction scratch, and each kernel's LDS around it
    struct SfRed
    {
        double red[kSfThreads];
        double redd[kSfThreads / 64];
        uint64_t redu[kSfThreads / 64];
        uint32_t bc[4];     // broadcast words
        uint32_t bslice[8]; // per-slice broadcast words (split rows)
    };
    struct SfLds : SfRed
    {
        uint32_t cnt[256];
        uint32_t hist[(1 << kHistBits) + 1]; // the last: a spare bin for non-candidates
        uint64_t keys[kGatherCap];
        uint32_t gcount[2]; // keys gathered so far above the threshold bin, in it
    };

    MG_DEV uint32_t sf_img(float x) { return f32_key(x + 0.0f); } // -0 ranks with +0
    MG_DEV bool sf_cand(float x) { return x > -__builtin_huge_valf(); } // NaN and -inf fail

    // work-group sums in a fixed order (every thread returns the total)
    MG_DEV double sf_sum_f64(double v, SfRed &L)
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
    MG_DEV uint64_t sf_red_u64(uint64_t v, SfRed &L, OP op)
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
    MG_DEV uint64_t sf_sum_u64(uint64_t v, SfRed &L)
    {
        return sf_red_u64(v, L, [](uint64_t a, uint64_t b) { return a + b; });
    }
    MG_DEV uint64_t sf_max_u64(uint64_t v, SfRed &L)
    {
        return sf_red_u64(v, L, [](uint64_t a, uint64_t b) { return a > b ? a : b; });
    }
    MG_DEV uint64_t sf_min_u64(uint64_t v, SfRed &L)
    {
        return sf_red_u64(v, L, [](uint64_t a, uint64_t b) { return a < b ? a : b; });
    }
    // exclusive prefix over the work-group in thread order; total in *tot
    MG_DEV int sf_scan(int v, SfRed &L, int *tot)
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
    MG_DEV double sf_scan_f64(double v, SfRed &L)
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

    // The sorted outputs from keys[0, ng) (LDS), C's largest ng in (value
    // desc, index asc) order (ncand = |C|, S its e sum, mx its maximum): the
    // top_p and min_p cuts as prefixes of that order, then softmax(x / T)
    // over the kept prefix into oi / op and its length into *out_n (-1 when
    // the cut lies past the ng keys at hand).
    MG_DEV void sf_emit_sorted(SfRed &L, const uint64_t *keys, int64_t ng, int64_t ncand, double S, float mx,
                               float temperature, float top_p, float min_p, int64_t *oi, float *op, int64_t *out_n)
    {
        const float pmax = float(1.0 / S), thr = min_p * pmax;
        auto minp_ok = [=](float x) { return !(min_p > 0.0f) || float(double(exp_diff(x, mx)) / S) >= thr; };
        const float y0 = mx / temperature;
        // thread t holds sorted entries 4t..4t+3
        const int t0 = 4 * int(threadIdx.x);
        float xv[4];
        double ev[4], own = 0.0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const bool in = t0 + e < ng;
            xv[e] = in ? key_f32(uint32_t(keys[t0 + e] >> 32)) : 0.0f;
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
            if (threadIdx.x == 0) *out_n = -1;
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
                oi[t0 + e] = int64_t(0xffffffffu - uint32_t(keys[t0 + e]));
                op[t0 + e] = float(double(exp_diff(xv[e] / temperature, y0)) / F);
            }
        if (threadIdx.x == 0) *out_n = n;
    }

    // region 0 (keys[0, n0)) sorted; region 1 (keys[kSortMax, kSortMax + n1)),
    // when two, sorted too and, unless ng < 0, its largest ng - n0 appended
    // to region 0 (every key of region 1 lies below region 0's)
    MG_DEV void sf_sort_regions(uint64_t *keys, int n0, int n1, int64_t ng, bool two)
    {
        int p0 = 1, p1 = 1;
        while (p0 < n0) p0 <<= 1;
        while (p1 < n1) p1 <<= 1;
        for (int i = n0 + int(threadIdx.x); i < p0; i += kSfThreads) keys[i] = 0; // zeros sort last
        if (two)
            for (int i = n1 + int(threadIdx.x); i < p1; i += kSfThreads) keys[kSortMax + i] = 0;
        __syncthreads();
        sf_sort_desc(keys, p0);
        if (two) {
            sf_sort_desc(keys + kSortMax, p1);
            if (ng >= 0) {
                for (int i = threadIdx.x; i < int(ng) - n0; i += kSfThreads) keys[n0 + i] = keys[kSortMax + i];
                __syncthreads();
            }
        }
    }

    // row `row` of lg, one work-group; S_given >= 0 is C's e sum as another
    // path summed it (then used in place of this one's, so a row gets the same
    // bits whichever path finishes it)
    MG_DEV void sample_row(SfLds &L, int64_t row, const float *__restrict__ lg, int64_t ld, int64_t V,
                           const int64_t *__restrict__ raw_amax, int64_t top_k, float temperature, float top_p,
                           float min_p, int64_t *__restrict__ out_ids, float *__restrict__ out_p,
                           int64_t *__restrict__ out_n, double S_given = -1.0)
    {
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
        if (gather || !(S_given >= 0.0)) {
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
        }
        if (S_given >= 0.0) S = S_given;

        if (!sorted) {
            // min_p: p >= min_p * max(p), p = e / S rounded to f32
            const float pmax = float(1.0 / S), thr = min_p * pmax;
            auto minp_ok = [=](float x) { return !(min_p > 0.0f) || float(double(exp_diff(x, mx)) / S) >= thr; };
            const float y0 = mx / temperature;
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
            sf_sort_regions(L.keys, int(L.gcount[0]), gall ? 0 : int(L.gcount[1]), ng, !gall);
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
        sf_emit_sorted(L, L.keys, ng, ncand, S, mx, temperature, top_p, min_p, oi, op, out_n + row);
    }

    __global__ __launch_bounds__(kSfThreads) void k_sample_rows(const float *__restrict__ lg, int64_t ld, int64_t V,
                                                               const int64_t *__restrict__ raw_amax, int64_t top_k,
                                                               float temperature, float top_p, float min_p,
                                                               int64_t *__restrict__ out_ids,
                                                               float *__restrict__ out_p, int64_t *__restrict__ out_n)
    {
        __shared__ SfLds L;
        sample_row(L, blockIdx.x, lg, ld, V, raw_amax, top_k, temperature, top_p, min_p, out_ids, out_p, out_n);
    }

    // ------------------------------------------------ split rows (sorted, no top_k cut)
    // Rows with sorted outputs and every candidate in C (top_k <= 0 or >= V)
    // split over G work-groups per row, one slice of slen entries each (64
    // rows then fill the chip): pass 1 per slice with its prefix histogram
    // (k_sample_split_stats), the row's decision from the slices' counts
    // (k_sample_split_decide: the point masses, the threshold bin bstar, and
    // where each slice's keys go), S per slice with the gathering into the
    // row's two key regions at those offsets (k_sample_split_gather, no
    // atomics between work-groups), the sort and cut per row
    // (k_sample_split_finish). A row whose threshold bin holds more than
    // kSortMax candidates is marked 2, and the finishing work-group runs the
    // one-work-group algorithm (sample_row) on it instead, with the S the
    // slices summed: the same selection and the same bits as the split path's.
    constexpr int kSplitMax = 8; // work-groups per row
    static_assert(kSplitMax <= int(sizeof(SfRed::bslice) / sizeof(uint32_t)), "a broadcast word per slice");

    struct SplitStat
    {
        uint64_t nfin, nc, best; // best: (image with NaN on top) << 32 | ~index
        uint32_t mk, pad;
    };
    struct SplitRow
    {
        float mx;
        uint32_t bstar;
        int32_t gall, pad;
        int64_t ncand;
        uint32_t n0, n1;               // keys in regions 0 and 1
        uint32_t off0[kSplitMax], off1[kSplitMax];
    };
    struct SplitWork
    {
        SplitStat *stat;  // [rows][G]
        uint32_t *hist;   // [rows][G][2^kHistBits]
        SplitRow *prm;    // [rows]
        int32_t *flag;    // [rows]: 0 finished, 1 split path, 2 left to k_sample_rows
        double *spart;    // [rows][G]
        uint64_t *keys;   // [rows][2 kSortMax]
        int64_t slen;     // entries per slice (a multiple of 4)
    };

    struct SfHistLds : SfRed
    {
        uint32_t hist[(1 << kHistBits) + 1]; // the last: a spare bin for non-candidates
    };
    struct SfKeysLds : SfRed
    {
        uint64_t keys[kGatherCap];
        uint32_t gcount[2];
    };
    struct SfMergeLds : SfRed
    {
        uint64_t keys[kGatherCap];
        uint64_t merged[kSortMax];
    };

    __global__ __launch_bounds__(kSfThreads) void k_sample_split_stats(const float *__restrict__ lg, int64_t ld,
                                                                      int64_t V, SplitWork w)
    {
        __shared__ SfHistLds L;
        constexpr int kBins = 1 << kHistBits;
        const int G = int(gridDim.x), g = int(blockIdx.x);
        const int64_t row = blockIdx.y;
        const int64_t base = int64_t(g) * w.slen;
        const int64_t len = base < V ? (V - base < w.slen ? V - base : w.slen) : 0;
        const float *lr = lg + row * ld + base;
        const bool al16 = (reinterpret_cast<uintptr_t>(lr) & 15u) == 0;
        for (int b = threadIdx.x; b < kBins; b += kSfThreads) L.hist[b] = 0;
        __syncthreads();
        int64_t nfin = 0, nc = 0;
        uint32_t mk = 0, bg = 0, bi = 0xffffffffu;
        sf_each(lr, len, al16, [&](int64_t i, float x) {
            nfin += __builtin_isfinite(x) ? 1 : 0;
            const bool cand = sf_cand(x);
            const uint32_t img = sf_img(x);
            nc += cand ? 1 : 0;
            mk = cand && img > mk ? img : mk;
            atomicAdd(&L.hist[cand ? img >> (32 - kHistBits) : uint32_t(kBins)], 1u);
            const uint32_t gg = x != x ? 0xffffffffu : img;
            if (gg > bg) {
                bg = gg;
                bi = uint32_t(base + i);
            }
        });
        nfin = int64_t(sf_sum_u64(uint64_t(nfin), L));
        nc = int64_t(sf_sum_u64(uint64_t(nc), L));
        const uint64_t best = sf_max_u64((uint64_t(bg) << 32) | uint64_t(0xffffffffu - bi), L);
        mk = uint32_t(sf_max_u64(mk, L));
        const int64_t sl = row * G + g;
        if (threadIdx.x == 0) w.stat[sl] = SplitStat{uint64_t(nfin), uint64_t(nc), best, mk, 0u};
        uint32_t *h = w.hist + sl * kBins;
        for (int b = threadIdx.x; b < kBins; b += kSfThreads) h[b] = L.hist[b];
    }

    __global__ __launch_bounds__(kSfThreads) void k_sample_split_decide(int64_t V, const int64_t *__restrict__ raw_amax,
                                                                       int G, float temperature,
                                                                       int64_t *__restrict__ out_ids,
                                                                       float *__restrict__ out_p,
                                                                       int64_t *__restrict__ out_n, SplitWork w)
    {
        __shared__ SfRed L;
        constexpr int kBins = 1 << kHistBits;
        constexpr int BPT = kBins / kSfThreads;
        const int64_t row = blockIdx.x;
        // every request first, so that the slices' counts and histograms come
        // back in one trip: lane g < G of each wave fetches slice g's counts
        // (read across the wave below), and thread t bins kBins-1-BPT*t-e of
        // every slice (slices past G re-read the last and count nothing)
        const int lane = int(threadIdx.x) & 63;
        const SplitStat my = w.stat[row * G + (lane < G ? lane : G - 1)];
        const uint32_t *h = w.hist + row * G * kBins;
        uint32_t hv[kSplitMax][BPT];
#pragma unroll
        for (int g = 0; g < kSplitMax; ++g)
#pragma unroll
            for (int e = 0; e < BPT; ++e)
                hv[g][e] = h[(g < G ? g : G - 1) * kBins + kBins - 1 - BPT * int(threadIdx.x) - e];
        auto rd64 = [](uint64_t v, int l) {
            return uint64_t(uint32_t(__builtin_amdgcn_readlane(int(uint32_t(v)), l))) |
                   (uint64_t(uint32_t(__builtin_amdgcn_readlane(int(uint32_t(v >> 32)), l))) << 32);
        };
        // the slices' counts, folded in slice order by every thread alike
        int64_t nfin = 0, nc = 0;
        uint64_t best = 0;
        uint32_t mk = 0;
        int64_t ncs[kSplitMax];
#pragma unroll
        for (int g = 0; g < kSplitMax; ++g) {
            const bool live = g < G;
            const int64_t tn = int64_t(rd64(my.nfin, g)), tc = int64_t(rd64(my.nc, g));
            const uint64_t tb = rd64(my.best, g);
            const uint32_t tm = uint32_t(__builtin_amdgcn_readlane(int(my.mk), g));
            nfin += live ? tn : 0;
            nc += live ? tc : 0;
            ncs[g] = live ? tc : 0;
            best = live && tb > best ? tb : best;
            mk = live && tm > mk ? tm : mk;
        }
        // the bins summed over the slices and their prefix from the top, for
        // every row alike (rows that need no threshold leave them unused)
        uint32_t c[BPT];
        int own = 0;
#pragma unroll
        for (int e = 0; e < BPT; ++e) {
            c[e] = 0;
#pragma unroll
            for (int g = 0; g < kSplitMax; ++g) c[e] += g < G ? hv[g][e] : 0u;
            own += int(c[e]);
        }
        int tot;
        int64_t acc = sf_scan(own, L, &tot);
        int64_t *oi = out_ids + row * V;
        float *op = out_p + row * V;
        if (nfin == 0 || !(temperature > 0.0f)) {
            if (threadIdx.x == 0) {
                oi[0] = nfin == 0 && raw_amax ? raw_amax[row] : int64_t(0xffffffffu - uint32_t(best));
                op[0] = 1.0f;
                out_n[row] = 1;
                w.flag[row] = 0;
            }
            return;
        }
        const float mx = key_f32(mk);
        if (!(mx < __builtin_huge_valf())) { // +inf among the candidates
            if (threadIdx.x == 0) {
                out_n[row] = -1;
                w.flag[row] = 0;
            }
            return;
        }
        const int64_t ng = nc < kSortMax ? nc : kSortMax;
        const bool gall = ng == nc;
        SplitRow r{};
        r.mx = mx;
        r.gall = gall ? 1 : 0;
        r.ncand = nc;
        if (gall) {
            // every candidate into region 0, slice by slice
            uint32_t at = 0;
#pragma unroll
            for (int g = 0; g < kSplitMax; ++g) {
                r.off0[g] = at;
                at += uint32_t(ncs[g]);
            }
            r.n0 = at;
        } else {
#pragma unroll
            for (int e = 0; e < BPT; ++e) {
                if (acc < ng && acc + c[e] >= ng) {
                    L.bc[0] = uint32_t(kBins - 1 - BPT * int(threadIdx.x) - e);
                    L.bc[1] = c[e];
                }
                acc += c[e];
            }
            __syncthreads();
            const uint32_t bstar = L.bc[0], inb = L.bc[1];
            __syncthreads();
            if (inb > uint32_t(kSortMax)) {
                // left to the one-work-group algorithm; the gathering kernel
                // still sums S by slices (mx)
                if (threadIdx.x == 0) {
                    w.prm[row] = r;
                    w.flag[row] = 2;
                }
                return;
            }
            // each slice's keys above bstar and in it, in slice order: the keys
            // above number fewer than ng <= kSortMax in all, so every partial
            // count of a slice fits 16 bits and four slices' counts travel in
            // one 64-bit sum; thread g < G fetches slice g's bstar bin, all G
            // requests in flight together, published by the sum's barriers
            const bool fetch = int(threadIdx.x) < G;
            const uint32_t nbl = h[(fetch ? int(threadIdx.x) : 0) * kBins + bstar];
            uint64_t ab[2] = {0, 0};
#pragma unroll
            for (int g = 0; g < kSplitMax; ++g) {
                uint32_t above = 0;
#pragma unroll
                for (int e = 0; e < BPT; ++e)
                    above += g < G && uint32_t(kBins - 1 - BPT * int(threadIdx.x) - e) > bstar ? hv[g][e] : 0u;
                ab[g / 4] += uint64_t(above) << (16 * (g % 4));
            }
            if (fetch) L.bslice[threadIdx.x] = nbl;
            ab[0] = sf_sum_u64(ab[0], L);
            if (G > 4) ab[1] = sf_sum_u64(ab[1], L);
            uint32_t a0 = 0, a1 = 0;
#pragma unroll
            for (int g = 0; g < kSplitMax; ++g) {
                if (g < G) {
                    const uint32_t na = uint32_t(ab[g / 4] >> (16 * (g % 4))) & 0xffffu;
                    r.off0[g] = a0;
                    r.off1[g] = a1;
                    a0 += na;
                    a1 += L.bslice[g];
                }
            }
            r.bstar = bstar;
            r.n0 = a0;
            r.n1 = a1;
        }
        if (threadIdx.x == 0) {
            w.prm[row] = r;
            w.flag[row] = 1;
        }
    }

    // S over the slice and its gathered keys, sorted in LDS, written as the
    // slice's runs of the row's two regions
    __global__ __launch_bounds__(kSfThreads) void k_sample_split_gather(const float *__restrict__ lg, int64_t ld,
                                                                       int64_t V, SplitWork w)
    {
        __shared__ SfKeysLds L;
        const int G = int(gridDim.x), g = int(blockIdx.x);
        const int64_t row = blockIdx.y;
        const int32_t flag = w.flag[row];
        if (flag != 1 && flag != 2) return;
        const SplitRow &r = w.prm[row]; // read in place (uniform loads)
        const int64_t base = int64_t(g) * w.slen;
        const int64_t len = base < V ? (V - base < w.slen ? V - base : w.slen) : 0;
        const float *lr = lg + row * ld + base;
        const bool al16 = (reinterpret_cast<uintptr_t>(lr) & 15u) == 0;
        if (threadIdx.x < 2) L.gcount[threadIdx.x] = 0;
        __syncthreads();
        const bool gall = r.gall != 0, gather = flag == 1;
        const float mx = r.mx;
        const uint32_t bstar = r.bstar;
        double S = 0.0;
        sf_each(lr, len, al16, [&](int64_t i, float x) {
            if (!sf_cand(x)) return;
            S += double(exp_diff(x, mx));
            const uint32_t img = sf_img(x), bin = img >> (32 - kHistBits);
            if (gather && (gall || bin >= bstar)) {
                const int reg = gall || bin > bstar ? 0 : 1;
                const uint32_t at = atomicAdd(&L.gcount[reg], 1u);
                L.keys[reg * kSortMax + int(at)] = (uint64_t(img) << 32) | uint64_t(0xffffffffu - uint32_t(base + i));
            }
        });
        S = sf_sum_f64(S, L); // (its barriers also publish the gathered keys)
        if (threadIdx.x == 0) w.spart[row * G + g] = S;
        if (!gather) return;
        const int n0 = int(L.gcount[0]), n1 = gall ? 0 : int(L.gcount[1]);
        sf_sort_regions(L.keys, n0, n1, -1, !gall);
        uint64_t *k0 = w.keys + row * (2 * kSortMax) + r.off0[g];
        uint64_t *k1 = w.keys + row * (2 * kSortMax) + kSortMax + r.off1[g];
        for (int i = threadIdx.x; i < n0; i += kSfThreads) k0[i] = L.keys[i];
        for (int i = threadIdx.x; i < n1; i += kSfThreads) k1[i] = L.keys[kSortMax + i];
    }

    // keys[0, n) as G descending runs (run q from off[q] to off[q+1], off[G]
    // = n): every key to its place in their merged order, when below lim
    // (its place is its index in its run plus, in every other run, the number
    // of larger keys: the keys are unique)
    MG_DEV void sf_merge_runs(const uint64_t *keys, int n, const uint32_t *off, int G, int lim, uint64_t *dst,
                              int at)
    {
        for (int i = threadIdx.x; i < n; i += kSfThreads) {
            const uint64_t k = keys[i];
            int pos = 0;
            for (int q = 0; q < G; ++q) {
                const int lo = int(off[q]), hi = q + 1 < G ? int(off[q + 1]) : n;
                if (i >= lo && i < hi) {
                    pos += i - lo;
                    continue;
                }
                // larger keys of run q: a prefix, found by bisection
                int a = lo, b = hi;
                while (a < b) {
                    const int m = (a + b) >> 1;
                    if (keys[m] > k)
                        a = m + 1;
                    else
                        b = m;
                }
                pos += a - lo;
            }
            if (pos < lim) dst[at + pos] = k;
        }
    }

    __global__ __launch_bounds__(kSfThreads) void k_sample_split_finish(const float *__restrict__ lg, int64_t ld,
                                                                       int64_t V, const int64_t *__restrict__ raw_amax,
                                                                       int64_t top_k, int G, float temperature,
                                                                       float top_p, float min_p,
                                                                       int64_t *__restrict__ out_ids,
                                                                       float *__restrict__ out_p,
                                                                       int64_t *__restrict__ out_n, SplitWork w)
    {
        __shared__ union
        {
            SfMergeLds m;
            SfLds full;
        } U;
        const int64_t row = blockIdx.x;
        const int32_t flag = w.flag[row];
        if (flag == 2) {
            double S = 0.0;
            for (int g = 0; g < G; ++g) S += w.spart[row * G + g];
            sample_row(U.full, row, lg, ld, V, raw_amax, top_k, temperature, top_p, min_p, out_ids, out_p, out_n, S);
            return;
        }
        if (flag != 1) return;
        SfMergeLds &L = U.m;
        const SplitRow &r = w.prm[row]; // read in place (uniform loads)
        double S = 0.0;
        for (int g = 0; g < G; ++g) S += w.spart[row * G + g];
        const int64_t ng = r.ncand < kSortMax ? r.ncand : kSortMax;
        const int n0 = int(r.n0), n1 = r.gall ? 0 : int(r.n1);
        const uint64_t *src = w.keys + row * (2 * kSortMax);
        for (int i = threadIdx.x; i < n0; i += kSfThreads) L.keys[i] = src[i];
        for (int i = threadIdx.x; i < n1; i += kSfThreads) L.keys[kSortMax + i] = src[kSortMax + i];
        __syncthreads();
        // region 0's runs merged in full, region 1's largest ng - n0 after them
        sf_merge_runs(L.keys, n0, r.off0, G, n0, L.merged, 0);
        if (n1 > 0) sf_merge_runs(L.keys + kSortMax, n1, r.off1, G, int(ng) - n0, L.merged, n0);
        __syncthreads();
        sf_emit_sorted(L, L.merged, ng, r.ncand, S, r.mx, temperature, top_p, min_p, out_ids + row * V,
                       out_p + row * V, out_n + row);
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
        const float T = float(temperature), tp = float(top_p), mp = float(min_p);
        // the split path: sorted outputs with no top_k cut, few enough rows that
        // G >= 2 work-groups per row fill the chip, and room in the workspace
        const bool sorted = top_k > 0 || tp < 1.0f;
        const int G = int(rows <= 256 / kSplitMax ? kSplitMax : 256 / rows);
        constexpr int64_t kBins = int64_t(1) << kHistBits;
        auto al = [](int64_t b) { return (b + 255) / 256 * 256; };
        const int64_t b_stat = al(rows * G * int64_t(sizeof(SplitStat))), b_hist = al(rows * G * kBins * 4),
                      b_prm = al(rows * int64_t(sizeof(SplitRow))), b_flag = al(rows * 4), b_sp = al(rows * G * 8),
                      b_keys = al(rows * 2 * kSortMax * 8);
        const bool split = sorted && (top_k <= 0 || top_k >= V) && G >= 2 && V >= 4 * 4096 &&
                           b_stat + b_hist + b_prm + b_flag + b_sp + b_keys <= c->work_bytes;
        if (!split) {
            hipLaunchKernelGGL(k_sample_rows, dim3(unsigned(rows)), dim3(kSfThreads), 0, c->stream, lg, ld, V,
                               raw_amax, top_k, T, tp, mp, out_ids, out_p, out_n);
            check_launch("k_sample_rows");
            return;
        }
        char *wb = static_cast<char *>(c->work);
        SplitWork w;
        w.stat = reinterpret_cast<SplitStat *>(wb);
        w.hist = reinterpret_cast<uint32_t *>(wb + b_stat);
        w.prm = reinterpret_cast<SplitRow *>(wb + b_stat + b_hist);
        w.flag = reinterpret_cast<int32_t *>(wb + b_stat + b_hist + b_prm);
        w.spart = reinterpret_cast<double *>(wb + b_stat + b_hist + b_prm + b_flag);
        w.keys = reinterpret_cast<uint64_t *>(wb + b_stat + b_hist + b_prm + b_flag + b_sp);
        w.slen = (V + 4 * G - 1) / (4 * G) * 4;
        const dim3 gs{unsigned(G), unsigned(rows), 1u};
        hipLaunchKernelGGL(k_sample_split_stats, gs, dim3(kSfThreads), 0, c->stream, lg, ld, V, w);
        check_launch("k_sample_split_stats");
        hipLaunchKernelGGL(k_sample_split_decide, dim3(unsigned(rows)), dim3(kSfThreads), 0, c->stream, V, raw_amax, G,
                           T, out_ids, out_p, out_n, w);
        check_launch("k_sample_split_decide");
        hipLaunchKernelGGL(k_sample_split_gather, gs, dim3(kSfThreads), 0, c->stream, lg, ld, V, w);
        check_launch("k_sample_split_gather");
        hipLaunchKernelGGL(k_sample_split_finish, dim3(unsigned(rows)), dim3(kSfThreads), 0, c->stream, lg, ld, V,
                           raw_amax, top_k, G, T, tp, mp, out_ids, out_p, out_n, w);
        check_launch("k_sample_split_finish");
    }
} // namespace mg
