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
//           descending, then index ascending (-0 and +0 are equal values).
//           NaN entries rank below -inf.
//
// Every (value, index) packs into one 64-bit key: an order-preserving image of
// the f32 value (NaN -> 0, -0 -> +0) above the complement of the index. Keys
// are unique and "the K largest keys" is exactly the order above, so every
// selection below is deterministic however the work is split.
//
// Pass 1 (k_vocab_chunk): one wave per 2048-key chunk, 32 keys per lane held
// in registers, no block barriers. Per chunk: the finite max, the sum of
// exp(x - max) (f32 terms and lane sums, f64 across lanes), the first index of
// the max, and the chunk's top-K keys sorted descending. The top-K (K <= 64)
// uses a bound that cannot miss: every lane keeps its two largest values, and
// the K-th largest of those 128 values has at least K elements at or above it,
// so all top-K elements are candidates; for random logits about K + K/8 pass.
// They are compacted through a ballot into LDS and bitonic-sorted in registers.
// A chunk whose bound is -inf or lets more than 128 candidates through, and
// every chunk when K > 64, selects the exact K-th key by bisection instead.
// Pass 2 (k_vocab_merge): one wave per row. lse and argmax fold the chunk
// partials (f64, FDLIBM exp/log). The row's top-K is selected from the first
// 8 keys of every chunk list; that is the exact answer when every list's 9th
// key (the first one left out) is below the selected K-th key, since deeper
// keys are smaller still. Otherwise the selection runs over the full lists.
#include "mg_device.hpp"
#include "mg_internal.hpp"

namespace mg
{
    constexpr int kVLane = 32;           // keys per lane in pass 1
    constexpr int kVChunk = 64 * kVLane; // 2048 keys per wave-chunk
    constexpr int kMaxK = 256;
    constexpr int kFastK = 64;           // pass 1 bound-based selection up to this K
    constexpr int kDepth = 8;            // pass 2: keys taken from each chunk list first
    constexpr int kMergeRegs = 16;       // pass 2: candidate keys per lane (1024 per row)

    struct VPart
    {
        double l;    // sum over the chunk's finite x of exp(x - m)
        float m;     // max of the chunk's finite x
        float bv;    // argmax value
        int32_t bi;  // argmax index (-1: the chunk holds only NaN)
        int32_t fin; // 1 if the chunk holds a finite entry
        int32_t nk;  // keys in the chunk's list: min(valid entries, K)
        int32_t pad;
    };

    // order-preserving 32-bit image of a logit: NaN lowest (1, below -inf's
    // 0x007fffff), -0 == +0; 0 marks an empty slot
    MG_DEV uint32_t vhi(float x)
    {
        return x != x ? 1u : f32_key(x + 0.0f);
    }
    MG_DEV uint64_t vkey(uint32_t hi, uint32_t j)
    {
        return (uint64_t(hi) << 32) | uint64_t(0xffffffffu - j);
    }
    MG_DEV uint32_t vkey_index(uint64_t k)
    {
        return 0xffffffffu - uint32_t(k);
    }

    // (value, index) argmax rule of the '>' scan: a beats b
    MG_DEV bool beats(float av, int ai, float bv, int bi)
    {
        if (ai < 0) return false;
        if (bi < 0) return true;
        return av > bv || (av == bv && ai < bi);
    }

    MG_DEV int wave_sum_i(int v)
    {
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
        return v;
    }
    MG_DEV int wave_min_i(int v)
    {
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
            const int o = __shfl_xor(v, m, 64);
            v = o < v ? o : v;
        }
        return v;
    }
    MG_DEV uint32_t wave_max_u32(uint32_t v)
    {
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
            const uint32_t o = __shfl_xor(v, m, 64);
            v = o > v ? o : v;
        }
        return v;
    }
    MG_DEV uint32_t wave_min_u32(uint32_t v)
    {
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
            const uint32_t o = __shfl_xor(v, m, 64);
            v = o < v ? o : v;
        }
        return v;
    }

    // Descending bitonic sort of the 64*SL values a wave holds SL per lane
    // (slot SL*lane + q in a[q]). Ascending/descending runs of the network are
    // chosen per slot; partners at distance >= SL live in lane ^ (j / SL).
    template <typename T, int SL>
    MG_DEV void wave_sort_desc(T (&a)[SL])
    {
        const int lane = threadIdx.x & 63;
        constexpr int N = 64 * SL;
#pragma unroll
        for (int k = 2; k <= N; k <<= 1) {
#pragma unroll
            for (int j = k >> 1; j > 0; j >>= 1) {
                if (j < SL) {
#pragma unroll
                    for (int q = 0; q < SL; ++q) {
                        const int p = q ^ j;
                        if (p > q) {
                            const bool desc = ((SL * lane + q) & k) == 0;
                            const T x = a[q], y = a[p];
                            const bool sw = desc ? (x < y) : (x > y);
                            a[q] = sw ? y : x;
                            a[p] = sw ? x : y;
                        }
                    }
                } else {
                    const int lj = j / SL;
                    const bool lower = (lane & lj) == 0;
#pragma unroll
                    for (int q = 0; q < SL; ++q) {
                        const T o = __shfl_xor(a[q], lj, 64);
                        const bool desc = ((SL * lane + q) & k) == 0;
                        const bool keep_max = lower == desc;
                        a[q] = keep_max ? (a[q] > o ? a[q] : o) : (a[q] < o ? a[q] : o);
                    }
                }
            }
        }
    }

    // LDS writes of one wave made visible to the same wave's later reads
    MG_DEV void wave_lds_sync()
    {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }

    MG_DEV int lane_rank(uint64_t mask)
    {
        return int(__builtin_amdgcn_mbcnt_hi(uint32_t(mask >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(mask), 0u)));
    }

    // ------------------------------------------------------------------ pass 1
    // lane element s sits at chunk offset VW*lane + 64*VW*(s/VW) + s%VW: VW
    // consecutive elements per 16-byte load, a wave covering 1 KiB per load
    template <int VW>
    MG_DEV int voff(int lane, int s)
    {
        return VW * lane + 64 * VW * (s / VW) + (s % VW);
    }

    template <class SI, int VW, int SL>
    __global__ __launch_bounds__(256) void k_vocab_chunk(const typename SI::raw *__restrict__ L, int64_t V, int K,
                                                         int nch, VPart *__restrict__ part,
                                                         uint64_t *__restrict__ cand)
    {
        using raw = typename SI::raw;
        __shared__ uint64_t slots[4][64 * SL];
        const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
        const int ch = int(blockIdx.x) * 4 + wv;
        const int64_t row = blockIdx.y;
        if (ch >= nch) return; // the whole wave leaves; nothing below syncs the block
        const int64_t cb = int64_t(ch) * kVChunk;
        const int nvalid = int(V - cb < kVChunk ? V - cb : kVChunk);
        const bool full = nvalid == kVChunk;
        const raw *xr = L + row * V + cb;

        float x[kVLane];
        bool loaded = false;
        if constexpr (VW > 1) {
            if (full) {
#pragma unroll
                for (int i = 0; i < kVLane / VW; ++i) {
                    const Vec<raw, VW> v = ld16_stream<raw, VW>(xr + VW * lane + 64 * VW * i);
#pragma unroll
                    for (int e = 0; e < VW; ++e) x[VW * i + e] = float(SI::dec(v.v[e]));
                }
                loaded = true;
            }
        }
        if (!loaded) {
            // tail chunk (or unaligned rows): -inf placeholders past V never
            // reach a sum, a max or the candidates, and are kept out of the
            // argmax and the exact selection by index
#pragma unroll
            for (int s = 0; s < kVLane; ++s) {
                const int o = voff<VW>(lane, s);
                x[s] = o < nvalid ? float(SI::dec(xr[o])) : -__builtin_huge_valf();
            }
        }

        // lane maximum and second maximum (two distinct elements), NaN/+inf flag
        float m1 = -__builtin_huge_valf(), m2 = -__builtin_huge_valf();
        bool sp = false;
#pragma unroll
        for (int s = 0; s < kVLane; ++s) {
            sp |= !(x[s] < __builtin_huge_valf());
            m2 = __builtin_fmaxf(m2, __builtin_fminf(m1, x[s]));
            m1 = __builtin_fmaxf(m1, x[s]);
        }
        const bool special = __builtin_amdgcn_ballot_w64(sp) != 0;
        if (special) {
            // NaN would pass through fminf as the other operand: redo with NaN
            // as -inf (it is never a candidate element)
            m1 = m2 = -__builtin_huge_valf();
#pragma unroll
            for (int s = 0; s < kVLane; ++s) {
                const float v = x[s] == x[s] ? x[s] : -__builtin_huge_valf();
                m2 = __builtin_fmaxf(m2, __builtin_fminf(m1, v));
                m1 = __builtin_fmaxf(m1, v);
            }
        }
        const float MX = wave_max(m1); // max over non-NaN entries (+inf included)

        // argmax: the first index holding MX
        int first = 0x7fffffff;
#pragma unroll
        for (int s = kVLane - 1; s >= 0; --s)
            if (x[s] == MX) first = voff<VW>(lane, s);
        first = wave_min_i(first);
        const int bi = first < nvalid ? int(cb) + first : -1;

        // lse partial over the finite entries
        float FM = MX;
        if (special) {
            float fm = -__builtin_huge_valf();
#pragma unroll
            for (int s = 0; s < kVLane; ++s)
                if (__builtin_isfinite(x[s])) fm = __builtin_fmaxf(fm, x[s]);
            FM = wave_max(fm);
        }
        const bool fin = FM > -__builtin_huge_valf();
        float ls = 0.0f;
        if (fin) {
            constexpr float c = 1.44269504088896341f;
            float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            if (!special) {
#pragma unroll
                for (int s = 0; s < kVLane; ++s) acc[s & 3] += __builtin_amdgcn_exp2f((x[s] - FM) * c); // -inf -> 0
            } else {
#pragma unroll
                for (int s = 0; s < kVLane; ++s)
                    acc[s & 3] += __builtin_isfinite(x[s]) ? __builtin_amdgcn_exp2f((x[s] - FM) * c) : 0.0f;
            }
            ls = (acc[0] + acc[1]) + (acc[2] + acc[3]);
        }
        const double l = wave_sum(double(ls));

        // ---- the chunk's top-K keys
        // hk = 0 past V: every count below looks at hk >= 1 only
        uint32_t hk[kVLane];
        if (full) {
#pragma unroll
            for (int s = 0; s < kVLane; ++s) hk[s] = vhi(x[s]);
        } else {
#pragma unroll
            for (int s = 0; s < kVLane; ++s) hk[s] = voff<VW>(lane, s) < nvalid ? vhi(x[s]) : 0u;
        }
        const int nk = nvalid < K ? nvalid : K;
        bool exact = SL * 64 > 128 || K > kFastK;
        uint32_t tk = 0;
        if (!exact) {
            float t[2] = {m1, m2};
            wave_sort_desc<float, 2>(t);
            const float tau = __shfl(t[(K - 1) & 1], (K - 1) >> 1, 64);
            int cnt = 0;
            tk = vhi(tau);
#pragma unroll
            for (int s = 0; s < kVLane; ++s) cnt += hk[s] >= tk ? 1 : 0;
            exact = !(tau > -__builtin_huge_valf()) || wave_sum_i(cnt) > 64 * SL;
        }
        // candidates: hk > th, or hk == th with chunk offset <= to
        uint32_t th = tk;
        int to = kVChunk;
        if (exact) {
            // th: the largest h with at least nk entries at or above it (>= 1,
            // since every valid entry has hk >= 1)
            th = 0;
            for (int b = 31; b >= 0; --b) {
                const uint32_t t = th | (1u << b);
                int c = 0;
#pragma unroll
                for (int s = 0; s < kVLane; ++s) c += hk[s] >= t ? 1 : 0;
                if (wave_sum_i(c) >= nk) th = t;
            }
            int gt = 0;
#pragma unroll
            for (int s = 0; s < kVLane; ++s) gt += hk[s] > th ? 1 : 0;
            const int need = nk - wave_sum_i(gt); // >= 1 entries with hk == th, lowest offsets first
            // to: the smallest offset with `need` tied entries at or below it
            int lo = -1, hi = kVChunk - 1;
            while (hi - lo > 1) {
                const int mid = (lo + hi) / 2;
                int c = 0;
#pragma unroll
                for (int s = 0; s < kVLane; ++s) {
                    c += (hk[s] == th && voff<VW>(lane, s) <= mid) ? 1 : 0;
                }
                if (wave_sum_i(c) >= need)
                    hi = mid;
                else
                    lo = mid;
            }
            to = hi;
        }

        // compact the candidates into this wave's LDS slots
        uint64_t *sl = slots[wv];
        int n = 0;
#pragma unroll
        for (int s = 0; s < kVLane; ++s) {
            const int o = voff<VW>(lane, s);
            const bool take = hk[s] > th || (hk[s] == th && o <= to);
            const uint64_t mask = __builtin_amdgcn_ballot_w64(take);
            if (mask) {
                if (take) sl[n + lane_rank(mask)] = vkey(hk[s], uint32_t(cb + o));
                n += __builtin_popcountll(mask);
            }
        }
        wave_lds_sync();
        uint64_t a[SL];
#pragma unroll
        for (int q = 0; q < SL; ++q) {
            const int i = SL * lane + q;
            a[q] = i < n ? sl[i] : 0;
        }
        wave_sort_desc<uint64_t, SL>(a);
        uint64_t *cr = cand + (row * nch + ch) * int64_t(K);
#pragma unroll
        for (int q = 0; q < SL; ++q) {
            const int i = SL * lane + q;
            if (i < K) cr[i] = i < nk ? a[q] : 0;
        }
        if (lane == 0) {
            VPart p;
            p.l = l;
            p.m = fin ? FM : 0.0f;
            p.bv = MX;
            p.bi = bi;
            p.fin = fin ? 1 : 0;
            p.nk = nk;
            p.pad = 0;
            part[row * nch + ch] = p;
        }
    }

    // ------------------------------------------------------------------ pass 2
    // K-th largest of the nonzero keys a wave holds R per lane (at least K
    // exist). Every search below builds its answer bit by bit from the top, a
    // fixed number of steps.
    template <int R>
    MG_DEV uint64_t wave_kth_key(const uint64_t (&r)[R], int K)
    {
        uint32_t hmin = 0xffffffffu, hmax = 0;
#pragma unroll
        for (int q = 0; q < R; ++q)
            if (r[q]) {
                const uint32_t h = uint32_t(r[q] >> 32);
                hmin = h < hmin ? h : hmin;
                hmax = h > hmax ? h : hmax;
            }
        hmin = wave_min_u32(hmin);
        hmax = wave_max_u32(hmax);
        // th: the largest h with count(hi >= h) >= K; it lies in [hmin, hmax],
        // whose members share the bits above the highest bit where they differ
        const uint32_t d = hmin ^ hmax;
        const int nb = d ? 32 - __builtin_clz(d) : 0;
        uint32_t th = nb == 32 ? 0u : (hmax & ~((1u << nb) - 1u));
        for (int b = nb - 1; b >= 0; --b) {
            const uint32_t t = th | (1u << b);
            int c = 0;
#pragma unroll
            for (int q = 0; q < R; ++q) c += (r[q] && uint32_t(r[q] >> 32) >= t) ? 1 : 0;
            if (wave_sum_i(c) >= K) th = t;
        }
        int gt = 0, eq = 0;
        uint64_t emin = ~uint64_t(0);
#pragma unroll
        for (int q = 0; q < R; ++q)
            if (r[q]) {
                const uint32_t h = uint32_t(r[q] >> 32);
                gt += h > th ? 1 : 0;
                if (h == th) {
                    ++eq;
                    emin = r[q] < emin ? r[q] : emin;
                }
            }
        const int need = K - wave_sum_i(gt); // 1 <= need <= keys with hi == th
        if (wave_sum_i(eq) == need) {
#pragma unroll
            for (int m = 32; m >= 1; m >>= 1) {
                const uint64_t o = __shfl_xor(emin, m, 64);
                emin = o < emin ? o : emin;
            }
            return emin;
        }
        // ties on the value: the need-th largest low word among them
        uint32_t lw = 0;
        for (int b = 31; b >= 0; --b) {
            const uint32_t t = lw | (1u << b);
            int c = 0;
#pragma unroll
            for (int q = 0; q < R; ++q) c += (r[q] && uint32_t(r[q] >> 32) == th && uint32_t(r[q]) >= t) ? 1 : 0;
            if (wave_sum_i(c) >= need) lw = t;
        }
        return (uint64_t(th) << 32) | lw;
    }

    // the same over every key of the row's full chunk lists, read from memory
    MG_DEV uint64_t wave_kth_key_mem(const uint64_t *cr, int64_t n, int K)
    {
        const int lane = threadIdx.x & 63;
        uint64_t k = 0;
        for (int b = 63; b >= 0; --b) {
            const uint64_t t = k | (uint64_t(1) << b);
            int c = 0;
            for (int64_t i = lane; i < n; i += 64) c += cr[i] >= t ? 1 : 0;
            if (wave_sum_i(c) >= K) k = t;
        }
        return k;
    }

    template <class SI, int SL>
    __global__ __launch_bounds__(64) void k_vocab_merge(const typename SI::raw *__restrict__ L, int64_t V, int K,
                                                        int nch, const VPart *__restrict__ part,
                                                        const uint64_t *__restrict__ cand, double *lse,
                                                        int64_t *amax, int64_t *top_idx, float *top_val)
    {
        __shared__ uint64_t sl[64 * SL];
        const int lane = threadIdx.x;
        const int64_t row = blockIdx.x;
        const VPart *pr = part + row * nch;
        const uint64_t *cr = cand + row * nch * int64_t(K);

        // lse and argmax: fold the chunk partials (lane-strided, then a
        // butterfly whose result every lane shares)
        float M = -__builtin_huge_valf(), bv = 0.0f;
        int bi = -1;
        bool any = false;
        for (int c = lane; c < nch; c += 64) {
            const VPart p = pr[c];
            if (p.fin) {
                M = p.m > M ? p.m : M;
                any = true;
            }
            if (beats(p.bv, p.bi, bv, bi)) {
                bv = p.bv;
                bi = p.bi;
            }
        }
        M = wave_max(M);
        any = __builtin_amdgcn_ballot_w64(any) != 0;
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
            const float ov = __shfl_xor(bv, m, 64);
            const int oi = __shfl_xor(bi, m, 64);
            if (beats(ov, oi, bv, bi)) {
                bv = ov;
                bi = oi;
            }
        }
        double S = 0.0;
        if (any)
            for (int c = lane; c < nch; c += 64) {
                const VPart p = pr[c];
                if (p.fin) S += p.l * mgm::exp(double(p.m) - double(M));
            }
        S = wave_sum(S);
        if (lane == 0) {
            if (lse) lse[row] = any ? double(M) + mgm::log(S) : -__builtin_huge_val();
            // the scan starts at index 0: a NaN there is never beaten
            const float x0 = float(SI::dec(L[row * V]));
            if (amax) amax[row] = (x0 != x0 || bi < 0) ? 0 : bi;
        }
        if (!top_idx && !top_val) return;

        // first try: the top kDepth keys of every chunk list
        uint64_t kap = 0;
        bool done = false;
        if (nch * kDepth <= 64 * kMergeRegs) {
            uint64_t r[kMergeRegs];
            int have = 0;
#pragma unroll
            for (int q = 0; q < kMergeRegs; ++q) {
                const int i = lane + 64 * q, c = i / kDepth, p = i % kDepth;
                r[q] = (c < nch && p < K) ? cr[int64_t(c) * K + p] : 0;
                have += r[q] ? 1 : 0;
            }
            if (wave_sum_i(have) >= K) {
                kap = wave_kth_key<kMergeRegs>(r, K);
                // every list's first key left out must fall below kap
                bool ok = true;
                if (K > kDepth)
                    for (int c = lane; c < nch; c += 64) ok &= cr[int64_t(c) * K + kDepth] < kap;
                done = __builtin_amdgcn_ballot_w64(!ok) == 0;
                if (done) {
                    int n = 0;
#pragma unroll
                    for (int q = 0; q < kMergeRegs; ++q) {
                        const bool take = r[q] >= kap && r[q] != 0;
                        const uint64_t mask = __builtin_amdgcn_ballot_w64(take);
                        if (mask) {
                            if (take) sl[n + lane_rank(mask)] = r[q];
                            n += __builtin_popcountll(mask);
                        }
                    }
                }
            }
        }
        if (!done) {
            const int64_t n_all = int64_t(nch) * K;
            kap = wave_kth_key_mem(cr, n_all, K);
            int n = 0;
            for (int64_t b = 0; b < n_all; b += 64) {
                const int64_t i = b + lane;
                const uint64_t k = i < n_all ? cr[i] : 0;
                const bool take = k >= kap && k != 0;
                const uint64_t mask = __builtin_amdgcn_ballot_w64(take);
                if (mask) {
                    if (take) sl[n + lane_rank(mask)] = k;
                    n += __builtin_popcountll(mask);
                }
            }
        }
        wave_lds_sync();
        // exactly K keys are >= kap (keys are unique)
        uint64_t a[SL];
#pragma unroll
        for (int q = 0; q < SL; ++q) {
            const int i = SL * lane + q;
            a[q] = i < K ? sl[i] : 0;
        }
        wave_sort_desc<uint64_t, SL>(a);
#pragma unroll
        for (int q = 0; q < SL; ++q) {
            const int i = SL * lane + q;
            if (i < K) {
                // a[q] is one of the K selected keys; an empty slot would be a
                // bug, reported as index -1 rather than read out of bounds
                const uint32_t j = vkey_index(a[q]);
                const bool ok = a[q] != 0 && int64_t(j) < V;
                if (top_idx) top_idx[row * K + i] = ok ? int64_t(j) : -1;
                if (top_val) top_val[row * K + i] = ok ? float(SI::dec(L[row * V + j])) : -__builtin_huge_valf();
            }
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
        const dim3 g1{unsigned((nch + 3) / 4), unsigned(rows), 1u};
        const dim3 g2{unsigned(rows), 1u, 1u};
        const bool small = K <= kFastK;
        auto go = [&](auto chunk, auto merge, const auto *x) {
            hipLaunchKernelGGL(chunk, g1, dim3(256), 0, c->stream, x, V, int(K), nch, part, cand);
            check_launch("k_vocab_chunk");
            hipLaunchKernelGGL(merge, g2, dim3(64), 0, c->stream, x, V, int(K), nch, part, cand, lse, amax, top_idx, top_val);
            check_launch("k_vocab_merge");
        };
        if (dt_in == F32) {
            const float *x = static_cast<const float *>(logits);
            const bool vec = V % 4 == 0 && aligned16(x);
            if (small && vec) go(k_vocab_chunk<SF32, 4, 2>, k_vocab_merge<SF32, 1>, x);
            else if (small) go(k_vocab_chunk<SF32, 1, 2>, k_vocab_merge<SF32, 1>, x);
            else if (vec) go(k_vocab_chunk<SF32, 4, 4>, k_vocab_merge<SF32, 4>, x);
            else go(k_vocab_chunk<SF32, 1, 4>, k_vocab_merge<SF32, 4>, x);
        } else if (dt_in == BF16) {
            const uint16_t *x = static_cast<const uint16_t *>(logits);
            const bool vec = V % 8 == 0 && aligned16(x);
            if (small && vec) go(k_vocab_chunk<SBf16, 8, 2>, k_vocab_merge<SBf16, 1>, x);
            else if (small) go(k_vocab_chunk<SBf16, 1, 2>, k_vocab_merge<SBf16, 1>, x);
            else if (vec) go(k_vocab_chunk<SBf16, 8, 4>, k_vocab_merge<SBf16, 4>, x);
            else go(k_vocab_chunk<SBf16, 1, 4>, k_vocab_merge<SBf16, 4>, x);
        } else {
            fail("vocab_reduce: input dtype must be f32 or bf16");
        }
    }
} // namespace mg
