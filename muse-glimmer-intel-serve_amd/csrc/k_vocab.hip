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
// in registers, no block barriers and no shuffles in the per-element work:
// counts are ballot popcounts, reductions are DPP. Per chunk: the finite max,
// the sum of exp(x - max) (f32 terms and lane sums, f64 across lanes), the
// first index of the max, a candidate list that contains the chunk's top-K,
// and the chunk's top-8 keys (the "block"). For K <= 64 the list is every
// element at or above a bound that cannot miss: each lane keeps its two
// largest values, and the K-th largest of those 128 values has at least K
// elements at or above it (about K + K/8 pass for random logits). When that
// bound is -inf or lets more than 128 through, and for every chunk when
// K > 64, the list is the exact top-K, selected by bit-by-bit bisection on the
// keys.
// Pass 2 (k_vocab_merge): one wave per row. lse and argmax fold the chunk
// partials (f64, FDLIBM exp/log). The row's K-th key is first selected from
// the blocks alone; that is exact when every chunk whose list runs past its
// block has its 8th key at or below the selected one (everything deeper is
// smaller still). Otherwise the selection runs over the full lists.
#include "mg_device.hpp"
#include "mg_internal.hpp"

#include <mutex>
#include <string>

namespace mg
{
    constexpr int kVLane = 32;           // keys per lane in pass 1
    constexpr int kVChunk = 64 * kVLane; // 2048 keys per wave-chunk
    constexpr int kMaxK = 256;
    constexpr int kFastK = 64;           // pass 1 bound-based selection up to this K
    constexpr int kBlk = 8;              // keys per chunk block
    constexpr int kMergeRegs = 16;       // pass 2: block keys per lane (1024 per row)

    struct VPart
    {
        double l;      // sum over the chunk's finite x of exp(x - m)
        uint64_t kd;   // the block's smallest key if keys outside the block can
                       // reach the row's top-K, else 0
        uint64_t top;  // the chunk's largest key: its argmax (first maximum, NaN lowest)
        float m;       // max of the chunk's finite x
        int32_t fin;   // 1 if the chunk holds a finite entry
        int32_t nlist; // keys in the chunk's candidate list
        int32_t pad;
    };

    // apply_output_tail (src/muse_glimmer.hpp:920-943) on one stored logit:
    // z*mult, z/cap, tanh, z*cap, each rounded to the logits' storage format —
    // the twin's values, bit for bit (mult 1 / cap 0 skip their steps).
    // Optionally written back in storage format. mult and cap are f32 values
    // (the twin's opmath, src/muse_glimmer.hpp:924-926) and z is stored, so
    // the product and quotient of two floats rounded once in f32 equal the
    // twin's f64 result rounded f64 -> f32 (products are exact in f64; for
    // the quotient, 53 >= 2*24 + 2 makes the double rounding innocuous).
    // tanh is tanh_stored (mg_device.hpp): a short f64 evaluation, accepted
    // when its error interval rounds to one stored value, else FDLIBM.
    struct VTail
    {
        float mult, cap;
        void *out;
    };
    template <class SI>
    MG_DEV float vtail(float x, const VTail &t)
    {
        float v = x;
        if (t.mult != 1.0f) v = SI::dec(SI::enc32(v * t.mult));
        if (t.cap != 0.0f) {
            v = SI::dec(SI::enc32(v / t.cap));
            v = tanh_stored<SI>(v);
            v = SI::dec(SI::enc32(v * t.cap));
        }
        return v;
    }

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

    // ------------------------------------------------------------------ pass 1
    // lane element s sits at chunk offset VW*lane + 64*VW*(s/VW) + s%VW: VW
    // consecutive elements per 16-byte load, a wave covering 1 KiB per load
    template <int VW>
    MG_DEV int voff(int lane, int s)
    {
        return VW * lane + 64 * VW * (s / VW) + (s % VW);
    }

    // Radix selection on 32-bit words held R per lane (0 = absent): the K-th
    // largest present word, and how many of the words equal to it belong to
    // the K largest (`take`). Bits shared by every present word are skipped;
    // the rest are resolved 8 at a time from the top with a 256-bin LDS
    // histogram (`hist`, this wave's own) and a DPP prefix sum over the lanes'
    // bins, so a 32-bit word costs at most 4 passes.
    template <int R>
    MG_DEV uint32_t wave_select(const uint32_t (&h)[R], int K, uint32_t *hist, int &take)
    {
        const int lane = threadIdx.x & 63;
        uint32_t hmin = 0xffffffffu, hmax = 0;
#pragma unroll
        for (int q = 0; q < R; ++q)
            if (h[q]) {
                hmin = h[q] < hmin ? h[q] : hmin;
                hmax = h[q] > hmax ? h[q] : hmax;
            }
        hmin = dpp_min_u32(hmin);
        hmax = dpp_max_u32(hmax);
        const uint32_t d = hmin ^ hmax;
        int nb = d ? 32 - __builtin_clz(d) : 0; // open bits: nb-1 .. 0
        uint32_t prefix = nb == 32 ? 0u : (hmax & ~((1u << nb) - 1u));
        int need = K;
        while (nb > 0) {
            const int w = nb < 8 ? nb : 8, sh = nb - w;
            const uint32_t fixed = nb == 32 ? 0u : ~((1u << nb) - 1u);
            wave_lds_sync();
            *reinterpret_cast<Vec<uint32_t, 4> *>(hist + 4 * lane) = Vec<uint32_t, 4>{{0u, 0u, 0u, 0u}};
            wave_lds_sync();
#pragma unroll
            for (int q = 0; q < R; ++q)
                if (h[q] && (h[q] & fixed) == prefix) atomicAdd(hist + ((h[q] >> sh) & ((1u << w) - 1u)), 1u);
            wave_lds_sync();
            const Vec<uint32_t, 4> c = *reinterpret_cast<const Vec<uint32_t, 4> *>(hist + 4 * lane);
            const int sl = int(c.v[0] + c.v[1] + c.v[2] + c.v[3]);
            const int incl = wave_prefix_sum(sl);
            const int above_lane = __builtin_amdgcn_readlane(incl, 63) - incl; // in higher bins
            const bool mine = above_lane < need && need <= above_lane + sl;
            int dg = 0, above = 0;
            if (mine) {
                int acc = above_lane;
                for (int e = 3; e >= 0; --e) {
                    if (acc + int(c.v[e]) >= need) {
                        dg = 4 * lane + e;
                        above = acc;
                        break;
                    }
                    acc += int(c.v[e]);
                }
            }
            const int src = int(__builtin_ctzll(__builtin_amdgcn_ballot_w64(mine)));
            dg = __builtin_amdgcn_readlane(dg, src);
            above = __builtin_amdgcn_readlane(above, src);
            prefix |= uint32_t(dg) << sh;
            need -= above;
            nb = sh;
        }
        take = need;
        return prefix;
    }

    // K-th largest of the nonzero keys a wave holds R per lane (at least K of
    // them): the high word by radix selection, then, when more keys share it
    // than remain to take, the low word by bit-by-bit bisection among them.
    template <int R>
    MG_DEV uint64_t wave_kth(const uint64_t (&r)[R], int K, uint32_t *hist)
    {
        uint32_t h[R];
#pragma unroll
        for (int q = 0; q < R; ++q) h[q] = uint32_t(r[q] >> 32); // keys have high word >= 1
        int need = 0;
        const uint32_t th = wave_select<R>(h, K, hist, need);
        int eq = 0;
        uint32_t lmin = 0xffffffffu;
#pragma unroll
        for (int q = 0; q < R; ++q) {
            const bool e = h[q] == th;
            eq += wave_count(e);
            lmin = (e && uint32_t(r[q]) < lmin) ? uint32_t(r[q]) : lmin;
        }
        if (eq == need) return (uint64_t(th) << 32) | dpp_min_u32(lmin);
        uint32_t lw = 0;
        for (int b = 31; b >= 0; --b) {
            const uint32_t t = lw | (1u << b);
            int c = 0;
#pragma unroll
            for (int q = 0; q < R; ++q) c += wave_count(h[q] == th && uint32_t(r[q]) >= t);
            if (c >= need) lw = t;
        }
        return (uint64_t(th) << 32) | lw;
    }

    template <class SI, int VW, int SL, bool TAIL>
    __global__ __launch_bounds__(256) void k_vocab_chunk(const typename SI::raw *__restrict__ L, int64_t V, int K,
                                                         int nch, VPart *__restrict__ part,
                                                         uint64_t *__restrict__ blk, uint64_t *__restrict__ lst,
                                                         VTail tail)
    {
        using raw = typename SI::raw;
        constexpr int CAP = 64 * SL; // list capacity
        __shared__ uint32_t sbits[4][CAP];
        __shared__ uint32_t soff[4][CAP];
        __shared__ __align__(16) uint32_t shist[4][256];
        const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
        const int ch = int(blockIdx.x) * 4 + wv;
        const int64_t row = blockIdx.y;
        if (ch >= nch) return; // the whole wave leaves; nothing below syncs the block
        const int64_t cb = int64_t(ch) * kVChunk;
        const int nvalid = int(V - cb < kVChunk ? V - cb : kVChunk);
        const bool full = nvalid == kVChunk;
        const raw *xr = L + row * V + cb;

        // the chunk as f32 bit patterns; the exact selection overwrites them
        // with the keys' high words
        uint32_t xb[kVLane];
        auto x = [&](int s) { return __builtin_bit_cast(float, xb[s]); };
        bool loaded = false;
        if constexpr (VW > 1) {
            if (full) {
#pragma unroll
                for (int i = 0; i < kVLane / VW; ++i) {
                    const Vec<raw, VW> v = ld16_stream<raw, VW>(xr + VW * lane + 64 * VW * i);
#pragma unroll
                    for (int e = 0; e < VW; ++e) xb[VW * i + e] = __builtin_bit_cast(uint32_t, float(SI::dec(v.v[e])));
                }
                loaded = true;
            }
        }
        if (!loaded) {
            // tail chunk (or unaligned rows): -inf placeholders past V never
            // reach a sum, a max or the candidates, and are kept out of the
            // argmax and the exact selection by offset
#pragma unroll
            for (int s = 0; s < kVLane; ++s) {
                const int o = voff<VW>(lane, s);
                xb[s] = __builtin_bit_cast(uint32_t, o < nvalid ? float(SI::dec(xr[o])) : -__builtin_huge_valf());
            }
        }

        if constexpr (TAIL) {
#pragma unroll
            for (int s = 0; s < kVLane; ++s)
                if (full || voff<VW>(lane, s) < nvalid) xb[s] = __builtin_bit_cast(uint32_t, vtail<SI>(x(s), tail));
            if (tail.out) {
                raw *orow = static_cast<raw *>(tail.out) + row * V + cb;
                bool stored = false;
                if constexpr (VW > 1) {
                    if (full) {
#pragma unroll
                        for (int i = 0; i < kVLane / VW; ++i) {
                            Vec<raw, VW> w;
#pragma unroll
                            for (int e = 0; e < VW; ++e) w.v[e] = SI::enc32(x(VW * i + e));
                            st16_stream<raw, VW>(orow + VW * lane + 64 * VW * i, w);
                        }
                        stored = true;
                    }
                }
                if (!stored) {
#pragma unroll
                    for (int s = 0; s < kVLane; ++s) {
                        const int o = voff<VW>(lane, s);
                        if (o < nvalid) orow[o] = SI::enc32(x(s));
                    }
                }
            }
        }

        // lane maximum and second maximum (two distinct elements)
        float m1 = -__builtin_huge_valf(), m2 = -__builtin_huge_valf();
#pragma unroll
        for (int s = 0; s < kVLane; ++s) {
            m2 = __builtin_fmaxf(m2, __builtin_fminf(m1, x(s)));
            m1 = __builtin_fmaxf(m1, x(s));
        }
        const float MX = dpp_max(m1); // max over the non-NaN entries

        // lse partial, first assuming every entry finite or -inf
        constexpr float c = 1.44269504088896341f;
        float FM = MX;
        double l = 0.0;
        bool special = !(MX < __builtin_huge_valf()) || !(MX > -__builtin_huge_valf());
        if (!special) {
            // 2^(x*c - rnd(MX*c)) with one fma; the rounding of MX*c, shared by
            // every term, is divided out exactly below
            const float FMc = MX * c;
            float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < kVLane; ++s) acc[s & 3] += __builtin_amdgcn_exp2f(__builtin_fmaf(x(s), c, -FMc));
            const double S = dpp_sum(double((acc[0] + acc[1]) + (acc[2] + acc[3])));
            const double dl = (double(FMc) - double(MX) * double(c)) * 0.69314718055994531;
            l = S * (1.0 + dl + 0.5 * dl * dl);
            special = S != S; // a NaN logit
        }
        if (special) {
            // NaN or +inf present, or no finite entry: the finite max, the sum
            // over finite entries, and m1/m2 with NaN taken as -inf (fminf
            // would otherwise pass NaN's partner through as a second element)
            float fm = -__builtin_huge_valf();
#pragma unroll
            for (int s = 0; s < kVLane; ++s)
                if (__builtin_isfinite(x(s))) fm = __builtin_fmaxf(fm, x(s));
            FM = dpp_max(fm);
            float acc = 0.0f;
            if (FM > -__builtin_huge_valf())
#pragma unroll
                for (int s = 0; s < kVLane; ++s)
                    acc += __builtin_isfinite(x(s)) ? __builtin_amdgcn_exp2f((x(s) - FM) * c) : 0.0f;
            l = dpp_sum(double(acc));
            m1 = m2 = -__builtin_huge_valf();
#pragma unroll
            for (int s = 0; s < kVLane; ++s) {
                const float v = x(s) == x(s) ? x(s) : -__builtin_huge_valf();
                m2 = __builtin_fmaxf(m2, __builtin_fminf(m1, v));
                m1 = __builtin_fmaxf(m1, v);
            }
        }
        const bool fin = FM > -__builtin_huge_valf();

        // ---- candidates
        const int nk = nvalid < K ? nvalid : K;
        bool exact = SL > 2;
        float tau = -__builtin_huge_valf();
        if (!exact) {
            // tau: the K-th largest of the 128 lane top-2 values
            const uint32_t k2[2] = {f32_key(m1 + 0.0f), f32_key(m2 + 0.0f)}; // >= key(-inf) > 0
            int unused = 0;
            tau = key_f32(wave_select<2>(k2, K, shist[wv], unused));
            exact = !(tau > -__builtin_huge_valf());
        }
        // exact: candidates are hk > th, or hk == th at offsets <= to
        uint32_t th = 0;
        int to = kVChunk;
        auto select_exact = [&]() {
            // the keys' high words replace the values (0 past V)
#pragma unroll
            for (int s = 0; s < kVLane; ++s) xb[s] = (full || voff<VW>(lane, s) < nvalid) ? vhi(x(s)) : 0u;
            int need = 0; // entries with hk == th to take, lowest offsets first
            th = wave_select<kVLane>(xb, nk, shist[wv], need);
            int lo = -1, hi = kVChunk - 1;
            while (hi - lo > 1) {
                const int mid = (lo + hi) / 2;
                int cnt = 0;
#pragma unroll
                for (int s = 0; s < kVLane; ++s) cnt += wave_count(xb[s] == th && voff<VW>(lane, s) <= mid);
                if (cnt >= need)
                    hi = mid;
                else
                    lo = mid;
            }
            to = hi;
        };
        if (exact) select_exact();

        // compact (bits, offset) of the candidates into this wave's LDS slots;
        // more than CAP of them (possible only through ties at tau) sends
        // the chunk to the exact selection
        uint32_t *sb = sbits[wv], *so = soff[wv];
        int n = 0;
        for (int pass = 0; pass < 2; ++pass) {
            n = 0;
#pragma unroll
            for (int s = 0; s < kVLane; ++s) {
                const int o = voff<VW>(lane, s);
                const uint32_t bits = xb[s];
                const bool take = exact ? (bits > th || (bits == th && o <= to)) : x(s) >= tau;
                const uint64_t mk = __builtin_amdgcn_ballot_w64(take);
                if (mk) {
                    const int p = n + lane_rank(mk);
                    if (take && p < CAP) {
                        sb[p] = bits;
                        so[p] = uint32_t(o);
                    }
                    n += __builtin_popcountll(mk);
                }
            }
            if (n <= CAP) break;
            // exact selection (the keys replace the values), then compact again
            exact = true;
            select_exact();
        }
        wave_lds_sync();
        uint64_t a[SL];
#pragma unroll
        for (int q = 0; q < SL; ++q) {
            const int i = SL * lane + q;
            a[q] = 0;
            if (i < n) {
                const uint32_t bits = sb[i];
                a[q] = vkey(exact ? bits : vhi(__builtin_bit_cast(float, bits)), uint32_t(cb + so[i]));
            }
        }
        const int64_t cid = row * nch + ch;
        uint64_t *lr = lst + cid * CAP;
#pragma unroll
        for (int q = 0; q < SL; ++q)
            if (SL * lane + q < n) lr[SL * lane + q] = a[q];

        // the block: the list's (= the chunk's) top D keys, D = min(8, K),
        // taken largest first. Keys are unique, so the wave maximum of the high
        // words, then of the low words among the slots holding that high word,
        // is the largest remaining key; it is cleared and lane i keeps the i-th.
        // Slots past the list's end hold 0 and make the block's tail 0.
        const int D = K < kBlk ? K : kBlk;
        uint64_t *br = blk + cid * kBlk;
        uint64_t kd = 0; // the D-th key when the list is longer than the block
        uint64_t top = 0; // the first key taken, the list's (= the chunk's) largest: its argmax
        {
            uint64_t r[SL];
#pragma unroll
            for (int q = 0; q < SL; ++q) r[q] = a[q];
            uint64_t mine = 0;
            for (int i = 0; i < D; ++i) {
                uint32_t hm = 0;
#pragma unroll
                for (int q = 0; q < SL; ++q) hm = uint32_t(r[q] >> 32) > hm ? uint32_t(r[q] >> 32) : hm;
                hm = dpp_max_u32(hm);
                uint32_t lm = 0;
#pragma unroll
                for (int q = 0; q < SL; ++q)
                    lm = (uint32_t(r[q] >> 32) == hm && uint32_t(r[q]) > lm) ? uint32_t(r[q]) : lm;
                lm = dpp_max_u32(lm);
                const uint64_t mk = (uint64_t(hm) << 32) | lm;
#pragma unroll
                for (int q = 0; q < SL; ++q) r[q] = r[q] == mk ? 0 : r[q];
                mine = lane == i ? mk : mine;
                top = i == 0 ? mk : top;
                kd = mk;
            }
            if (lane < kBlk) br[lane] = mine;
        }
        if (n <= D) kd = 0;
        if (lane == 0) {
            VPart p;
            p.l = l;
            p.kd = (D < K && n > D) ? kd : 0;
            p.m = fin ? FM : 0.0f;
            p.top = top;
            p.fin = fin ? 1 : 0;
            p.nlist = n;
            p.pad = 0;
            part[cid] = p;
        }
    }

    // ------------------------------------------------------------------ pass 2
    // K-th largest key over every chunk's candidate list, read from memory
    MG_DEV uint64_t lists_kth(const VPart *pr, const uint64_t *ls, int nch, int cap, int K)
    {
        const int lane = threadIdx.x & 63;
        auto count = [&](auto pred) {
            int c = 0;
            for (int ch = 0; ch < nch; ++ch) {
                const int nl = pr[ch].nlist < cap ? pr[ch].nlist : cap;
                for (int p0 = 0; p0 < nl; p0 += 64) {
                    const int p = p0 + lane;
                    const uint64_t k = p < nl ? ls[int64_t(ch) * cap + p] : 0;
                    c += wave_count(k != 0 && pred(k));
                }
            }
            return c;
        };
        uint32_t th = 0;
        for (int b = 31; b >= 0; --b) {
            const uint32_t t = th | (1u << b);
            if (count([&](uint64_t k) { return uint32_t(k >> 32) >= t; }) >= K) th = t;
        }
        const int need = K - count([&](uint64_t k) { return uint32_t(k >> 32) > th; });
        uint32_t lw = 0;
        for (int b = 31; b >= 0; --b) {
            const uint32_t t = lw | (1u << b);
            if (count([&](uint64_t k) { return uint32_t(k >> 32) == th && uint32_t(k) >= t; }) >= need) lw = t;
        }
        return (uint64_t(th) << 32) | lw;
    }

    template <class SI, int SL, bool TAIL>
    __global__ __launch_bounds__(64) void k_vocab_merge(const typename SI::raw *__restrict__ L, int64_t V, int K,
                                                        int nch, int cap, const VPart *__restrict__ part,
                                                        const uint64_t *__restrict__ blk,
                                                        const uint64_t *__restrict__ lst, double *lse,
                                                        int64_t *amax, int64_t *top_idx, float *top_val, VTail tail)
    {
        __shared__ uint64_t sel[64 * SL];
        __shared__ __align__(16) uint32_t hist[256];
        const int lane = threadIdx.x;
        const int64_t row = blockIdx.x;
        const VPart *pr = part + row * nch;
        const uint64_t *bk = blk + row * nch * int64_t(kBlk);
        const uint64_t *ls = lst + row * nch * int64_t(cap);
        float x0 = float(SI::dec(L[row * V]));
        if constexpr (TAIL) x0 = vtail<SI>(x0, tail);
        const bool want_top = top_idx || top_val;
        const int D = K < kBlk ? K : kBlk;
        const bool regs = want_top && nch * D <= 64 * kMergeRegs;

        // the lane's chunk partials (up to two: rows of up to 128 chunks) and
        // the blocks' keys, all requested before any is used, so one round
        // trip serves the fold, the blocks and the block check
        constexpr int PPL = 2;
        const bool pregs = nch <= 64 * PPL;
        VPart pv[PPL];
#pragma unroll
        for (int k = 0; k < PPL; ++k) {
            const int c = lane + 64 * k;
            if (pregs && c < nch) {
                pv[k] = pr[c];
            } else {
                pv[k].l = 0.0;
                pv[k].kd = pv[k].top = 0;
                pv[k].m = -__builtin_huge_valf();
                pv[k].fin = pv[k].nlist = pv[k].pad = 0;
            }
        }
        uint64_t r[kMergeRegs];
#pragma unroll
        for (int q = 0; q < kMergeRegs; ++q) {
            const int i = lane + 64 * q;
            const int c = D == kBlk ? i / kBlk : i / D, p = D == kBlk ? i % kBlk : i - c * D;
            r[q] = regs && c < nch ? bk[int64_t(c) * kBlk + p] : 0;
        }

        // lse and argmax: fold the chunk partials; the largest chunk key is
        // the row's first maximum
        float M = -__builtin_huge_valf();
        uint64_t ak = 0;
        bool any = false;
        auto fold_max = [&](const VPart &p) {
            if (p.fin) {
                M = p.m > M ? p.m : M;
                any = true;
            }
            ak = p.top > ak ? p.top : ak;
        };
        if (pregs) {
#pragma unroll
            for (int k = 0; k < PPL; ++k) fold_max(pv[k]); // absent ones: fin 0, top 0
        } else {
            for (int c = lane; c < nch; c += 64) fold_max(pr[c]);
        }
        M = dpp_max(M);
        ak = dpp_reduce(ak, uint64_t(0), [](uint64_t u, uint64_t v) { return u > v ? u : v; });
        any = __builtin_amdgcn_ballot_w64(any) != 0;
        // sum of l_c * e^(m_c - M): the f32 difference and hardware exp2 keep
        // each term within a few ulp of f32, far inside the lse tolerance
        double S = 0.0;
        auto fold_sum = [&](const VPart &p) {
            if (p.fin) S += p.l * double(__builtin_amdgcn_exp2f((p.m - M) * 1.44269504088896341f));
        };
        if (any) {
            if (pregs) {
#pragma unroll
                for (int k = 0; k < PPL; ++k) fold_sum(pv[k]);
            } else {
                for (int c = lane; c < nch; c += 64) fold_sum(pr[c]);
            }
        }
        S = dpp_sum(S);
        if (lane == 0) {
            if (lse) lse[row] = any ? double(M) + mgm::log(S) : -__builtin_huge_val();
            // the scan starts at index 0: a NaN there is never beaten
            if (amax) amax[row] = (x0 != x0 || ak == 0) ? 0 : int64_t(vkey_index(ak));
        }
        if (!want_top) return;

        // first try: the blocks alone
        bool done = false;
        if (regs) {
            int have = 0;
#pragma unroll
            for (int q = 0; q < kMergeRegs; ++q) have += wave_count(r[q] != 0);
            if (have >= K) {
                const uint64_t kap = wave_kth<kMergeRegs>(r, K, hist);
                bool bad = false;
                if (pregs) {
#pragma unroll
                    for (int k = 0; k < PPL; ++k) bad |= pv[k].kd != 0 && pv[k].kd > kap;
                } else {
                    for (int c = lane; c < nch; c += 64) {
                        const uint64_t kd = pr[c].kd;
                        bad |= kd != 0 && kd > kap;
                    }
                }
                done = __builtin_amdgcn_ballot_w64(bad) == 0;
                if (done) {
                    int n = 0;
#pragma unroll
                    for (int q = 0; q < kMergeRegs; ++q) {
                        const bool take = r[q] != 0 && r[q] >= kap;
                        const uint64_t mk = __builtin_amdgcn_ballot_w64(take);
                        if (mk) {
                            if (take && n + lane_rank(mk) < 64 * SL) sel[n + lane_rank(mk)] = r[q];
                            n += __builtin_popcountll(mk);
                        }
                    }
                }
            }
        }
        if (!done) {
            const uint64_t kap = lists_kth(pr, ls, nch, cap, K);
            int n = 0;
            for (int c = 0; c < nch; ++c) {
                const int nl = pr[c].nlist < cap ? pr[c].nlist : cap;
                for (int p0 = 0; p0 < nl; p0 += 64) {
                    const int p = p0 + lane;
                    const uint64_t k = p < nl ? ls[int64_t(c) * cap + p] : 0;
                    const bool take = k != 0 && k >= kap;
                    const uint64_t mk = __builtin_amdgcn_ballot_w64(take);
                    if (mk) {
                        if (take && n + lane_rank(mk) < 64 * SL) sel[n + lane_rank(mk)] = k;
                        n += __builtin_popcountll(mk);
                    }
                }
            }
        }
        wave_lds_sync();
        // exactly K keys were selected (keys are unique)
        uint64_t a[SL];
#pragma unroll
        for (int q = 0; q < SL; ++q) {
            const int i = SL * lane + q;
            a[q] = i < K ? sel[i] : 0;
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
                float tv = -__builtin_huge_valf();
                const uint32_t hk = uint32_t(a[q] >> 32);
                if (ok && hk != 1u && hk != f32_key(0.0f)) {
                    // the key's high word is the (transformed) value itself
                    tv = key_f32(hk);
                } else if (ok) {
                    // NaN and +-0 share a key per class: read the value back
                    tv = float(SI::dec(L[row * V + j]));
                    if constexpr (TAIL) tv = vtail<SI>(tv, tail);
                }
                if (top_val) top_val[row * K + i] = tv;
            }
        }
    }

    // The pass on `stream` with its partials in `work` (work_bytes long);
    // `room` names where they live for the error raised when they do not fit.
    static void vocab_pass(hipStream_t stream, void *work, int64_t work_bytes, const char *room, const void *logits,
                           int64_t rows, int64_t V, int dt_in, int64_t K, double *lse, int64_t *amax,
                           int64_t *top_idx, float *top_val, bool tail_on, double mult, double cap, void *logits_out)
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
        const bool small = K <= kFastK;
        const int lcap = small ? 128 : 256; // list capacity per chunk
        const int64_t nc = rows * nch;
        const int64_t need_bytes = nc * int64_t(sizeof(VPart) + sizeof(uint64_t) * (kBlk + lcap));
        need(need_bytes <= work_bytes, "vocab_reduce: the partials of " + std::to_string(rows) + " rows x " +
                                           std::to_string(nch) + " chunks need " + std::to_string(need_bytes) +
                                           " bytes, more than " + room + " (" + std::to_string(work_bytes) + ")");
        VPart *part = static_cast<VPart *>(work);
        uint64_t *blk = reinterpret_cast<uint64_t *>(part + nc);
        uint64_t *lst = blk + nc * kBlk;
        const dim3 g1{unsigned((nch + 3) / 4), unsigned(rows), 1u};
        const dim3 g2{unsigned(rows), 1u, 1u};
        // python-float scalars are f32 opmath values outside f64 (src/muse_glimmer.hpp:924-926)
        const VTail tail{float(mult), float(cap), logits_out};
        auto go = [&](auto chunk, auto merge, const auto *x) {
            hipLaunchKernelGGL(chunk, g1, dim3(256), 0, stream, x, V, int(K), nch, part, blk, lst, tail);
            check_launch("k_vocab_chunk");
            hipLaunchKernelGGL(merge, g2, dim3(64), 0, stream, x, V, int(K), nch, lcap, part, blk, lst, lse, amax,
                               top_idx, top_val, tail);
            check_launch("k_vocab_merge");
        };
        auto pick = [&](auto si, auto vw, const auto *x) {
            using SI = decltype(si);
            constexpr int VW = decltype(vw)::value;
            if (small && tail_on) go(k_vocab_chunk<SI, VW, 2, true>, k_vocab_merge<SI, 1, true>, x);
            else if (small) go(k_vocab_chunk<SI, VW, 2, false>, k_vocab_merge<SI, 1, false>, x);
            else if (tail_on) go(k_vocab_chunk<SI, VW, 4, true>, k_vocab_merge<SI, 4, true>, x);
            else go(k_vocab_chunk<SI, VW, 4, false>, k_vocab_merge<SI, 4, false>, x);
        };
        if (dt_in == F32) {
            const float *x = static_cast<const float *>(logits);
            if (V % 4 == 0 && aligned16(x) && (!logits_out || aligned16(logits_out)))
                pick(SF32{}, std::integral_constant<int, 4>{}, x);
            else
                pick(SF32{}, std::integral_constant<int, 1>{}, x);
        } else if (dt_in == BF16) {
            const uint16_t *x = static_cast<const uint16_t *>(logits);
            if (V % 8 == 0 && aligned16(x) && (!logits_out || aligned16(logits_out)))
                pick(SBf16{}, std::integral_constant<int, 8>{}, x);
            else
                pick(SBf16{}, std::integral_constant<int, 1>{}, x);
        } else {
            fail("vocab_reduce: input dtype must be f32 or bf16");
        }
    }

    void launch_vocab(mg_ctx *c, const void *logits, int64_t rows, int64_t V, int dt_in, int64_t K,
                      double *lse, int64_t *amax, int64_t *top_idx, float *top_val, bool tail_on, double mult,
                      double cap, void *logits_out)
    {
        vocab_pass(c->stream, c->work, c->work_bytes, "the context workspace (raise workspace_bytes at mg_open)",
                   logits, rows, V, dt_in, K, lse, amax, top_idx, top_val, tail_on, mult, cap, logits_out);
    }

    // ------------------------------------------------- allocation-free variant
    // The same pass with its partials in `scratch`, a fixed array in device
    // memory (one copy per GPU, held until the process ends) instead of a
    // context's workspace: nothing is allocated, on the first call or later.
    // The kernels write every partial before they read it, so the array needs
    // no clearing between calls; calls that overlap on one GPU (two streams)
    // share it and race.
    static __device__ __align__(256) unsigned char scratch[kVocabScratchBytes];

    // scratch's device address on the current device, looked up once per device
    // (hipGetSymbolAddress allocates nothing); host code passes this address,
    // never the array's name, which on the host is a stand-in.
    static void *scratch_address()
    {
        constexpr int kMaxDevices = 64;
        static std::mutex mu;
        static void *addr[kMaxDevices] = {};
        int dev = -1;
        check(hipGetDevice(&dev), "vocab_reduce_noalloc: hipGetDevice");
        need(dev >= 0 && dev < kMaxDevices, "vocab_reduce_noalloc: device index out of range");
        std::lock_guard<std::mutex> lock(mu);
        if (!addr[dev]) {
            void *p = nullptr;
            check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "vocab_reduce_noalloc: hipGetSymbolAddress(scratch)");
            need(p != nullptr, "vocab_reduce_noalloc: no device address for the scratch array");
            addr[dev] = p;
        }
        return addr[dev];
    }

    void launch_vocab_noalloc(hipStream_t stream, const void *logits, int64_t rows, int64_t V, int dt_in, int64_t K,
                              double *lse, int64_t *amax, int64_t *top_idx, float *top_val)
    {
        vocab_pass(stream, scratch_address(), kVocabScratchBytes, "the fixed scratch array", logits, rows, V, dt_in,
                   K, lse, amax, top_idx, top_val, false, 1.0, 0.0, nullptr);
    }
} // namespace mg
