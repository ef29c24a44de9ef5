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
// the f32 value (NaN -> 1, -0 -> +0) above the complement of the index. Keys
// are unique and "the K largest keys" is exactly the order above, so every
// selection below is deterministic however the work is split.
//
// Pass 1 (k_vocab_chunk): one wave per 4096-key chunk, 64 keys per lane held
// in registers (a row of 201088 keys is 50 chunks; 64 rows fill the chip's
// wave slots once). Per chunk: the finite max, the sum of exp(x - max) (f32
// terms, f64 across lanes), and the chunk's top D = min(16, K) keys in order
// (the "block"), whose first is the chunk's argmax. The block costs little:
// t, the D-th largest of the 64 lane maxima, has at least D keys at or above
// it, so the keys >= t (about D + 1 for random logits) hold the block; they
// are compacted through ballots and ranked by a count over the others. Chunks
// where that set is empty of meaning (more than 64 keys >= t, or NaN needed
// to fill the block) select their block exactly by radix selection.
// Pass 2 (k_vocab_merge): one wave per row. lse and argmax fold the chunk
// partials (f64, FDLIBM exp/log). The row's K-th key kap is selected from the
// blocks; it is the answer when no chunk's D-th key lies above kap (every key
// outside a block is below that chunk's D-th key). Otherwise the chunks that
// fail the check are re-read and their exact top-K computed, and the
// selection runs again over those lists and the other chunks' blocks: exact
// for any input, slower only where one chunk holds more than D of the row's
// top K.
#include "mg_device.hpp"
#include "mg_softcap_fast.hpp"
#include "mg_wave_sort.hpp"
#include "mg_internal.hpp"

#include <mutex>
#include <string>

namespace mg
{
    constexpr int kVLane = 64;           // keys per lane in pass 1
    constexpr int kVChunk = 64 * kVLane; // 4096 keys per wave-chunk
    constexpr int kMaxK = 256;
    constexpr int kBlk = 16;             // keys per chunk block
    constexpr int kCand = 64;            // candidates a chunk ranks (one per lane)
    constexpr int kMergeRegs = 16;       // pass 2: block keys per lane (the blocks of 64 chunks)
    constexpr int kUnionCap = 4096;      // pass 2 fallback: keys staged in LDS

    struct VPart
    {
        double l;      // sum over the chunk's finite x of exp(x - m)
        uint64_t kd;   // the block's last key when the chunk holds more keys than
                       // its block (every other key is below it), else 0
        uint64_t top;  // the chunk's largest key: its argmax (first maximum, NaN lowest)
        float m;       // max of the chunk's finite x
        int32_t fin;   // 1 if the chunk holds a finite entry
        int32_t pad0, pad1;
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
        float rcap; // RN(1 / cap) for 1 <= |cap| <= 2^20, else 0 (the IEEE quotient)
    };
    template <class SI>
    MG_DEV float vtail(float x, const VTail &t)
    {
        float v = x;
        if (t.mult != 1.0f) v = SI::dec(SI::enc32(v * t.mult));
        if (t.cap != 0.0f) {
            // v / cap correctly rounded: Markstein's correction of v * rcap
            // (mg_softcap_fast.hpp) while no step can under- or overflow
            // (the IEEE quotient only in waves that have a lane outside)
            float q = mgm::softcap_quotient(v, t.cap, t.rcap);
            const float av = __builtin_fabsf(v);
            const bool fast = t.rcap != 0.0f && av > 0x1p-100f && av < 0x1p100f;
            if (__builtin_amdgcn_ballot_w64(!fast) != 0 && !fast) {
                float c = t.cap;
                __asm__ volatile("" : "+v"(c)); // keeps the division inside the branch
                q = v / c;
            }
            v = SI::dec(SI::enc32(q));
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

    // ------------------------------------------------------------------ pass 1

    // The tail on VW stored values side by side: the common path (|z / cap| < 1
    // with a certain rounding) branch-free, a wave with any value outside it
    // through vtail for those values. z: decoded inputs in, stored results out.
    template <class SI, int VW>
    MG_DEV void tail_vec(float (&z)[VW], const VTail &t, const double *tab)
    {
        if (t.cap == 0.0f) {
#pragma unroll
            for (int e = 0; e < VW; ++e) z[e] = vtail<SI>(z[e], t);
            return;
        }
        float r[VW];
        uint32_t slow = 0;
#pragma unroll
        for (int e = 0; e < VW; ++e) {
            float w = z[e];
            if (t.mult != 1.0f) w = SI::dec(SI::enc32(w * t.mult));
            const float az = __builtin_fabsf(w);
            const float q = SI::dec(SI::enc32(mgm::softcap_quotient(w, t.cap, t.rcap)));
            const double a = __builtin_fabs(double(q));
            const double ac = __builtin_fmin(a, 0x1.fffffffffffffp-1);
            const double th = mgm::tanh_table_abs(ac, tab);
            double tl, tu;
            mgm::tanh_interval(th, tl, tu);
            const auto lo = SI::enc64(tl), hi = SI::enc64(tu);
            const bool ok = t.rcap != 0.0f && az > 0x1p-100f && az < 0x1p100f && a < 1.0 && lo == hi;
            r[e] = SI::dec(SI::enc32(__builtin_copysignf(SI::dec(lo), q) * t.cap));
            slow |= ok ? 0u : 1u << e;
        }
        if (__builtin_amdgcn_ballot_w64(slow != 0) != 0) {
#pragma unroll
            for (int e = 0; e < VW; ++e)
                if ((slow >> e) & 1u) r[e] = vtail<SI>(z[e], t);
        }
#pragma unroll
        for (int e = 0; e < VW; ++e) z[e] = r[e];
    }

    // A chunk's logits as f32 bit patterns (past V: -inf, which no sum, max or
    // candidate takes), tail-transformed and optionally written back
    template <class SI, int VW, bool TAIL>
    MG_DEV void chunk_load(const typename SI::raw *__restrict__ xr, int nvalid, const VTail &tail,
                           typename SI::raw *orow, uint32_t (&xb)[kVLane], const double *tab)
    {
        using raw = typename SI::raw;
        const int lane = threadIdx.x & 63;
        const bool full = nvalid == kVChunk;
        bool loaded = false;
        if constexpr (VW > 1) {
            if (full) {
#pragma unroll
                for (int i = 0; i < kVLane / VW; i += 2) {
                    float z[2 * VW];
#pragma unroll
                    for (int g = 0; g < 2; ++g) {
                        const Vec<raw, VW> v = ld16_stream<raw, VW>(xr + VW * lane + 64 * VW * (i + g));
#pragma unroll
                        for (int e = 0; e < VW; ++e) z[VW * g + e] = float(SI::dec(v.v[e]));
                    }
                    // two vectors at a time through the tail: eight or sixteen
                    // independent f64 chains hide each other's latency
                    if constexpr (TAIL && (SI::dt == F32 || SI::dt == BF16)) tail_vec<SI, 2 * VW>(z, tail, tab);
#pragma unroll
                    for (int e = 0; e < 2 * VW; ++e) xb[VW * i + e] = __builtin_bit_cast(uint32_t, z[e]);
                }
                loaded = true;
            }
        }
        if (!loaded) {
#pragma unroll
            for (int s = 0; s < kVLane; ++s) {
                const int o = voff<VW>(lane, s);
                xb[s] = __builtin_bit_cast(uint32_t, o < nvalid ? float(SI::dec(xr[o])) : -__builtin_huge_valf());
            }
        }
        if constexpr (TAIL) {
            if (!loaded || !(SI::dt == F32 || SI::dt == BF16)) // (else the vectors took it as they arrived)
#pragma unroll
                for (int s = 0; s < kVLane; ++s)
                    if (full || voff<VW>(lane, s) < nvalid)
                        xb[s] = __builtin_bit_cast(uint32_t, vtail<SI>(__builtin_bit_cast(float, xb[s]), tail));
            if (orow) {
                bool stored = false;
                if constexpr (VW > 1) {
                    if (full) {
#pragma unroll
                        for (int i = 0; i < kVLane / VW; ++i) {
                            Vec<raw, VW> w;
#pragma unroll
                            for (int e = 0; e < VW; ++e) w.v[e] = SI::enc32(__builtin_bit_cast(float, xb[VW * i + e]));
                            st16_stream<raw, VW>(orow + VW * lane + 64 * VW * i, w);
                        }
                        stored = true;
                    }
                }
                if (!stored) {
#pragma unroll
                    for (int s = 0; s < kVLane; ++s) {
                        const int o = voff<VW>(lane, s);
                        if (o < nvalid) orow[o] = SI::enc32(__builtin_bit_cast(float, xb[s]));
                    }
                }
            }
        }
    }

    // Exact top-nk keys of a loaded chunk (nk <= 16), largest first, into
    // sb (high words) and so (offsets): xb becomes the keys' high words (0
    // past nvalid), and each of nk rounds takes the largest remaining key —
    // the largest high word, at its lowest offset — and clears it. Register
    // only; the chunk kernel's rare path (ties at t, NaN in a block).
    template <int VW>
    MG_DEV void chunk_exact_top(uint32_t (&xb)[kVLane], int nvalid, int nk, uint32_t *sb, uint32_t *so)
    {
        const int lane = threadIdx.x & 63;
        const bool full = nvalid == kVChunk;
#pragma unroll
        for (int s = 0; s < kVLane; ++s)
            xb[s] = (full || voff<VW>(lane, s) < nvalid) ? vhi(__builtin_bit_cast(float, xb[s])) : 0u;
        for (int i = 0; i < nk; ++i) {
            uint32_t hm = 0;
#pragma unroll
            for (int s = 0; s < kVLane; ++s) hm = xb[s] > hm ? xb[s] : hm;
            hm = dpp_max_u32(hm);
            // within a lane offsets grow with s: the lane's first slot holding hm
            int first = kVLane;
#pragma unroll
            for (int s = kVLane - 1; s >= 0; --s) first = xb[s] == hm ? s : first;
            const uint32_t of = first < kVLane ? uint32_t(VW * lane + 64 * VW * (first / VW) + first % VW) : 0xffffffffu;
            const uint32_t om = dpp_min_u32(of);
            const int clear = of == om ? first : kVLane; // in the one lane holding it
#pragma unroll
            for (int s = 0; s < kVLane; ++s) xb[s] = s == clear ? 0u : xb[s];
            if (lane == 0) {
                sb[i] = hm;
                so[i] = om;
            }
        }
    }

    MG_DEV uint64_t readlane64(uint64_t v, int l)
    {
        const uint32_t lo = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(v)), l));
        const uint32_t hi = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(v >> 32)), l));
        return (uint64_t(hi) << 32) | lo;
    }

    // Pass 1 on chunk `ch` of `row`, one wave: the chunk's partial and block.
    // sb, so and sel are LDS arrays of kCand entries.
    template <class SI, int VW, bool TAIL>
    MG_DEV void chunk_pass(const typename SI::raw *__restrict__ L, int64_t ld, int64_t V, int K, int nch,
                           VPart *__restrict__ part, uint64_t *__restrict__ blk, const VTail &tail, int ch,
                           int64_t row, uint32_t *sb, uint32_t *so, uint64_t *sel, const double *tab)
    {
        using raw = typename SI::raw;
        const int lane = threadIdx.x & 63;
        const int64_t cb = int64_t(ch) * kVChunk;
        const int nvalid = int(V - cb < kVChunk ? V - cb : kVChunk);
        uint32_t xb[kVLane];
        auto x = [&](int s) { return __builtin_bit_cast(float, xb[s]); };
        chunk_load<SI, VW, TAIL>(L + row * ld + cb, nvalid, tail,
                                 tail.out ? static_cast<raw *>(tail.out) + row * V + cb : nullptr, xb, tab);

        // lane maximum over the non-NaN entries (fmax passes NaN's partner on)
        float m1 = -__builtin_huge_valf();
#pragma unroll
        for (int s = 0; s < kVLane; ++s) m1 = __builtin_fmaxf(m1, x(s));
        const float MX = dpp_max(m1);

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
            // NaN or +inf present, or no finite entry: the finite max and the
            // sum over the finite entries
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
        }
        const bool fin = FM > -__builtin_huge_valf();

        // ---- the block: the chunk's top D keys
        const int D = K < kBlk ? K : kBlk;
        // t: the D-th largest lane maximum, equal values counted (the lane
        // maxima sorted by a bitonic network, read at lane D-1); at least D
        // keys are >= t (-inf when fewer than D lanes hold a finite maximum).
        // m1 is never NaN (fmax drops NaN operands) and -0 sorts as +0.
        float t;
        {
            uint32_t mk[1] = {f32_key(m1 + 0.0f)};
            wave_bitonic_desc<uint32_t, 1>(mk);
            t = key_f32(uint32_t(__builtin_amdgcn_readlane(int(mk[0]), D - 1)));
        }
        // candidates: the keys >= t (never NaN; the -inf placeholders past V
        // only when t is -inf, which takes the exact path), compacted into LDS
        int n = 0;
        if (t > -__builtin_huge_valf()) {
#pragma unroll
            for (int s = 0; s < kVLane; ++s) {
                const bool take = x(s) >= t;
                const uint64_t mk = __builtin_amdgcn_ballot_w64(take);
                if (mk) {
                    const int p = n + lane_rank(mk);
                    if (take && p < kCand) {
                        sb[p] = xb[s];
                        so[p] = uint32_t(voff<VW>(lane, s));
                    }
                    n += __builtin_popcountll(mk);
                }
            }
        }
        // t = -inf (fewer than D lanes with a finite maximum), too many keys
        // (ties at t): the exact top D instead (sb then holds high words)
        const bool exact = !(t > -__builtin_huge_valf()) || n > kCand;
        if (exact) {
            n = nvalid < D ? nvalid : D;
            wave_lds_sync();
            chunk_exact_top<VW>(xb, nvalid, n, sb, so);
        }
        wave_lds_sync();
        // rank the n <= 64 candidates (keys are unique, so ranks are distinct)
        const uint64_t key = lane < n ? vkey(exact ? sb[lane] : vhi(__builtin_bit_cast(float, sb[lane])),
                                             uint32_t(cb + so[lane]))
                                      : 0;
        int rank = 0;
        for (int j = 0; j < n; ++j) rank += readlane64(key, j) > key ? 1 : 0;
        if (lane < n) sel[rank] = key;
        wave_lds_sync();
        const int nb = n < D ? n : D; // keys in the block
        const int64_t cid = row * nch + ch;
        if (lane < kBlk) blk[cid * kBlk + lane] = lane < nb ? sel[lane] : 0;
        if (lane == 0) {
            VPart p;
            p.l = l;
            p.kd = nvalid > nb ? sel[nb - 1] : 0;
            p.top = sel[0];
            p.m = fin ? FM : 0.0f;
            p.fin = fin ? 1 : 0;
            p.pad0 = p.pad1 = 0;
            part[cid] = p;
        }
    }

    template <class SI, int VW, bool TAIL>
    __global__ __launch_bounds__(64) void k_vocab_chunk(const typename SI::raw *__restrict__ L, int64_t ld,
                                                        int64_t V, int K, int nch, VPart *__restrict__ part,
                                                        uint64_t *__restrict__ blk, VTail tail)
    {
        __shared__ uint32_t sb[kCand], so[kCand];
        __shared__ uint64_t sel[kCand];
        __shared__ __align__(16) double tab[TAIL ? 128 : 2]; // the tanh table, read at random: LDS, not the cache
        if constexpr (TAIL) {
            *reinterpret_cast<Vec<double, 2> *>(tab + 2 * (threadIdx.x & 63)) =
                *reinterpret_cast<const Vec<double, 2> *>(mgm::kTanhTab + 2 * (threadIdx.x & 63));
            wave_lds_sync();
        }
        chunk_pass<SI, VW, TAIL>(L, ld, V, K, nch, part, blk, tail, int(blockIdx.x), blockIdx.y, sb, so, sel, tab);
    }

    // ------------------------------------------------------------------ pass 2
    // The K-th largest key over a key source, by 8-bit radix selection with an
    // LDS histogram: each pass counts the keys that match the digits fixed so
    // far, per value of the next digit. `each(f)` calls f(key) for every key
    // of the source held by this lane (0 = no key); at least K keys exist.
    template <class EACH>
    MG_DEV uint64_t source_kth(EACH each, int K, uint32_t *hist)
    {
        const int lane = threadIdx.x & 63;
        uint64_t prefix = 0;
        int need = K;
        for (int sh = 56; sh >= 0; sh -= 8) {
            const uint64_t fixed = sh == 56 ? 0 : ~((uint64_t(1) << (sh + 8)) - 1);
            wave_lds_sync();
            *reinterpret_cast<Vec<uint32_t, 4> *>(hist + 4 * lane) = Vec<uint32_t, 4>{{0u, 0u, 0u, 0u}};
            wave_lds_sync();
            each([&](uint64_t k) {
                if (k && (k & fixed) == prefix) atomicAdd(hist + int((k >> sh) & 0xff), 1u);
            });
            wave_lds_sync();
            const Vec<uint32_t, 4> cv = *reinterpret_cast<const Vec<uint32_t, 4> *>(hist + 4 * lane);
            const int sl = int(cv.v[0] + cv.v[1] + cv.v[2] + cv.v[3]);
            const int incl = wave_prefix_sum(sl);
            const int above_lane = __builtin_amdgcn_readlane(incl, 63) - incl; // in higher bins
            const bool mine = above_lane < need && need <= above_lane + sl;
            int dg = 0, above = 0;
            if (mine) {
                int acc = above_lane;
                for (int e = 3; e >= 0; --e) {
                    if (acc + int(cv.v[e]) >= need) {
                        dg = 4 * lane + e;
                        above = acc;
                        break;
                    }
                    acc += int(cv.v[e]);
                }
            }
            const int src = int(__builtin_ctzll(__builtin_amdgcn_ballot_w64(mine)));
            dg = __builtin_amdgcn_readlane(dg, src);
            above = __builtin_amdgcn_readlane(above, src);
            prefix |= uint64_t(dg) << sh;
            need -= above;
        }
        return prefix;
    }

    // lse and argmax of a row from its chunk partials: each(f) calls f on
    // every partial this lane holds. The largest chunk key is the row's first
    // maximum; x0 is the row's first logit (tail-transformed).
    template <class EACH>
    MG_DEV void fold_row(EACH each, float x0, int64_t row, double *lse, int64_t *amax)
    {
        const int lane = threadIdx.x & 63;
        float M = -__builtin_huge_valf();
        uint64_t ak = 0;
        bool any = false;
        each([&](const VPart &p) {
            if (p.fin) {
                M = p.m > M ? p.m : M;
                any = true;
            }
            ak = p.top > ak ? p.top : ak;
        });
        M = dpp_max(M);
        ak = dpp_reduce(ak, uint64_t(0), [](uint64_t u, uint64_t v) { return u > v ? u : v; });
        any = __builtin_amdgcn_ballot_w64(any) != 0;
        // sum of l_c * e^(m_c - M): the f32 difference and hardware exp2 keep
        // each term within a few ulp of f32, far inside the lse tolerance
        double S = 0.0;
        if (any)
            each([&](const VPart &p) {
                if (p.fin) S += p.l * double(__builtin_amdgcn_exp2f((p.m - M) * 1.44269504088896341f));
            });
        S = dpp_sum(S);
        if (lane == 0) {
            if (lse) lse[row] = any ? double(M) + mgm::log(S) : -__builtin_huge_val();
            // the scan starts at index 0: a NaN there is never beaten
            if (amax) amax[row] = (x0 != x0 || ak == 0) ? 0 : int64_t(vkey_index(ak));
        }
    }

    // The K selected keys, sorted, slot 64*q + lane of a[q], to the outputs
    template <class SI, bool TAIL, int SL>
    MG_DEV void emit_top(const typename SI::raw *__restrict__ L, int64_t ld, int64_t V, int K, int64_t row,
                         const uint64_t *a, int64_t *top_idx, float *top_val, const VTail &tail)
    {
        const int lane = threadIdx.x & 63;
#pragma unroll
        for (int q = 0; q < SL; ++q) {
            const int i = 64 * q + lane;
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
                    tv = float(SI::dec(L[row * ld + j]));
                    if constexpr (TAIL) tv = vtail<SI>(tv, tail);
                }
                if (top_val) top_val[row * K + i] = tv;
            }
        }
    }

    // Exact top nk = min(K, nvalid) keys (K <= 64) of one chunk, re-read from
    // the logits, sorted into stage[0..63] (0 past nk). t, the K-th largest
    // lane maximum, has at least K keys at or above it; when at most 256
    // keys reach it they are sorted by a bitonic network, else (ties, NaN,
    // fewer than K finite lane maxima) nk rounds of chunk_exact_top select
    // them. stage holds 256 keys; sb and so kCand words each.
    template <class SI, int VW, bool TAIL>
    MG_DEV int chunk_topk(const typename SI::raw *__restrict__ xr, int nvalid, int K, const VTail &tail, int64_t cb,
                          uint64_t *stage, uint32_t *sb, uint32_t *so)
    {
        const int lane = threadIdx.x & 63;
        uint32_t xb[kVLane];
        auto x = [&](int s) { return __builtin_bit_cast(float, xb[s]); };
        chunk_load<SI, VW, TAIL>(xr, nvalid, tail, nullptr, xb, mgm::kTanhTab); // (rare: the table from memory)
        float m1 = -__builtin_huge_valf();
#pragma unroll
        for (int s = 0; s < kVLane; ++s) m1 = __builtin_fmaxf(m1, x(s));
        uint32_t mk[1] = {f32_key(m1 + 0.0f)};
        wave_bitonic_desc<uint32_t, 1>(mk);
        const float t = key_f32(uint32_t(__builtin_amdgcn_readlane(int(mk[0]), K - 1)));
        const int nk = nvalid < K ? nvalid : K;
        int n = 0;
        wave_lds_sync();
        if (t > -__builtin_huge_valf()) {
#pragma unroll
            for (int s = 0; s < kVLane; ++s) {
                const bool take = x(s) >= t;
                const uint64_t m = __builtin_amdgcn_ballot_w64(take);
                if (m) {
                    const int p = n + lane_rank(m);
                    if (take && p < 256) stage[p] = vkey(vhi(x(s)), uint32_t(cb + voff<VW>(lane, s)));
                    n += __builtin_popcountll(m);
                }
            }
        }
        if (t > -__builtin_huge_valf() && n <= 256) {
            wave_lds_sync();
            uint64_t v[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] = 64 * q + lane < n ? stage[64 * q + lane] : 0;
            if (n <= 64) {
                uint64_t v1[1] = {v[0]};
                wave_bitonic_desc<uint64_t, 1>(v1);
                v[0] = v1[0];
            } else if (n <= 128) {
                uint64_t v2[2] = {v[0], v[1]};
                wave_bitonic_desc<uint64_t, 2, true>(v2);
                v[0] = v2[0];
            } else {
                wave_bitonic_desc<uint64_t, 4, true>(v);
            }
            wave_lds_sync();
            stage[lane] = lane < nk ? v[0] : 0;
        } else {
            wave_lds_sync();
            chunk_exact_top<VW>(xb, nvalid, nk, sb, so);
            wave_lds_sync();
            stage[lane] = lane < nk ? vkey(sb[lane], uint32_t(cb + so[lane])) : 0;
        }
        wave_lds_sync();
        return nk;
    }

    // Pass 2, one wave per row. FAST (K <= 64, at most 64 chunks, at least K
    // block keys): lane c first holds chunk c's block and tries the threshold
    // selection below; the general selection runs only where that cannot
    // prove its answer.
    template <class SI, int VW, int SL, bool TAIL, bool FAST>
    __global__ __launch_bounds__(64) void k_vocab_merge(const typename SI::raw *__restrict__ L, int64_t ld,
                                                        int64_t V, int K, int nch, const VPart *__restrict__ part,
                                                        const uint64_t *__restrict__ blk, uint64_t *__restrict__ lst,
                                                        double *lse, int64_t *amax, int64_t *top_idx, float *top_val,
                                                        VTail tail)
    {
        __shared__ uint64_t sel[kMaxK];
        __shared__ uint64_t ukeys[kUnionCap];
        __shared__ __align__(16) uint32_t hist[256];
        const int lane = threadIdx.x;
        const int64_t row = blockIdx.x;
        const VPart *pr = part + row * nch;
        const uint64_t *bk = blk + row * int64_t(nch) * kBlk;
        uint64_t *ls = lst + row * int64_t(nch) * kMaxK;
        float x0 = float(SI::dec(L[row * ld]));
        if constexpr (TAIL) x0 = vtail<SI>(x0, tail);
        const bool want_top = top_idx || top_val;
        const int D = K < kBlk ? K : kBlk;
        const bool regs = want_top && nch * kBlk <= 64 * kMergeRegs;

        // the lane's chunk partials (up to two: rows of up to 128 chunks) and
        // the blocks' keys, all requested before any is used
        constexpr int PPL = 2;
        const bool pregs = nch <= 64 * PPL;
        VPart pv[PPL];
#pragma unroll
        for (int k = 0; k < PPL; ++k) {
            const int cc = lane + 64 * k;
            if (pregs && cc < nch) {
                pv[k] = pr[cc];
            } else {
                pv[k].l = 0.0;
                pv[k].kd = pv[k].top = 0;
                pv[k].m = -__builtin_huge_valf();
                pv[k].fin = pv[k].pad0 = pv[k].pad1 = 0;
            }
        }
        uint64_t r[kMergeRegs];
        auto load_r = [&]() {
#pragma unroll
            for (int q = 0; q < kMergeRegs; ++q) {
                const int i = lane + 64 * q;
                r[q] = regs && i / kBlk < nch ? bk[i] : 0;
            }
        };
        uint64_t b[kBlk]; // FAST: chunk `lane`'s block
        if constexpr (FAST) {
#pragma unroll
            for (int i = 0; i < kBlk; i += 2) {
                Vec<uint64_t, 2> w{{0, 0}};
                if (lane < nch) w = *reinterpret_cast<const Vec<uint64_t, 2> *>(bk + lane * kBlk + i);
                b[i] = w.v[0];
                b[i + 1] = w.v[1];
            }
        } else {
            load_r();
        }

        auto emit = [&](const uint64_t *a) { emit_top<SI, TAIL, SL>(L, ld, V, K, row, a, top_idx, top_val, tail); };

        auto each_part = [&](auto f) {
            if (pregs) {
#pragma unroll
                for (int k = 0; k < PPL; ++k) f(pv[k]); // absent ones: fin 0, top 0
            } else {
                for (int cc = lane; cc < nch; cc += 64) f(pr[cc]);
            }
        };
        fold_row(each_part, x0, row, lse, amax);
        if (!want_top) return;

        if constexpr (FAST) {
            // T: the K-th largest high word among the first h keys of every
            // block (h * nch >= K heads, 128 at most), by a bitonic sort of
            // two registers. At least K keys have high word >= T, so the
            // union's K-th key kap has high word >= T too, and the keys whose
            // high word reaches T (a prefix of each sorted block) hold the
            // union's top K. When at most 128 of them exist they are sorted;
            // kap is the K-th, and the answer holds when no chunk's D-th key
            // (kd: every key outside its block lies below it) exceeds kap.
            const int h0 = (K + nch - 1) / nch;
            const int h = h0 < D ? h0 : D;
#pragma unroll
            for (int i = 0; i < kBlk; ++i)
                if (i < h && lane < nch) hist[lane * h + i] = uint32_t(b[i] >> 32);
            wave_lds_sync();
            uint32_t hv[2];
#pragma unroll
            for (int q = 0; q < 2; ++q) hv[q] = 64 * q + lane < nch * h ? hist[64 * q + lane] : 0u;
            wave_bitonic_desc<uint32_t, 2, true>(hv);
            const uint32_t T = uint32_t(__builtin_amdgcn_readlane(int(hv[0]), K - 1));
            int c = 0;
#pragma unroll
            for (int i = 0; i < kBlk; ++i) c += uint32_t(b[i] >> 32) >= T ? 1 : 0;
            const int incl = wave_prefix_sum(c);
            const int ns = __builtin_amdgcn_readlane(incl, 63);
            uint64_t R = 0; // the running top 64 keys, sorted
            bool have = false;
            if (T != 0 && ns <= 128) {
                const int off = incl - c;
#pragma unroll
                for (int i = 0; i < kBlk; ++i) {
                    if (__builtin_amdgcn_ballot_w64(i < c) == 0) break;
                    if (i < c) sel[off + i] = b[i];
                }
                wave_lds_sync();
                uint64_t v[2];
#pragma unroll
                for (int q = 0; q < 2; ++q) v[q] = 64 * q + lane < ns ? sel[64 * q + lane] : 0;
                if (ns <= 64) {
                    uint64_t v1[1] = {v[0]};
                    wave_bitonic_desc<uint64_t, 1>(v1);
                    R = v1[0];
                } else {
                    wave_bitonic_desc<uint64_t, 2, true>(v);
                    R = v[0];
                }
                have = true;
            }
            if (!have) {
                // no usable T (fewer than K heads with keys, or too many
                // survivors): all block keys, 64 at a time
                for (int i0 = 0; i0 < nch * kBlk; i0 += 64) {
                    uint64_t v[1] = {i0 + lane < nch * kBlk ? bk[i0 + lane] : 0};
                    wave_bitonic<uint64_t, 1, false>(v);
                    R = top64_merge(R, v[0]);
                }
            }
            // R holds the blocks' top 64 (or all of their keys). A chunk whose
            // D-th key lies above R's K-th may hold more of the row's top K:
            // it is re-read and its top K past the block merged in. Keys
            // outside every block and list are then below R's K-th key.
            uint64_t fail = __builtin_amdgcn_ballot_w64(lane < nch && pv[0].kd > readlane64(R, K - 1));
            while (fail) {
                const int cc = int(__builtin_ctzll(fail));
                fail &= fail - 1;
                const int64_t cb = int64_t(cc) * kVChunk;
                const int nv = int(V - cb < kVChunk ? V - cb : kVChunk);
                wave_lds_sync();
                const int nk = chunk_topk<SI, VW, TAIL>(L + row * ld + cb, nv, K, tail, cb, sel, hist, hist + kCand);
                // its keys past the first D (the block's), ascending
                const int i = D + 63 - lane;
                R = top64_merge(R, i < nk ? sel[i] : 0);
                // R only grows: chunks it now proves need no re-read
                fail &= __builtin_amdgcn_ballot_w64(lane < nch && pv[0].kd > readlane64(R, K - 1));
            }
            emit(&R);
            return;
        }

        auto nvalid_of = [&](int cc) {
            const int64_t cb = int64_t(cc) * kVChunk;
            return int(V - cb < kVChunk ? V - cb : kVChunk);
        };
        // the blocks as a key source (kBlk slots per chunk, 0 past a block's end)
        auto each_block = [&](auto f) {
            for (int i0 = 0; i0 < nch * kBlk; i0 += 64) {
                const int i = i0 + lane;
                f(i < nch * kBlk ? bk[i] : uint64_t(0));
            }
        };

        // first try: kap from the blocks, proved by every chunk's D-th key
        uint64_t kap = 0;
        int have = 0;
        if (regs) {
#pragma unroll
            for (int q = 0; q < kMergeRegs; ++q) have += wave_count(r[q] != 0);
            if (have >= K) kap = wave_kth<kMergeRegs>(r, K, hist);
        } else {
            each_block([&](uint64_t k) { have += wave_count(k != 0); });
            if (have >= K) kap = source_kth(each_block, K, hist);
        }
        // chunk cc fails when keys outside its block may reach the top K
        auto fails = [&](int cc) { return kap == 0 || pr[cc].kd > kap; };
        bool bad = false;
        if (kap != 0) {
            if (pregs) {
#pragma unroll
                for (int k = 0; k < PPL; ++k) bad |= pv[k].kd > kap;
            } else {
                for (int cc = lane; cc < nch; cc += 64) bad |= pr[cc].kd > kap;
            }
        }
        bad = kap == 0 || __builtin_amdgcn_ballot_w64(bad) != 0;

        int n = 0; // keys selected into sel
        if (!bad && regs) {
            // the K keys >= kap are all in the blocks held in registers
#pragma unroll
            for (int q = 0; q < kMergeRegs; ++q) {
                const bool take = r[q] != 0 && r[q] >= kap;
                const uint64_t mk = __builtin_amdgcn_ballot_w64(take);
                if (mk) {
                    if (take && n + lane_rank(mk) < kMaxK) sel[n + lane_rank(mk)] = r[q];
                    n += __builtin_popcountll(mk);
                }
            }
        } else {
            // failing chunks: re-read into LDS as keys, exact top min(K, nvalid)
            // by radix selection there, written to the list area
            if (bad) {
                for (int cc = 0; cc < nch; ++cc) {
                    if (!fails(cc)) continue;
                    const int nv = nvalid_of(cc);
                    const int64_t cb = int64_t(cc) * kVChunk;
                    const typename SI::raw *xr = L + row * ld + cb;
                    wave_lds_sync();
#pragma unroll 16
                    for (int p0 = 0; p0 < kVChunk; p0 += 64) {
                        const int p = p0 + lane;
                        uint64_t k = 0;
                        if (p < nv) {
                            float v = float(SI::dec(xr[p]));
                            if constexpr (TAIL) v = vtail<SI>(v, tail);
                            k = vkey(vhi(v), uint32_t(cb + p));
                        }
                        ukeys[p] = k;
                    }
                    wave_lds_sync();
                    auto each_chunk = [&](auto f) {
                        for (int p0 = 0; p0 < nv; p0 += 64) f(ukeys[p0 + lane]);
                    };
                    const int nk = nv < K ? nv : K;
                    const uint64_t kth = source_kth(each_chunk, nk, hist);
                    int m = 0;
                    each_chunk([&](uint64_t k) {
                        const bool take = k != 0 && k >= kth;
                        const uint64_t mk = __builtin_amdgcn_ballot_w64(take);
                        if (take) ls[cb / kVChunk * kMaxK + m + lane_rank(mk)] = k;
                        m += __builtin_popcountll(mk);
                    });
                }
                // the lists are read back by other lanes of this wave
                __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
                wave_lds_sync();
            }
            // the source: failing chunks' lists, the other chunks' blocks
            auto each_src = [&](auto f) {
                for (int cc = 0; cc < nch; ++cc) {
                    const bool fl = bad && fails(cc);
                    const int nv = nvalid_of(cc);
                    const int cnt = fl ? (nv < K ? nv : K) : kBlk;
                    const uint64_t *src = fl ? ls + int64_t(cc) * kMaxK : bk + int64_t(cc) * kBlk;
                    for (int p0 = 0; p0 < cnt; p0 += 64) {
                        const int p = p0 + lane;
                        f(p < cnt ? src[p] : uint64_t(0));
                    }
                }
            };
            // staged in LDS when it fits, so the radix passes read LDS
            int total = 0;
            for (int cc = 0; cc < nch; ++cc) {
                const int nv = nvalid_of(cc);
                total += (bad && fails(cc)) ? (nv < K ? nv : K) : kBlk;
            }
            const bool staged = total <= kUnionCap;
            int nu = 0;
            if (staged) {
                each_src([&](uint64_t k) {
                    const uint64_t mk = __builtin_amdgcn_ballot_w64(k != 0);
                    if (k) ukeys[nu + lane_rank(mk)] = k;
                    nu += __builtin_popcountll(mk);
                });
                wave_lds_sync();
            }
            auto each_lds = [&](auto f) {
                for (int i0 = 0; i0 < nu; i0 += 64) {
                    const int i = i0 + lane;
                    f(i < nu ? ukeys[i] : uint64_t(0));
                }
            };
            const uint64_t kap2 = staged ? source_kth(each_lds, K, hist) : source_kth(each_src, K, hist);
            auto pick = [&](uint64_t k) {
                const bool take = k != 0 && k >= kap2;
                const uint64_t mk = __builtin_amdgcn_ballot_w64(take);
                if (take && n + lane_rank(mk) < kMaxK) sel[n + lane_rank(mk)] = k;
                n += __builtin_popcountll(mk);
            };
            if (staged)
                each_lds(pick);
            else
                each_src(pick);
        }
        wave_lds_sync();
        // exactly K keys were selected (keys are unique), slot 64*q + lane
        uint64_t a[SL];
#pragma unroll
        for (int q = 0; q < SL; ++q) {
            const int i = 64 * q + lane;
            a[q] = i < K ? sel[i] : 0;
        }
        wave_bitonic_desc<uint64_t, SL>(a);
        emit(a);
    }


    // RN(1 / cap) where the tail takes Markstein's quotient (1 <= |cap| <= 2^20:
    // with 2^-100 < |v| < 2^100 the quotient and the remainder stay normal)
    static float tail_rcap(double cap)
    {
        const float c = float(cap), ac = std::fabs(c);
        return ac >= 1.0f && ac <= 0x1p20f ? recip_rn(c) : 0.0f;
    }

    // The pass on `stream` with its partials in `work` (work_bytes long);
    // `room` names where they live for the error raised when they do not fit.
    static void vocab_pass(hipStream_t stream, void *work, int64_t work_bytes, const char *room, const void *logits,
                           int64_t ld, int64_t rows, int64_t V, int dt_in, int64_t K, double *lse, int64_t *amax,
                           int64_t *top_idx, float *top_val, bool tail_on, double mult, double cap, void *logits_out)
    {
        need(rows >= 0 && V > 0, "vocab_reduce: bad shape");
        need(V < (int64_t(1) << 31), "vocab_reduce: V must be < 2^31");
        need(logits != nullptr, "vocab_reduce: NULL logits");
        ld = ld ? ld : V;
        need(ld >= V, "vocab_reduce: row stride smaller than V");
        const bool want_top = top_idx || top_val;
        if (!want_top) K = 1;
        need(K >= 1 && K <= kMaxK, "vocab_reduce: K must be in [1, 256]");
        need(K <= V, "vocab_reduce: K larger than the vocabulary");
        need(rows <= 65535, "vocab_reduce: at most 65535 rows per call");
        if (rows == 0) return;
        const int nch = int((V + kVChunk - 1) / kVChunk);
        const int64_t nc = rows * nch;
        // the blocks start 256-aligned after the partials (16-byte loads)
        const int64_t part_bytes = (nc * int64_t(sizeof(VPart)) + 255) / 256 * 256;
        const int64_t need_bytes = part_bytes + nc * int64_t(sizeof(uint64_t) * (kBlk + kMaxK));
        need(need_bytes <= work_bytes, "vocab_reduce: the partials of " + std::to_string(rows) + " rows x " +
                                           std::to_string(nch) + " chunks need " + std::to_string(need_bytes) +
                                           " bytes, more than " + room + " (" + std::to_string(work_bytes) + ")");
        VPart *part = static_cast<VPart *>(work);
        uint64_t *blk = reinterpret_cast<uint64_t *>(static_cast<char *>(work) + part_bytes);
        uint64_t *lst = blk + nc * kBlk;
        const dim3 g1{unsigned(nch), unsigned(rows), 1u};
        const dim3 g2{unsigned(rows), 1u, 1u};
        // python-float scalars are f32 opmath values outside f64 (src/muse_glimmer.hpp:924-926)
        const VTail tail{float(mult), float(cap), logits_out, tail_rcap(cap)};
        auto go = [&](auto chunk, auto merge, const auto *x) {
            hipLaunchKernelGGL(chunk, g1, dim3(64), 0, stream, x, ld, V, int(K), nch, part, blk, tail);
            check_launch("k_vocab_chunk");
            hipLaunchKernelGGL(merge, g2, dim3(64), 0, stream, x, ld, V, int(K), nch, part, blk, lst, lse, amax,
                               top_idx, top_val, tail);
            check_launch("k_vocab_merge");
        };
        // the threshold merge needs lane = chunk and at least K block keys
        const int D = K < kBlk ? int(K) : kBlk;
        const bool fast = K <= 64 && nch <= 64 && int64_t(nch) * D >= K;
        auto pick = [&](auto si, auto vw, const auto *x) {
            using SI = decltype(si);
            constexpr int VW = decltype(vw)::value;
            if (fast && tail_on)
                go(k_vocab_chunk<SI, VW, true>, k_vocab_merge<SI, VW, 1, true, true>, x);
            else if (fast)
                go(k_vocab_chunk<SI, VW, false>, k_vocab_merge<SI, VW, 1, false, true>, x);
            else if (K <= 64 && tail_on)
                go(k_vocab_chunk<SI, VW, true>, k_vocab_merge<SI, VW, 1, true, false>, x);
            else if (K <= 64)
                go(k_vocab_chunk<SI, VW, false>, k_vocab_merge<SI, VW, 1, false, false>, x);
            else if (tail_on)
                go(k_vocab_chunk<SI, VW, true>, k_vocab_merge<SI, VW, 4, true, false>, x);
            else
                go(k_vocab_chunk<SI, VW, false>, k_vocab_merge<SI, VW, 4, false, false>, x);
        };
        const bool out_ok = !logits_out || aligned16(logits_out);
        if (dt_in == F32) {
            const float *x = static_cast<const float *>(logits);
            if (V % 4 == 0 && ld % 4 == 0 && aligned16(x) && out_ok)
                pick(SF32{}, std::integral_constant<int, 4>{}, x);
            else
                pick(SF32{}, std::integral_constant<int, 1>{}, x);
        } else if (dt_in == BF16) {
            const uint16_t *x = static_cast<const uint16_t *>(logits);
            if (V % 8 == 0 && ld % 8 == 0 && aligned16(x) && out_ok)
                pick(SBf16{}, std::integral_constant<int, 8>{}, x);
            else
                pick(SBf16{}, std::integral_constant<int, 1>{}, x);
        } else {
            fail("vocab_reduce: input dtype must be f32 or bf16");
        }
    }

    void launch_vocab(mg_ctx *c, const void *logits, int64_t ld, int64_t rows, int64_t V, int dt_in, int64_t K,
                      double *lse, int64_t *amax, int64_t *top_idx, float *top_val, bool tail_on, double mult,
                      double cap, void *logits_out)
    {
        vocab_pass(c->stream, c->work, c->work_bytes, "the context workspace (raise workspace_bytes at mg_open)",
                   logits, ld, rows, V, dt_in, K, lse, amax, top_idx, top_val, tail_on, mult, cap, logits_out);
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
    // (hipGetSymbolAddress allocates nothing; each GPU holds its own copy at its
    // own address); host code passes this address, never the array's name,
    // which on the host is a stand-in.
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

    void launch_vocab_noalloc(hipStream_t stream, const void *logits, int64_t ld, int64_t rows, int64_t V,
                              int dt_in, int64_t K, double *lse, int64_t *amax, int64_t *top_idx, float *top_val)
    {
        // the kernels run on the stream's device: make it current so the
        // scratch address is that device's copy (the C ABI restores the
        // caller's device on return); NULL is the current device's stream
        if (stream) {
            int sd = -1, cur = -1;
            check(hipStreamGetDevice(stream, &sd), "vocab_reduce_noalloc: hipStreamGetDevice");
            check(hipGetDevice(&cur), "vocab_reduce_noalloc: hipGetDevice");
            if (sd != cur) check(hipSetDevice(sd), "vocab_reduce_noalloc: hipSetDevice");
        }
        vocab_pass(stream, scratch_address(), kVocabScratchBytes, "the fixed scratch array", logits, ld, rows, V,
                   dt_in, K, lse, amax, top_idx, top_val, false, 1.0, 0.0, nullptr);
    }
} // namespace mg
