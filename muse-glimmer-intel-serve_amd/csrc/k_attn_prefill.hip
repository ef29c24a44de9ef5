// Tiled prefill attention for gfx950: the softmax's caller over a whole
// prompt chunk, on the matrix cores.
//
// Reference: the GPU engine's --flash-prefill tier (attention_flash,
// src/gpu/gpu_engine.cpp:3292-3372, with k_flash_softmax 1481-1545 and
// k_flash_finish 1547-1560) over the KV ring of k_kv_append (481-492): query
// row t (position pos0 + t) of head h attends keys j in [lo_t, pos0 + t],
// lo_t = window > 0 ? max(0, pos0 + t - window + 1) : 0, key j in slot
// j % slots of kv head h / (q_heads / kv_heads);
//   S = q.k * scaling, masked keys excluded; per key tile the running
//   (max, sumexp) fold, the accumulator rescale, and P = bf16(e) for the p.v
//   product (e summed in f32); out = acc / sumexp (f32).
// The same numerical contract as the reference's tier: a tile-wise summation
// schedule with bf16 probabilities in the second product, gated on an
// envelope rather than bits.
//
// Layout of the work: a work-group serves one KV head and 256 (query row,
// head) pairs of up to 8 query heads of its GQA group, row-major (51.2 rows of
// a 5-head group), in eight waves of two 16-pair tiles each: two waves on each
// of the CU's four SIMDs, up to 256 VGPRs a wave (225 at head_dim 128), and
// every K and V fragment a wave reads from LDS feeds both of its tiles, so the
// LDS carries half the bytes per pair that one-tile waves need (sixteen such
// waves, four a SIMD, ran 8 % slower; twelve that also computed the next
// step's scores ahead of the softmax, 15 % slower); every K/V tile staged in
// LDS is used by all of them; larger groups (16 for 32 q / 2 kv heads) take
// several work-groups. Per 64-key step j:
//   staging   coalesced 16-byte loads (whole 256-byte key rows per
//             instruction) of K(j+1) and then V(j+1), held in registers while
//             the step computes, then written to the free LDS buffers (padded
//             rows, conflict-free reads); one barrier per step;
//   S^T       A = 16 keys x 32 dims of K(j) from LDS, B = one of the wave's
//             16-pair tiles (registers): C lane (pair n, c) holds keys
//             4c..4c+3 of the key tile, four key tiles per step;
//   softmax   per query row in f32 (hardware exp2 of fma(score, scale, -ref)),
//             the row max and sum across the four lane groups by permlane
//             swaps; a row's reference maximum moves only when passed by more
//             than 8 (log2 units), so most steps rescale nothing;
//   P V       A = P of two key tiles, straight from the S^T layout, B = V from
//             LDS through the transposing ds_read_b64_tr_b16.
// Work-groups of the last query tiles (the most keys) start first.
#include "mg_device.hpp"
#include "mg_internal.hpp"

namespace mg
{
    constexpr int kPfWaves = 8; // waves per work-group
    constexpr int kPfRT = 2;    // 16-pair tiles per wave

    struct PfArgs
    {
        int64_t T, nkv, ldq, ldo, slots, pos0, window, nqt;
        int64_t hpg, nsub; // query heads per kv head; work-groups per (kv head, tile), HPG heads each
        float scale2;      // |scaling| * log2(e), 2^-126 in place of 0
        uint32_t qsign;    // 0x80008000 when scaling < 0: q enters with its sign flipped
    };

    // HPG query heads per work-group, KB = head_dim / 32, KT 16-key tiles per
    // step, W waves of RT x 16 (query row, head) pairs each: pair p of the
    // work-group's (kv head, head subset) is query row p / HPG, head p % HPG,
    // so a wave's columns may mix rows and heads (each column is masked and
    // normalised on its own); a wave's RT tiles share every K and V fragment
    // it reads from LDS
    template <int HPG, int KB, int KT, int W, int RT>
    __global__ __launch_bounds__(64 * W) void k_attn_prefill(const uint16_t *__restrict__ q,
                                                            const uint16_t *__restrict__ kc,
                                                            const uint16_t *__restrict__ vc, PfArgs a,
                                                            float *__restrict__ out)
    {
        constexpr int D = 32 * KB, NT = 2 * KB; // NT output tiles of 16 dims
        // LDS row strides (elements), D + 16 for both: the 16-byte reads of K rows
        // and the transposing reads of V run free of bank conflicts (D + 8 for K
        // stalled a quarter of the LDS cycles)
        constexpr int SK = D + 16, SV = D + 16;
        constexpr int KS = 16 * KT;             // keys per step
        constexpr int NTHR = 64 * W;
        constexpr int PW = 16 * RT * W;                  // pairs per work-group
        constexpr int LPR = D / 8;                       // 16-byte pieces per key row
        constexpr int NPC = KS * LPR;                    // pieces per tile of K (or V)
        constexpr int PPH = (NPC + NTHR - 1) / NTHR;     // staged pieces per thread (K or V)
        __shared__ __align__(16) uint16_t lk[2][KS * SK];
        __shared__ __align__(16) uint16_t lv[2][KS * SV];
        const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63, tid = threadIdx.x;
        const int n = lane & 15, c = lane >> 4;
        // the last pair tiles attend the most keys: they start first
        const int64_t per_tile = a.nkv * a.nsub;
        const int64_t qt = a.nqt - 1 - int64_t(blockIdx.x) / per_tile;
        const int64_t gs = int64_t(blockIdx.x) - (int64_t(blockIdx.x) / per_tile) * per_tile;
        const int64_t g = gs / a.nsub;
        const int64_t h0 = g * a.hpg + (gs - g * a.nsub) * HPG; // the subset's first query head
        const int64_t npair = a.T * HPG;
        const int64_t pb0 = qt * PW;                                   // the work-group's first pair
        const int64_t pl = (pb0 + PW < npair ? pb0 + PW : npair) - 1;  // its last live pair
        const int64_t khi = a.pos0 + pl / HPG;                         // last key any row attends
        const int64_t p0 = a.pos0 + pb0 / HPG;
        const int64_t klo = a.window > 0 ? (p0 - a.window + 1 > 0 ? p0 - a.window + 1 : 0) : 0;
        const int64_t rowstride = a.nkv * D;
        const int64_t pw0 = pb0 + 16 * RT * wv; // this wave's first pair

        // B of S^T: lane (pair n, c) of tile u holds q[row][head][32 kb + 8c ..]
        // of pair pw0 + 16 u + n
        bf16x8 qop[RT][KB];
        int64_t qp[RT], ql[RT]; // this lane's query positions and window starts
#pragma unroll
        for (int u = 0; u < RT; ++u) {
            const int64_t pr = pw0 + 16 * u + n;
            const int64_t pc = pr <= pl ? pr : pl;
            const int64_t row = pc / HPG, hd = h0 + (pc - row * HPG);
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
                Vec<uint32_t, 4> w = __builtin_bit_cast(Vec<uint32_t, 4>, ld_bf16x8(q + row * a.ldq + hd * D + 32 * kb + 8 * c));
#pragma unroll
                for (int i = 0; i < 4; ++i) w.v[i] ^= a.qsign;
                qop[u][kb] = __builtin_bit_cast(bf16x8, w);
            }
            qp[u] = a.pos0 + pr / HPG;
            ql[u] = a.window > 0 ? (qp[u] - a.window + 1 > 0 ? qp[u] - a.window + 1 : 0) : 0;
        }
        // the wave's rows: first and last position (for the unmasked-step test)
        const int64_t wp0 = a.pos0 + pw0 / HPG, wp1 = a.pos0 + (pw0 + 16 * RT - 1) / HPG;

        // staging, K and V separately (one of them in registers at a time):
        // piece i of a tile is key i / LPR, 16 bytes at column i % LPR;
        // thread tid takes pieces tid + NTHR u
        Vec<uint32_t, 4> stg[PPH];
        auto stage = [&](const uint16_t *src, int64_t jb, int64_t sb) {
            if (jb + KS - 1 <= khi && sb + KS <= a.slots) {
                // a whole step inside the ring: fixed offsets from one base
                const uint16_t *base = src + sb * rowstride + g * D;
#pragma unroll
                for (int u = 0; u < PPH; ++u) {
                    const int i = tid + NTHR * u;
                    const int key = i / LPR, col = i - key * LPR;
                    if (i < NPC) stg[u] = *reinterpret_cast<const Vec<uint32_t, 4> *>(base + key * rowstride + 8 * col);
                }
                return;
            }
#pragma unroll
            for (int u = 0; u < PPH; ++u) {
                const int i = tid + NTHR * u;
                const int key = i / LPR, col = i - key * LPR;
                int64_t sl = sb + key;
                sl = sl >= a.slots ? sl - a.slots : sl;
                stg[u] = Vec<uint32_t, 4>{{0u, 0u, 0u, 0u}};
                if (i < NPC && jb + key <= khi)
                    stg[u] = *reinterpret_cast<const Vec<uint32_t, 4> *>(src + sl * rowstride + g * D + 8 * col);
            }
        };
        auto commit = [&](uint16_t *dst, int stride) {
#pragma unroll
            for (int u = 0; u < PPH; ++u) {
                const int i = tid + NTHR * u;
                const int key = i / LPR, col = i - key * LPR;
                if (i < NPC) *reinterpret_cast<Vec<uint32_t, 4> *>(dst + key * stride + 8 * col) = stg[u];
            }
        };

        f32x4 o[RT][NT];
#pragma unroll
        for (int u = 0; u < RT; ++u)
#pragma unroll
            for (int t = 0; t < NT; ++t) o[u][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        float m[RT], l[RT];
#pragma unroll
        for (int u = 0; u < RT; ++u) {
            m[u] = -__builtin_huge_valf();
            l[u] = 0.0f;
        }

        // S^T tiles of one step from a K buffer: lane (pair n, c) of tile u
        // holds keys 16 t + 4c + r, unscaled (scale2 > 0 multiplies inside the
        // exponent, and the row maximum of the scaled scores is the scaled maximum)
        auto scores = [&](const uint16_t *sk, float (&sx)[RT][KT][4]) {
#pragma unroll
            for (int t = 0; t < KT; ++t) {
                bf16x8 kt[KB]; // K as A: lane (key n, c) holds dims 32 kb + 8c.. of key 16 t + n
#pragma unroll
                for (int kb = 0; kb < KB; ++kb)
                    kt[kb] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const Vec<uint32_t, 4> *>(
                                                            sk + (16 * t + n) * SK + 32 * kb + 8 * c));
#pragma unroll
                for (int u = 0; u < RT; ++u) {
                    f32x4 st = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int kb = 0; kb < KB; ++kb) st = mfma_bf16(kt[kb], qop[u][kb], st);
#pragma unroll
                    for (int r = 0; r < 4; ++r) sx[u][t][r] = st[r];
                }
            }
        };
        auto wrap = [&](int64_t sl) { return sl >= a.slots ? sl - a.slots : sl; };

        // At the top of step j, K(j) is in lk[cur] and V(j) in lv[cur]; the
        // other buffers (K(j-1) and V(j-1), read before the last barrier) are
        // free for K(j+1) and V(j+1).
        int64_t sb = klo % a.slots; // ring slot of key jb
        stage(kc, klo, sb);
        commit(lk[0], SK);
        stage(vc, klo, sb);
        commit(lv[0], SV);
        __syncthreads();
        int cur = 0;
        auto step = [&](int64_t jb) {
            const int64_t s1 = wrap(sb + KS);
            const bool more = jb + KS <= khi;
            if (more) stage(kc, jb + KS, s1); // K(j+1), in flight through the scores and softmax
            float s[RT][KT][4];
            scores(lk[cur], s);
            // every row of the wave attends the whole step unless it reaches
            // past the wave's first row or before its last row's window
            const bool full = jb + KS - 1 <= wp0 && (a.window <= 0 || jb >= wp1 - a.window + 1);
            if (!full) {
#pragma unroll
                for (int u = 0; u < RT; ++u)
#pragma unroll
                    for (int t = 0; t < KT; ++t)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int64_t j = jb + 16 * t + 4 * c + r;
                            s[u][t][r] = (j > qp[u] || j < ql[u]) ? -__builtin_huge_valf() : s[u][t][r];
                        }
            }
            // online softmax per pair; P for the p.v product, element 4(t%2) + r
            // of pair t/2 is key 16 t + 4c + r
            bf16x8 pb[RT][KT / 2];
            bool moved = false;
            float corr[RT];
#pragma unroll
            for (int u = 0; u < RT; ++u) {
                float mx = -__builtin_huge_valf();
#pragma unroll
                for (int t = 0; t < KT; ++t)
#pragma unroll
                    for (int r = 0; r < 4; ++r) mx = __builtin_fmaxf(mx, s[u][t][r]);
                mx = rows4_max(mx) * a.scale2;
                // lazy reference: a pair's reference moves only when its new
                // maximum passes the old by more than 8 (log2 units), so its
                // weights stay at most 2^8 (exact to scale in f32 and bf16)
                // and most steps rescale nothing; a pair with nothing attended
                // yet (m = -inf) takes the first finite maximum
                const bool mv = mx > m[u] + 8.0f;
                const float mn = mv ? mx : m[u];
                // a pair with nothing attended yet keeps a zero reference: its
                // weights are 2^-inf = 0 and nothing is rescaled into NaN
                const float mref = mn == -__builtin_huge_valf() ? 0.0f : mn;
                float ev[KT][4];
#pragma unroll
                for (int t = 0; t < KT; ++t)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        ev[t][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[u][t][r], a.scale2, -mref));
                        pb[u][t / 2][4 * (t % 2) + r] = __bf16(ev[t][r]);
                    }
                // four partial sums: a short chain ahead of the barrier
                float ps4[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    ps4[r] = ev[0][r];
#pragma unroll
                    for (int t = 1; t < KT; ++t) ps4[r] += ev[t][r];
                }
                const float ps = (ps4[0] + ps4[1]) + (ps4[2] + ps4[3]);
                corr[u] = __builtin_amdgcn_exp2f(m[u] - mref);
                moved |= mv;
                l[u] = (mv ? l[u] * corr[u] : l[u]) + ps;
                m[u] = mn;
            }
            if (more) commit(lk[cur ^ 1], SK); // K(j+1) over K(j-1)
            if (more) stage(vc, jb + KS, s1);
            if (__builtin_amdgcn_ballot_w64(moved) != 0) {
                // O rows are pairs 4c + r: their factors come from lanes 4c + r
#pragma unroll
                for (int u = 0; u < RT; ++u) {
                    float cr[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) cr[r] = __shfl(corr[u], 4 * c + r, 64);
#pragma unroll
                    for (int t = 0; t < NT; ++t)
#pragma unroll
                        for (int r = 0; r < 4; ++r) o[u][t][r] *= cr[r];
                }
            }
            // V as B of P V: lane (dim n, c) gets keys 32 i + 4c + r and
            // 32 i + 16 + 4c + r of dim 16 s + n from the transposing read (lanes
            // 4j + q address key 32 i + 4c + j (+16), dims 16 s + 4q..)
            const uint16_t *vr = lv[cur] + (4 * c + (n >> 2)) * SV + 4 * (n & 3);
#pragma unroll
            for (int i = 0; i < KT / 2; ++i)
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const bf16x4 v0 = lds_read_tr(vr + 32 * i * SV + 16 * t);
                    const bf16x4 v1 = lds_read_tr(vr + (32 * i + 16) * SV + 16 * t);
                    const bf16x8 vb = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
#pragma unroll
                    for (int u = 0; u < RT; ++u) o[u][t] = mfma_bf16(pb[u][i], vb, o[u][t]);
                }
            if (more) commit(lv[cur ^ 1], SV); // V(j+1) over V(j-1)
            __syncthreads(); // the next buffers are written; these are free again
            cur ^= 1;
            sb = s1;
        };
        for (int64_t jb = klo; jb <= khi; jb += KS) step(jb);

        // out = acc / sumexp, pairs 16 u + 4c + r from lanes 4c + r
#pragma unroll
        for (int u = 0; u < RT; ++u) {
            const float lt = rows4_sum(l[u]);
            const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float ir = __shfl(inv, 4 * c + r, 64);
                const int64_t pr = pw0 + 16 * u + 4 * c + r;
                if (pr <= pl) {
                    const int64_t row = pr / HPG, hd = h0 + (pr - row * HPG);
                    float *dst = out + row * a.ldo + hd * D + n;
#pragma unroll
                    for (int t = 0; t < NT; ++t) dst[16 * t] = o[u][t][r] * ir;
                }
            }
        }
    }

    void launch_attn_prefill(mg_ctx *c, const uint16_t *q, int64_t ldq, const uint16_t *kc, const uint16_t *vc,
                             int64_t T, int64_t nq, int64_t nkv, int64_t D, int64_t slots, int64_t pos0,
                             int64_t window, double scaling, float *out, int64_t ldo)
    {
        need(nq > 0 && nkv > 0 && nq % nkv == 0, "attn_prefill: q_heads must be a multiple of kv_heads");
        const int64_t hpg = nq / nkv;
        // a work-group serves up to 8 query heads of one kv head; larger
        // groups split over work-groups of the largest divisor <= 8
        int64_t hw = hpg;
        while (hw > 8 || hpg % hw != 0) --hw;
        const int64_t nsub = hpg / hw;
        need(D == 64 || D == 128, "attn_prefill: head_dim must be 64 or 128");
        need(T >= 0 && pos0 >= 0 && slots > 0, "attn_prefill: bad shape");
        need(q && kc && vc && out, "attn_prefill: NULL tensor");
        if (ldq == 0) ldq = nq * D;
        if (ldo == 0) ldo = nq * D;
        need(ldq >= nq * D && ldo >= nq * D && ldq % 8 == 0, "attn_prefill: token stride too small or unaligned");
        need(aligned16(q) && aligned16(kc) && aligned16(vc), "attn_prefill: q and caches must be 16-byte aligned");
        if (T == 0) return;
        const int64_t lo0 = window > 0 ? (pos0 - window + 1 > 0 ? pos0 - window + 1 : 0) : 0;
        need(pos0 + T - 1 - lo0 + 1 <= slots,
             "attn_prefill: the attended keys do not fit the cache ring (pos0 + T - lo > cache_slots)");
        const int64_t nqt = (T * hw + 16 * kPfRT * kPfWaves - 1) / (16 * kPfRT * kPfWaves);
        need(nqt * nkv * nsub <= int64_t(0x7fffffff), "attn_prefill: too many query tiles");
        // the kernel scales inside the exponent by a positive factor: a negative
        // scaling flips the sign of q instead (exact in bf16 and in the products),
        // and a zero one becomes 2^-126, under which every exponent of a finite
        // score is below 2^-100 in magnitude and exp2 returns 1 as it does at 0
        const float s2 = float(double(float(scaling)) * 1.4426950408889634);
        const PfArgs a{T, nkv, ldq, ldo, slots, pos0, window, nqt, hpg, nsub,
                       s2 == 0.0f ? 0x1p-126f : __builtin_fabsf(s2), s2 < 0.0f ? 0x80008000u : 0u};
        const dim3 grid{unsigned(nqt * nkv * nsub), 1u, 1u};
        auto go = [&](auto kern, int waves) {
            hipLaunchKernelGGL(kern, grid, dim3(unsigned(64 * waves)), 0, c->stream, q, kc, vc, a, out);
        };
        // kPfWaves waves of kPfRT x 16 (row, head) pairs for groups of up to 8 heads; 64-key steps
#define MG_PF_CASE(H)                                                                                               \
    case H:                                                                                                         \
        D == 128 ? go(k_attn_prefill<H, 4, 4, kPfWaves, kPfRT>, kPfWaves) : go(k_attn_prefill<H, 2, 4, kPfWaves, kPfRT>, kPfWaves); \
        break;
        switch (hw) {
            MG_PF_CASE(1)
            MG_PF_CASE(2)
            MG_PF_CASE(3)
            MG_PF_CASE(4)
            MG_PF_CASE(5)
            MG_PF_CASE(6)
            MG_PF_CASE(7)
            MG_PF_CASE(8)
        default: fail("attn_prefill: unsupported group size");
        }
#undef MG_PF_CASE
        check_launch("k_attn_prefill");
    }
} // namespace mg
