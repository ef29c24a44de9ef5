// Split-K decode attention for gfx950: the softmax's caller at decode.
//
// Reference: the flash-decode split and combine of the GPU engine
// (k_attn_decode_split, src/gpu/gpu_engine.cpp:1690-1812; k_attn_decode_combine,
// 1816-1857) over the KV ring of k_kv_append (481-492): for one query token at
// position qpos and every query head h (KV head g = h / groups),
//   s_j = (q_h . k_j) * scaling   for keys j in [lo, qpos], lo = window ?
//                                 max(0, qpos - window + 1) : 0, key j in slot j % slots
//   out_h = sum_j softmax(s)_j v_j                      (f32)
// Like the reference's split-K path this is a different summation schedule
// from the sequential recurrence, so its contract is a numerical envelope,
// not bits.
//
// MI355X layout of the work: one wave per (KV head, split) runs ALL the
// query heads of its GQA group (5 for the 30B-class config, 16 for 32 q / 2 kv
// heads; larger groups take several waves of up to 16 heads), so every K and
// V row is read from HBM once, and both products run on the matrix cores
// (v_mfma_f32_16x16x32_bf16; lane l = 16c + n holds row/column n and
// k-elements 8c..8c+7 of an operand, and C rows 4c..4c+3 of column n).
// Per step of 32 keys:
//   staging         coalesced 16-byte streaming loads (each instruction reads
//                   whole 256-byte key rows), requested one step ahead, then
//                   written to LDS (padded rows);
//   S^T = K Q^T     A = 16 keys x 32 dims of K read from LDS, B = the group's q
//                   rows (zero-padded to 16): C lane (head n, c) holds the
//                   scores of keys 4c..4c+3 of the tile for head n;
//   O += P V        A = P (heads x 32 keys, two tiles) straight from the S^T
//                   layout; B = V read from LDS with the transposing
//                   ds_read_b64_tr_b16 (lane (dim n, c) gets keys 4c..4c+3 of
//                   dim n). P enters as bf16(p) + bf16(p - bf16(p)) in two
//                   products, so each weight is within 2^-16 of p
//                   (relative; bf16 carries 8 significant bits).
// Online softmax per head in f32 (hardware exp2 on log2-scaled scores), the
// running sums and O rows rescaled only in steps where a head's maximum
// moved. Splits are at least 256 keys and long contexts get about one wave
// per SIMD (1024 waves), each streaming its keys. A second kernel, one
// work-group per (query head, 16 dims), merges the splits: global max, split
// weights, the weighted sum of the split accumulators.
#include "mg_device.hpp"
#include "mg_internal.hpp"

namespace mg
{
    constexpr int kAttnSplit = 256;    // shortest split (keys)
    constexpr int kAttnWaves = 1024;   // splits x kv heads aimed at for long contexts

    struct AttnArgs
    {
        int64_t nq, nkv, slots, qpos, lo, per;
        int nsplit;
        int hpg, nsub; // query heads per kv head; waves per (kv head, split), HPG heads each
        float scale2;  // scaling * log2(e)
    };

    template <int HPG, int KB> // HPG query heads per wave (<= 16), KB = head_dim / 32
    __global__ __launch_bounds__(256) void k_attn_split(const uint16_t *__restrict__ q,
                                                        const uint16_t *__restrict__ kc,
                                                        const uint16_t *__restrict__ vc, AttnArgs a,
                                                        float *__restrict__ pm, float *__restrict__ pl,
                                                        float *__restrict__ pa)
    {
        constexpr int D = 32 * KB, NT = 2 * KB; // NT output tiles of 16 dims
        constexpr int LPR = D / 8;              // lanes per 16-byte-piece row of a key
        constexpr int NLD = D / 16;             // coalesced 16-byte loads per lane per 32 keys
        constexpr int SK = D + 8, SV = D + 16;  // LDS row strides (elements): conflict-free reads
        __shared__ __align__(16) uint16_t lk[4][32 * SK];
        __shared__ __align__(16) uint16_t lv[4][32 * SV];
        const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
        const int64_t w = int64_t(blockIdx.x) * 4 + wv;
        if (w >= a.nkv * a.nsub * a.nsplit) return; // whole wave; nothing below syncs the block
        // the kv heads of one split are neighbours: they read the same ring rows
        const int sp = int(w / (a.nkv * a.nsub));
        const int64_t gs = w - int64_t(sp) * (a.nkv * a.nsub);
        const int64_t g = gs / a.nsub;
        const int64_t h0 = g * a.hpg + (gs - g * a.nsub) * HPG; // the wave's first query head
        const int64_t j0 = a.lo + int64_t(sp) * a.per;
        const int64_t j1 = j0 + a.per - 1 < a.qpos ? j0 + a.per - 1 : a.qpos;
        const int n = lane & 15, c = lane >> 4;
        const bf16x8 zero8 = {};
        uint16_t *sk = lk[wv], *sv = lv[wv];

        // B of S^T: lane (head n, c) holds q[n][32 kb + 8c ..], zero for padding heads
        bf16x8 qop[KB];
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
            qop[kb] = n < HPG ? ld_bf16x8(q + (h0 + n) * D + 32 * kb + 8 * c) : zero8;

        f32x4 o[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) o[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        float m = -__builtin_huge_valf(), l = 0.0f; // head n (replicated over c)
        const int64_t rowstride = a.nkv * D;
        // coalesced staging: lane l loads the 16-byte piece l % LPR of keys
        // l / LPR + (64 / LPR) i of the step
        const int pc = lane % LPR, pr = lane / LPR;
        const uint16_t *kg = kc + g * D + 8 * pc, *vg = vc + g * D + 8 * pc;
        Vec<uint32_t, 4> stk[NLD], stv[NLD];
        auto stage = [&](int64_t sb, int rem) {
            if (rem >= 31 && sb + 32 <= a.slots) {
                // the whole step, no ring wrap: one base, constant row steps
                const int64_t step = (64 / LPR) * rowstride;
                const uint16_t *pk = kg + (sb + pr) * rowstride, *pv = vg + (sb + pr) * rowstride;
#pragma unroll
                for (int i = 0; i < NLD; ++i) {
                    stk[i] = ld16_stream<uint32_t, 4>(reinterpret_cast<const uint32_t *>(pk + i * step));
                    stv[i] = ld16_stream<uint32_t, 4>(reinterpret_cast<const uint32_t *>(pv + i * step));
                }
                return;
            }
#pragma unroll
            for (int i = 0; i < NLD; ++i) {
                const int key = pr + (64 / LPR) * i;
                int64_t sl = sb + key;
                sl = sl >= a.slots ? sl - a.slots : sl;
                if (key <= rem) {
                    stk[i] = ld16_stream<uint32_t, 4>(reinterpret_cast<const uint32_t *>(kg + sl * rowstride));
                    stv[i] = ld16_stream<uint32_t, 4>(reinterpret_cast<const uint32_t *>(vg + sl * rowstride));
                } else {
                    stk[i] = Vec<uint32_t, 4>{{0u, 0u, 0u, 0u}};
                    stv[i] = stk[i];
                }
            }
        };
        int64_t sb = j0 % a.slots; // ring slot of key jb
        if (j0 <= j1) stage(sb, int(j1 - j0 < 64 ? j1 - j0 : 64));
        for (int64_t jb = j0; jb <= j1; jb += 32) {
            const int rem = int(j1 - jb < 64 ? j1 - jb : 64); // keys jb + i, i <= rem, are attended
#pragma unroll
            for (int i = 0; i < NLD; ++i) {
                const int key = pr + (64 / LPR) * i;
                *reinterpret_cast<Vec<uint32_t, 4> *>(sk + key * SK + 8 * pc) = stk[i];
                *reinterpret_cast<Vec<uint32_t, 4> *>(sv + key * SV + 8 * pc) = stv[i];
            }
            wave_lds_sync();
            // K as A of S^T: lane (key n, c) holds dims 32 kb + 8c.. of key 16 t + n
            bf16x8 kt[2][KB];
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int kb = 0; kb < KB; ++kb)
                    kt[t][kb] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const Vec<uint32_t, 4> *>(
                                                               sk + (16 * t + n) * SK + 32 * kb + 8 * c));
            // the next step's K and V are requested now
            int64_t sn = sb + 32;
            sn = sn >= a.slots ? sn - a.slots : sn;
            if (jb + 32 <= j1) stage(sn, int(j1 - jb - 32 < 64 ? j1 - jb - 32 : 64));
            // scores of keys jb + 16 t + 4c + r for head n
            float sc[2][4];
            float mx = -__builtin_huge_valf();
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                f32x4 st = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int kb = 0; kb < KB; ++kb) st = mfma_bf16(kt[t][kb], qop[kb], st);
#pragma unroll
                for (int r = 0; r < 4; ++r) sc[t][r] = st[r] * a.scale2;
                if (rem < 31)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        sc[t][r] = 16 * t + 4 * c + r <= rem ? sc[t][r] : -__builtin_huge_valf();
#pragma unroll
                for (int r = 0; r < 4; ++r) mx = __builtin_fmaxf(mx, sc[t][r]);
            }
            mx = rows4_max(mx);
            const float mn = __builtin_fmaxf(m, mx);
            // P as A of the P V product: element 4t + r of lane (head n, c) is key 16 t + 4c + r
            bf16x8 phi, plo;
            float ps = 0.0f;
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float p = __builtin_amdgcn_exp2f(sc[t][r] - mn);
                    ps += p;
                    const __bf16 hi = __bf16(p);
                    phi[4 * t + r] = hi;
                    plo[4 * t + r] = __bf16(p - float(hi));
                }
            if (__builtin_amdgcn_ballot_w64(mn != m) != 0) {
                // some head's running max moved: rescale its sum and its O row
                // (rows are heads 4c + r; their factors come from lanes 4c + r)
                const float corr = __builtin_amdgcn_exp2f(m - mn); // first step: 2^-inf = 0
                l *= corr;
                float cr[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) cr[r] = __shfl(corr, 4 * c + r, 64);
#pragma unroll
                for (int t = 0; t < NT; ++t)
#pragma unroll
                    for (int r = 0; r < 4; ++r) o[t][r] *= cr[r];
            }
            l += ps;
            m = mn;
            // V as B of P V: lane (dim n, c) needs keys 4c + r and 16 + 4c + r
            // of dim 16 s + n; the transposing read gives it from lanes 4j + q
            // addressing key 4c + j (+16), dims 16 s + 4q..
            const uint16_t *vr = sv + (4 * c + (n >> 2)) * SV + 4 * (n & 3);
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const bf16x4 v0 = lds_read_tr(vr + 16 * t);
                const bf16x4 v1 = lds_read_tr(vr + 16 * SV + 16 * t);
                const bf16x8 vb = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
                o[t] = mfma_bf16(phi, vb, o[t]);
                o[t] = mfma_bf16(plo, vb, o[t]);
            }
            wave_lds_sync(); // this step's reads are done before the next step's writes
            sb = sn;
        }
        l = rows4_sum(l);
        const bool empty = j0 > j1;
        if (c == 0 && n < HPG) {
            const int64_t base = (h0 + n) * a.nsplit + sp;
            pm[base] = empty ? -__builtin_huge_valf() : m;
            pl[base] = empty ? 0.0f : l;
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int hh = 4 * c + r;
            if (hh < HPG) {
                float *dst = pa + ((h0 + hh) * a.nsplit + sp) * D + n;
#pragma unroll
                for (int t = 0; t < NT; ++t) dst[16 * t] = o[t][r];
            }
        }
    }

    // merge the splits of one query head for 16 of its dims (one work-group
    // per (head, 16 dims)): M = max m_s, weights 2^(m_s - M),
    // out = sum_s w_s acc_s / sum_s w_s l_s. Thread 16 sg + d takes dim d of
    // splits sg, sg + 16, ...; the 16 partial sums are added in LDS.
    __global__ __launch_bounds__(256) void k_attn_combine(const float *__restrict__ pm, const float *__restrict__ pl,
                                                          const float *__restrict__ pa, float *__restrict__ out,
                                                          int64_t D, int nsplit)
    {
        __shared__ double redl[4];
        __shared__ float redm[4];
        __shared__ float part[4][16];
        const int64_t h = blockIdx.x;
        const int d0 = 16 * int(blockIdx.y);
        const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
        const float *mh = pm + h * nsplit, *lh = pl + h * nsplit;
        float M = -__builtin_huge_valf();
        for (int s = tid; s < nsplit; s += 256) M = __builtin_fmaxf(M, mh[s]);
        M = dpp_max(M);
        if (lane == 0) redm[wv] = M;
        __syncthreads();
        M = __builtin_fmaxf(__builtin_fmaxf(redm[0], redm[1]), __builtin_fmaxf(redm[2], redm[3]));
        double L = 0.0;
        for (int s = tid; s < nsplit; s += 256)
            if (mh[s] != -__builtin_huge_valf()) L += double(__builtin_amdgcn_exp2f(mh[s] - M)) * double(lh[s]);
        L = dpp_sum(L);
        if (lane == 0) redl[wv] = L;
        // the 16 output dims: each thread takes whole splits (64 contiguous
        // bytes of one split's partial each), so a thread has its loads in
        // flight together; then a sum over the wave and over the four waves
        float o[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) o[e] = 0.0f;
        for (int s = tid; s < nsplit; s += 256) {
            const float ms = mh[s];
            if (ms != -__builtin_huge_valf()) {
                const float wgt = __builtin_amdgcn_exp2f(ms - M);
                const Vec<float, 4> *src = reinterpret_cast<const Vec<float, 4> *>(pa + (h * nsplit + s) * D + d0);
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const Vec<float, 4> v = src[k];
#pragma unroll
                    for (int e = 0; e < 4; ++e) o[4 * k + e] = __builtin_fmaf(wgt, v.v[e], o[4 * k + e]);
                }
            }
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) o[e] = dpp_sum_f32(o[e]);
        if (lane == 0)
#pragma unroll
            for (int e = 0; e < 16; ++e) part[wv][e] = o[e];
        __syncthreads();
        if (tid < 16) {
            L = (redl[0] + redl[1]) + (redl[2] + redl[3]);
            const float inv = L > 0.0 ? float(1.0 / L) : 0.0f;
            out[h * D + d0 + tid] = ((part[0][tid] + part[1][tid]) + (part[2][tid] + part[3][tid])) * inv;
        }
    }

    void launch_attn_decode(mg_ctx *c, const uint16_t *q, const uint16_t *kc, const uint16_t *vc, int64_t nq,
                            int64_t nkv, int64_t D, int64_t slots, int64_t qpos, int64_t window, double scaling,
                            float *out)
    {
        need(nq > 0 && nkv > 0 && nq % nkv == 0, "attn_decode: q_heads must be a multiple of kv_heads");
        const int64_t hpg = nq / nkv;
        // a wave serves up to 16 query heads (the MFMA's 16 columns); larger
        // groups split over waves of the largest divisor <= 16
        int64_t hw = hpg;
        while (hw > 16 || hpg % hw != 0) --hw;
        const int64_t nsub = hpg / hw;
        need(D == 64 || D == 128, "attn_decode: head_dim must be 64 or 128");
        need(q && kc && vc && out, "attn_decode: NULL tensor");
        need(aligned16(kc) && aligned16(vc) && aligned16(q), "attn_decode: tensors must be 16-byte aligned");
        need(qpos >= 0 && slots > 0, "attn_decode: bad position or cache size");
        const int64_t lo = window > 0 ? (qpos - window + 1 > 0 ? qpos - window + 1 : 0) : 0;
        const int64_t total = qpos - lo + 1;
        need(total <= slots, "attn_decode: the attended keys do not fit the cache ring (qpos - lo + 1 > cache_slots)");
        // splits of at least 256 keys, few enough that a long context runs as
        // about one wave per SIMD, each streaming its keys with the next step's
        // loads in flight; a multiple of 32 keys (one step)
        int64_t ns = (total + kAttnSplit - 1) / kAttnSplit;
        const int64_t ns_cap = kAttnWaves / (nkv * nsub) > 1 ? kAttnWaves / (nkv * nsub) : 1;
        ns = ns < ns_cap ? ns : ns_cap;
        int64_t per = (total + ns - 1) / ns;
        per = (per + 31) / 32 * 32;
        const int nsplit = int((total + per - 1) / per);
        // maxima and sums first, then the partial outputs from a 16-byte boundary
        // (the combine reads them as 16-byte vectors)
        const int64_t pa_off = (2 * nq * nsplit + 3) / 4 * 4;
        const int64_t need_bytes = (pa_off + nq * nsplit * D) * int64_t(sizeof(float));
        need(need_bytes <= c->work_bytes, "attn_decode: partials exceed the context workspace (raise workspace_bytes at mg_open)");
        float *pm = static_cast<float *>(c->work);
        float *pl = pm + nq * nsplit;
        float *pa = pm + pa_off;
        const AttnArgs a{nq, nkv, slots, qpos, lo, per, nsplit, int(hpg), int(nsub),
                         float(double(float(scaling)) * 1.4426950408889634)};
        need((nkv * nsub * nsplit + 3) / 4 < (int64_t(1) << 31), "attn_decode: too many heads");
        const dim3 g1{unsigned((nkv * nsub * nsplit + 3) / 4), 1u, 1u};
        auto go = [&](auto kern) {
            hipLaunchKernelGGL(kern, g1, dim3(256), 0, c->stream, q, kc, vc, a, pm, pl, pa);
        };
#define MG_ATTN_CASE(H)                                                                                             \
    case H: D == 128 ? go(k_attn_split<H, 4>) : go(k_attn_split<H, 2>); break;
        switch (hw) {
            MG_ATTN_CASE(1)
            MG_ATTN_CASE(2)
            MG_ATTN_CASE(3)
            MG_ATTN_CASE(4)
            MG_ATTN_CASE(5)
            MG_ATTN_CASE(6)
            MG_ATTN_CASE(7)
            MG_ATTN_CASE(8)
            MG_ATTN_CASE(9)
            MG_ATTN_CASE(10)
            MG_ATTN_CASE(11)
            MG_ATTN_CASE(12)
            MG_ATTN_CASE(13)
            MG_ATTN_CASE(14)
            MG_ATTN_CASE(15)
            MG_ATTN_CASE(16)
        default: fail("attn_decode: unsupported group size");
        }
#undef MG_ATTN_CASE
        check_launch("k_attn_split");
        hipLaunchKernelGGL(k_attn_combine, dim3(unsigned(nq), unsigned(D / 16)), dim3(256), 0, c->stream, pm, pl, pa,
                           out, D, nsplit);
        check_launch("k_attn_combine");
    }
} // namespace mg
