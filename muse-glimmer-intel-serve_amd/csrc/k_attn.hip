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
// MI355X layout of the work: one wave per (KV head, 256-key split) runs ALL
// the query heads of its GQA group (5 for the 30B), so every K and V row is
// read from HBM once. For q.k each lane owns one key and forms the dot from
// bf16 pairs with v_dot2_f32_bf16 against the group's q rows held in LDS
// (broadcast reads); for p.v the weights go to LDS and each lane takes 8 of
// the head's dimensions (one 16-byte load of V) for every 4th key, the four
// lane groups summed once per split. Online softmax per head in f32
// (hardware exp2 on log2-scaled scores). A second kernel, four waves per
// query head, merges the splits: global max, split weights, then the weighted
// sum of the split accumulators (16-byte loads, the waves' sums added in LDS).
#include "mg_device.hpp"
#include "mg_internal.hpp"

namespace mg
{
    constexpr int kAttnSplit = 256; // keys per split
    typedef __bf16 bf16x2a __attribute__((ext_vector_type(2)));

    struct AttnArgs
    {
        int64_t nq, nkv, slots, qpos, lo, per;
        int nsplit;
        float scale2; // scaling * log2(e)
    };

    template <int HPG, int ND> // ND = head_dim / 2 (bf16 pairs per row), <= 64
    __global__ __launch_bounds__(256) void k_attn_split(const uint16_t *__restrict__ q,
                                                        const uint16_t *__restrict__ kc,
                                                        const uint16_t *__restrict__ vc, AttnArgs a,
                                                        float *__restrict__ pm, float *__restrict__ pl,
                                                        float *__restrict__ pa)
    {
        constexpr int D = 2 * ND;
        __shared__ __align__(16) uint32_t sq[4][HPG][64];
        __shared__ __align__(16) float spw[4][HPG][64];
        const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
        const int64_t w = int64_t(blockIdx.x) * 4 + wv;
        if (w >= a.nkv * a.nsplit) return; // whole wave
        const int64_t g = w / a.nsplit;
        const int sp = int(w - g * a.nsplit);
        const int64_t j0 = a.lo + int64_t(sp) * a.per;
        const int64_t j1 = j0 + a.per - 1 < a.qpos ? j0 + a.per - 1 : a.qpos;

        // the group's q rows as bf16 pairs
#pragma unroll
        for (int hh = 0; hh < HPG; ++hh)
            sq[wv][hh][lane] = lane < ND ? reinterpret_cast<const uint32_t *>(q + (g * HPG + hh) * D)[lane] : 0u;
        wave_lds_sync();

        // p.v: lane = 16 * kk + dg owns dims 8*dg..8*dg+7 for keys u = kk (mod 4)
        const int kk = lane >> 4, dg = lane & 15;
        const bool dim_on = 8 * dg < D;
        float m[HPG], l[HPG], acc[HPG][8];
#pragma unroll
        for (int hh = 0; hh < HPG; ++hh) {
            m[hh] = -__builtin_huge_valf();
            l[hh] = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[hh][e] = 0.0f;
        }
        const int64_t rowstride = a.nkv * D;
        const uint32_t *vbase = reinterpret_cast<const uint32_t *>(vc + g * D);
        for (int64_t jb = j0; jb <= j1; jb += 64) {
            // ring slots without a division per key: keys jb.. are consecutive
            const int64_t sb = jb % a.slots;
            const int64_t j = jb + lane;
            const bool valid = j <= j1;
            int64_t sj = sb + lane;
            sj = sj >= a.slots ? sj - a.slots : sj;
            float s[HPG];
#pragma unroll
            for (int hh = 0; hh < HPG; ++hh) s[hh] = 0.0f;
            if (valid) {
                const uint32_t *kr = reinterpret_cast<const uint32_t *>(kc + sj * rowstride + g * D);
                Vec<uint32_t, 4> kv[ND / 4];
#pragma unroll
                for (int p = 0; p < ND / 4; ++p) kv[p] = ld16<uint32_t, 4>(kr + 4 * p); // cached: 16-byte pieces of each line
#pragma unroll
                for (int p = 0; p < ND / 4; ++p) {
#pragma unroll
                    for (int hh = 0; hh < HPG; ++hh) {
                        const Vec<uint32_t, 4> qv = *reinterpret_cast<const Vec<uint32_t, 4> *>(&sq[wv][hh][4 * p]);
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            s[hh] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2a, qv.v[e]),
                                                                    __builtin_bit_cast(bf16x2a, kv[p].v[e]), s[hh], false);
                    }
                }
            }
            // online softmax, log2 domain; the key weights go to LDS
#pragma unroll
            for (int hh = 0; hh < HPG; ++hh) {
                const float t = valid ? s[hh] * a.scale2 : -__builtin_huge_valf();
                const float mn = __builtin_fmaxf(m[hh], dpp_max(t));
                const float corr = __builtin_amdgcn_exp2f(m[hh] - mn); // first step: 2^-inf = 0
                const float pw = __builtin_amdgcn_exp2f(t - mn);
                spw[wv][hh][lane] = pw;
                l[hh] = l[hh] * corr + dpp_sum_f32(pw);
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[hh][e] *= corr;
                m[hh] = mn;
            }
            wave_lds_sync();
            // p . v over this step's keys: 4 keys at a time, one per lane group
            const int nk = int(j1 - jb + 1 < 64 ? j1 - jb + 1 : 64);
            for (int u0 = 0; u0 < nk; u0 += 16) {
                Vec<uint32_t, 4> vv[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int u = u0 + 4 * r + kk;
                    int64_t su = sb + u;
                    su = su >= a.slots ? su - a.slots : su;
                    if (u < nk && dim_on)
                        vv[r] = ld16_stream<uint32_t, 4>(vbase + su * (rowstride / 2) + 4 * dg);
                    else
                        vv[r] = Vec<uint32_t, 4>{{0u, 0u, 0u, 0u}};
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int u = u0 + 4 * r + kk;
                    if (u < nk) {
                        float v[8];
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            v[2 * e] = bf16_f32(vv[r].v[e] & 0xffffu);
                            v[2 * e + 1] = bf16_f32(vv[r].v[e] >> 16);
                        }
#pragma unroll
                        for (int hh = 0; hh < HPG; ++hh) {
                            const float wgt = spw[wv][hh][u];
#pragma unroll
                            for (int e = 0; e < 8; ++e) acc[hh][e] = __builtin_fmaf(wgt, v[e], acc[hh][e]);
                        }
                    }
                }
            }
            wave_lds_sync(); // the next step rewrites spw
        }
        // the four lane groups' partial sums
#pragma unroll
        for (int hh = 0; hh < HPG; ++hh)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                acc[hh][e] += __shfl_xor(acc[hh][e], 16, 64);
                acc[hh][e] += __shfl_xor(acc[hh][e], 32, 64);
            }
#pragma unroll
        for (int hh = 0; hh < HPG; ++hh) {
            const int64_t h = g * HPG + hh, base = h * a.nsplit + sp;
            if (lane == 0) {
                pm[base] = j0 > j1 ? -__builtin_huge_valf() : m[hh];
                pl[base] = j0 > j1 ? 0.0f : l[hh];
            }
            if (kk == 0 && dim_on) {
                Vec<float, 4> lo, hi;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    lo.v[e] = acc[hh][e];
                    hi.v[e] = acc[hh][4 + e];
                }
                *reinterpret_cast<Vec<float, 4> *>(pa + base * D + 8 * dg) = lo;
                *reinterpret_cast<Vec<float, 4> *>(pa + base * D + 8 * dg + 4) = hi;
            }
        }
    }

    // merge the splits of one query head (four waves): M = max m_s, weights
    // 2^(m_s - M), out = sum_s w_s acc_s / sum_s w_s l_s. Lane 16*kk + dg of
    // wave w takes dims 8*dg.. of splits s = 4*(4*i + w) + kk ... i.e. every
    // 16th split from 4*w + kk; the 16 partial vectors are added in LDS.
    __global__ __launch_bounds__(256) void k_attn_combine(const float *__restrict__ pm, const float *__restrict__ pl,
                                                          const float *__restrict__ pa, float *__restrict__ out,
                                                          int64_t D, int nsplit)
    {
        __shared__ float wsp[1024];
        __shared__ double redl[4];
        __shared__ float redm[4];
        __shared__ __align__(16) float part[16][128];
        const int64_t h = blockIdx.x;
        const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
        const float *mh = pm + h * nsplit, *lh = pl + h * nsplit;
        float M = -__builtin_huge_valf();
        for (int s = tid; s < nsplit; s += 256) M = __builtin_fmaxf(M, mh[s]);
        M = dpp_max(M);
        if (lane == 0) redm[wv] = M;
        __syncthreads();
        M = __builtin_fmaxf(__builtin_fmaxf(redm[0], redm[1]), __builtin_fmaxf(redm[2], redm[3]));
        double L = 0.0;
        for (int s = tid; s < nsplit; s += 256) {
            const float wgt = mh[s] == -__builtin_huge_valf() ? 0.0f : __builtin_amdgcn_exp2f(mh[s] - M);
            wsp[s] = wgt;
            L += double(wgt) * double(lh[s]);
        }
        L = dpp_sum(L);
        if (lane == 0) redl[wv] = L;
        __syncthreads();
        L = (redl[0] + redl[1]) + (redl[2] + redl[3]);
        const int kk = lane >> 4, dg = lane & 15, grp = 4 * wv + kk; // 16 groups
        float o[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
        if (8 * dg < D)
            for (int s = grp; s < nsplit; s += 16) {
                const float w = wsp[s];
                const float *src = pa + (h * nsplit + s) * D + 8 * dg;
                const Vec<float, 4> a0 = *reinterpret_cast<const Vec<float, 4> *>(src);
                const Vec<float, 4> a1 = *reinterpret_cast<const Vec<float, 4> *>(src + 4);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    o[e] = __builtin_fmaf(w, a0.v[e], o[e]);
                    o[4 + e] = __builtin_fmaf(w, a1.v[e], o[4 + e]);
                }
            }
        if (8 * dg < D)
#pragma unroll
            for (int e = 0; e < 8; ++e) part[grp][8 * dg + e] = o[e];
        __syncthreads();
        const float inv = L > 0.0 ? float(1.0 / L) : 0.0f;
        for (int64_t d = tid; d < D; d += 256) {
            float t = 0.0f;
#pragma unroll
            for (int g2 = 0; g2 < 16; ++g2) t += part[g2][d];
            out[h * D + d] = t * inv;
        }
    }

    void launch_attn_decode(mg_ctx *c, const uint16_t *q, const uint16_t *kc, const uint16_t *vc, int64_t nq,
                            int64_t nkv, int64_t D, int64_t slots, int64_t qpos, int64_t window, double scaling,
                            float *out)
    {
        need(nq > 0 && nkv > 0 && nq % nkv == 0, "attn_decode: q_heads must be a multiple of kv_heads");
        const int64_t hpg = nq / nkv;
        need(hpg <= 8, "attn_decode: at most 8 query heads per kv head");
        need(D == 64 || D == 128, "attn_decode: head_dim must be 64 or 128");
        need(q && kc && vc && out, "attn_decode: NULL tensor");
        need(aligned16(kc) && aligned16(vc) && aligned16(q), "attn_decode: tensors must be 16-byte aligned");
        need(qpos >= 0 && slots > 0, "attn_decode: bad position or cache size");
        const int64_t lo = window > 0 ? (qpos - window + 1 > 0 ? qpos - window + 1 : 0) : 0;
        const int64_t total = qpos - lo + 1;
        need(total <= slots, "attn_decode: the attended keys do not fit the cache ring (qpos - lo + 1 > cache_slots)");
        const int nsplit = int((total + kAttnSplit - 1) / kAttnSplit);
        need(nsplit <= 1024, "attn_decode: context longer than 1024 splits of 256 keys");
        const int64_t need_bytes = nq * nsplit * int64_t(sizeof(float)) * (D + 2);
        need(need_bytes <= c->work_bytes, "attn_decode: partials exceed the context workspace (raise workspace_bytes at mg_open)");
        float *pm = static_cast<float *>(c->work);
        float *pl = pm + nq * nsplit;
        float *pa = pl + nq * nsplit;
        const AttnArgs a{nq, nkv, slots, qpos, lo, kAttnSplit, nsplit, float(double(float(scaling)) * 1.4426950408889634)};
        const dim3 g1{unsigned((nkv * nsplit + 3) / 4), 1u, 1u};
        auto go = [&](auto kern) {
            hipLaunchKernelGGL(kern, g1, dim3(256), 0, c->stream, q, kc, vc, a, pm, pl, pa);
        };
#define MG_ATTN_CASE(H)                                                                                             \
    case H: D == 128 ? go(k_attn_split<H, 64>) : go(k_attn_split<H, 32>); break;
        switch (hpg) {
            MG_ATTN_CASE(1)
            MG_ATTN_CASE(2)
            MG_ATTN_CASE(3)
            MG_ATTN_CASE(4)
            MG_ATTN_CASE(5)
            MG_ATTN_CASE(6)
            MG_ATTN_CASE(7)
            MG_ATTN_CASE(8)
        default: fail("attn_decode: unsupported group size");
        }
#undef MG_ATTN_CASE
        check_launch("k_attn_split");
        hipLaunchKernelGGL(k_attn_combine, dim3(unsigned(nq)), dim3(256), 0, c->stream, pm, pl, pa, out, D, nsplit);
        check_launch("k_attn_combine");
    }
} // namespace mg
