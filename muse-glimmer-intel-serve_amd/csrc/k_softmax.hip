// Scaled, masked row softmax for gfx950.
//
// Row operator of attention_forward's softmax (src/muse_glimmer.hpp:828-885):
//   s = rnd_in(x * scale)            scale as an f32 opmath value; s rounds to
//                                    the input dtype as the eager path does (844-845)
//   softcap (cap != 0):              s = rnd_in(cap * rnd_in(tanh(rnd_in(s / cap)))),
//                                    apply_output_tail's op order (920-943), with
//                                    FDLIBM's tanh bits: the capped score is exact
//   masked keys (causal / window):   excluded, probability exactly 0
//   p = exp(s - max) / sum           written once at the output dtype
// The reference evaluates the exponentials and the sum in f64 (twin) or f32
// (compat, 856-870); here the exponentials are f32 (an accurate exp of the
// exactly formed s - max) summed in f64 in a fixed order, which keeps p within
// a few f32 ulp of the f64 value: the bf16 output is within 1 ulp of the
// twin's and the f32 output within 1e-6 relative.
//
// Rows of up to 2048 keys: one wave per row (the fast path runs one-wave
// work-groups), the row in registers (8 keys per lane per chunk), one read
// and one write of HBM. Longer rows (decode,
// q = 1, k = 131072): split over work-groups of 4096 keys; pass A writes each
// chunk's (max, sum) partial, pass B merges the partials of its row in chunk
// order (the k_attn_decode_combine rule, src/gpu/gpu_engine.cpp:1816-1857, with
// the sum rescaled in f64), re-reads its chunk (an L2 hit: a chunk goes to the
// same XCD in both passes) and writes the probabilities.
#include "mg_device.hpp"
#include "mg_internal.hpp"
#include "mg_softcap_fast.hpp"

namespace mg
{
    constexpr int kSplitChunk = 4096; // keys per work-group in the split path (256 x 16)
    constexpr unsigned kLdsPerCu = 160u * 1024u; // gfx950
    constexpr unsigned kFastWavesNoCap = 5;      // waves per SIMD of the fast path without a cap
    constexpr float kNegInf = -__builtin_huge_valf();

    struct SmArgs
    {
        int64_t nrows, q, kc;
        int64_t ldx, ldy; // row strides of scores and probabilities, in elements
        float scale, cap;
        float rcap; // RN(1 / cap): the fast path's quotient (mg_softcap_fast.hpp)
        int mask;
        int64_t window, q_pos0;
    };

    // visible key range [lo, hi] of the row
    MG_DEV void row_range(const SmArgs &a, int64_t row, int64_t &lo, int64_t &hi)
    {
        mask_range(a.mask, a.q_pos0 + row % a.q, a.kc, a.window, lo, hi);
    }

    // score transform: scale (and softcap) with the input dtype's materializations
    template <class SI, bool CAP>
    MG_DEV float score(const SmArgs &a, float x)
    {
        float s = SI::dec(SI::enc32(x * a.scale));
        if (CAP) {
            // rnd(tanh) with FDLIBM's bits (tanh_stored), so the capped score
            // is bit-identical to the twin's
            s = SI::dec(SI::enc32(s / a.cap));
            s = tanh_stored<SI>(s);
            s = SI::dec(SI::enc32(s * a.cap));
        }
        return s;
    }

    // the plain capped-score chain for the keys the fast one does not certify;
    // out of line, so the unrolled per-key code stays small
    __attribute__((noinline)) __device__ float capped_score_slow(float x, float scale, float cap)
    {
        const float s = (x * scale) / cap; // f32 operations: the twin's f64 ones rounded to f32
        return float(mgm::tanh(double(s))) * cap;
    }

    // 8 raw f32 scores of a row -> capped scores (bit e of vis set: key e is
    // visible, else it becomes -inf). Each key takes mgm::softcap_score_fast;
    // the few it does not certify (|s / cap| >= 2^-5, or a rounding too close
    // to call) are redone by the plain chain, behind one wave-uniform branch.
    MG_DEV void cap8(const SmArgs &a, float *v, uint32_t vis)
    {
        float x[8];
        uint32_t slow = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            x[e] = v[e];
            bool ok;
            const float c = mgm::softcap_score_fast(x[e], a.scale, a.cap, a.rcap, ok);
            const bool in = (vis >> e) & 1u;
            v[e] = in ? c : kNegInf;
            slow |= uint32_t(in && !ok) << e;
        }
        if (__builtin_amdgcn_ballot_w64(slow != 0u)) {
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if ((slow >> e) & 1u) v[e] = capped_score_slow(x[e], a.scale, a.cap);
        }
    }

    // 8 consecutive values -> f32 (two 16-byte loads for f32, one for 16-bit)
    template <class SI>
    MG_DEV void load8(const typename SI::raw *p, float *v)
    {
        if constexpr (sizeof(typename SI::raw) == 4) {
            const Vec<float, 4> a = ld16<float, 4>(reinterpret_cast<const float *>(p));
            const Vec<float, 4> b = ld16<float, 4>(reinterpret_cast<const float *>(p) + 4);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[e] = a.v[e];
                v[e + 4] = b.v[e];
            }
        } else {
            const Vec<uint16_t, 8> a = ld16<uint16_t, 8>(reinterpret_cast<const uint16_t *>(p));
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = SI::dec(a.v[e]);
        }
    }
    template <class SO>
    MG_DEV void store8(typename SO::raw *p, const float *v)
    {
        if constexpr (sizeof(typename SO::raw) == 4) {
            Vec<float, 4> a, b;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                a.v[e] = v[e];
                b.v[e] = v[e + 4];
            }
            st16<float, 4>(reinterpret_cast<float *>(p), a);
            st16<float, 4>(reinterpret_cast<float *>(p) + 4, b);
        } else {
            Vec<uint16_t, 8> a;
#pragma unroll
            for (int e = 0; e < 8; ++e) a.v[e] = SO::enc32(v[e]);
            st16<uint16_t, 8>(reinterpret_cast<uint16_t *>(p), a);
        }
    }

    // 8 consecutive f32 scores, non-temporal (read once; measured ~25% faster
    // than cached loads for the row softmax)
    MG_DEV void load8_stream(const float *p, float *v)
    {
        const Vec<float, 4> a = ld16_stream<float, 4>(p), b = ld16_stream<float, 4>(p + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[e] = a.v[e];
            v[e + 4] = b.v[e];
        }
    }

    // load the 8 keys j0..j0+7 of a row as transformed scores; masked or
    // out-of-row keys become -inf
    template <class SI, bool CAP>
    MG_DEV void load_scores(const SmArgs &a, const typename SI::raw *xr, int64_t j0, int64_t lo,
                            int64_t hi, bool vec, float *s)
    {
        if (j0 > hi || j0 + 7 < lo || j0 >= a.kc) {
#pragma unroll
            for (int e = 0; e < 8; ++e) s[e] = kNegInf;
            return;
        }
        float v[8];
        if (vec && j0 + 8 <= a.kc) {
            load8<SI>(xr + j0, v);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = j0 + e < a.kc ? float(SI::dec(xr[j0 + e])) : 0.0f;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int64_t j = j0 + e;
            s[e] = (j >= lo && j <= hi) ? score<SI, CAP>(a, v[e]) : kNegInf;
        }
    }

    template <class SO>
    MG_DEV void store_probs(const SmArgs &a, typename SO::raw *yr, int64_t j0, bool vec, const float *p)
    {
        if (j0 >= a.kc) return;
        if (vec && j0 + 8 <= a.kc) {
            store8<SO>(yr + j0, p);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (j0 + e < a.kc) yr[j0 + e] = SO::enc32(p[e]);
        }
    }

    // --------------------------------------------------------- one wave per row
    // Accurate row: transformed scores, exp of the exactly formed s - max, f64
    // sum, one rounding at the output. Lane `lane` owns keys 8*(lane + 64c) + e.
    template <class SI, class SO, int CH, bool CAP>
    MG_DEV void softmax_row_accurate(const SmArgs &a, const typename SI::raw *xr, typename SO::raw *yr,
                                     int64_t lo, int64_t hi, bool vec, int lane)
    {
        float s[CH][8];
        float m = kNegInf;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            load_scores<SI, CAP>(a, xr, int64_t(lane + 64 * c) * 8, lo, hi, vec, s[c]);
#pragma unroll
            for (int e = 0; e < 8; ++e) m = s[c][e] > m ? s[c][e] : m;
        }
        m = wave_max(m);
        double sum = 0.0; // f64: the row sum adds no error at the f32 output's scale
#pragma unroll
        for (int c = 0; c < CH; ++c)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                s[c][e] = s[c][e] == kNegInf ? 0.0f : exp_diff(s[c][e], m);
                sum += double(s[c][e]);
            }
        sum = wave_sum(sum);
        const float inv = m == kNegInf ? 0.0f : float(1.0 / sum);
#pragma unroll
        for (int c = 0; c < CH; ++c) {
#pragma unroll
            for (int e = 0; e < 8; ++e) s[c][e] *= inv;
            store_probs<SO>(a, yr, int64_t(lane + 64 * c) * 8, vec, s[c]);
        }
    }

    template <class SI, class SO, int CH, bool CAP>
    __global__ __launch_bounds__(256) void k_softmax_wave(const typename SI::raw *__restrict__ x,
                                                          typename SO::raw *__restrict__ y, SmArgs a,
                                                          bool vec)
    {
        const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
        if (row >= a.nrows) return; // whole wave leaves; no block barrier below
        int64_t lo, hi;
        row_range(a, row, lo, hi);
        softmax_row_accurate<SI, SO, CH, CAP>(a, x + row * a.ldx, y + row * a.ldy, lo, hi, vec, threadIdx.x & 63);
    }

    // Lean row for f32 scores and 16-bit probabilities (the attention-score
    // configuration). Scores are taken in the log2 domain,
    // p = 2^(x*c2 - max*c2) / sum on the hardware exp2, c2 = scale*log2 e > 0:
    // the max is taken over the raw scores (multiplying by c2 > 0 keeps the
    // order) and each key costs one fma, one exp2 and one add before the
    // normalisation; relative error a few 1e-7, well inside the 16-bit
    // output's half-ulp of 2e-3, so outputs stay within 1 ulp of the twin.
    // With a softcap (CAP) each visible key first becomes the twin's capped
    // score, bit for bit (cap8: mgm::softcap_score_fast, and the plain chain
    // for the keys it does not certify), and c2 = log2 e.
    // Key indices are 32-bit (rows of at most 2048 keys); chunks entirely
    // visible skip the per-key mask, chunks entirely masked skip the
    // arithmetic and store zeros. A row whose sum is not finite (NaN or
    // infinite scores) is redone on the accurate path.
    //
    // One row of the fast path in a wave's registers: lane `lane` holds keys
    // 512 c + 8 lane + e, raw scores until fast_finish transforms them.
    // key of element e of chunk c in lane `lane`: two runs of 4 keys, 256 apart,
    // so each 16-byte load instruction of the wave covers 1 KiB contiguously
    MG_DEV int fast_key(int c, int e, int lane) { return c * 512 + (e >> 2) * 256 + lane * 4 + (e & 3); }

    template <int CH>
    struct FastRow
    {
        float v[CH][8];
        int64_t lo64, hi64;
        bool live;
    };

    // issue the loads of a row's visible 512-key chunks (nothing waits on them
    // here; the finish waits for each chunk's own loads).
    // VEC (rows of a multiple of 8 keys, 16-byte aligned): every lane issues
    // its two 16-byte loads per chunk as raw buffer loads over the row's
    // visible prefix [0, hi]; loads of keys past hi (and lanes wholly below lo,
    // sent past the end) are out of range, return zeros and touch no memory.
    // With no branch around them the compiler counts the loads exactly and a
    // chunk waits only for its own data. Otherwise keys load one by one.
    template <int CH, bool VEC>
    MG_DEV void fast_load(const SmArgs &a, const float *__restrict__ x, int64_t row, int lane, FastRow<CH> &r)
    {
        // a row past the end gets the empty range, so its loads (out of
        // range) touch nothing; no branch, so the load count stays exact
        r.live = row < a.nrows;
        row_range(a, row, r.lo64, r.hi64);
        r.lo64 = r.live ? r.lo64 : 0;
        r.hi64 = r.live ? r.hi64 : -1;
        const int lo = int(r.lo64), hi = int(r.hi64); // 0 <= lo <= kc, -1 <= hi < kc <= 2048
        const float *xr = x + row * a.ldx;
        if constexpr (VEC) {
            typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
            // word 3 of a gfx9 raw buffer descriptor (32-bit data, no swizzle)
            const __amdgpu_buffer_rsrc_t rs =
                __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(xr), short(0), (hi + 1) * 4, 0x00020000);
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                const int ja = c * 512 + lane * 4, jb = ja + 256;
                const int offa = ja + 3 >= lo ? ja * 4 : 0x40000000;
                const int offb = jb + 3 >= lo ? jb * 4 : 0x40000000;
                const u32x4 p = __builtin_amdgcn_raw_buffer_load_b128(rs, offa, 0, 2); // 2: non-temporal
                const u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(rs, offb, 0, 2);
                // (element to a prvalue first: this clang lowers bit_cast of an
                // ext_vector element lvalue to a read of element 0)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    r.v[c][e] = __builtin_bit_cast(float, uint32_t(p[e]));
                    r.v[c][e + 4] = __builtin_bit_cast(float, uint32_t(q[e]));
                }
            }
        } else {
#pragma unroll
            for (int c = 0; c < CH; ++c) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int j = fast_key(c, e, lane);
                    r.v[c][e] = (j >= lo && j <= hi) ? xr[j] : 0.0f;
                }
            }
        }
    }

    // transform, normalise and store a loaded row; returns true (nothing
    // stored) for a row whose sum is not finite (NaN or infinite scores),
    // which the caller redoes on the accurate path
    template <class SO, int CH, bool CAP>
    MG_DEV bool fast_finish(const SmArgs &a, typename SO::raw *__restrict__ y, int64_t row, float c2, bool vec,
                            int lane, FastRow<CH> &r)
    {
        using ro = typename SO::raw;
        if (!r.live) return false;
        const int kc = int(a.kc), lo = int(r.lo64), hi = int(r.hi64);
        float m = kNegInf;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int cb = c * 512;
            if (cb > hi || cb + 511 < lo) continue;
            if (cb >= lo && cb + 511 <= hi) {
                if constexpr (CAP) cap8(a, r.v[c], 0xffu);
            } else {
                // a row without visible keys (lo = 0, hi = -1, mask_range)
                // skipped every chunk above, so here 0 <= hi - lo < kc
                uint32_t vis = 0;
#pragma unroll
                for (int e = 0; e < 8; ++e) vis |= uint32_t(unsigned(fast_key(c, e, lane) - lo) <= unsigned(hi - lo)) << e;
                if constexpr (CAP) {
                    cap8(a, r.v[c], vis);
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) r.v[c][e] = (vis >> e) & 1u ? r.v[c][e] : kNegInf;
                }
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) m = __builtin_fmaxf(m, r.v[c][e]);
        }
        m = dpp_max(m);
        float sum = 0.0f;
        if (m != kNegInf) {
            const float mc = m * c2;
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                const int cb = c * 512;
                if (cb > hi || cb + 511 < lo) continue;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    r.v[c][e] = __builtin_amdgcn_exp2f(__builtin_fmaf(r.v[c][e], c2, -mc)); // masked: exp2(-inf) = 0
                    sum += r.v[c][e];
                }
            }
        }
        sum = dpp_sum_f32(sum);
        ro *yr = y + row * a.ldy;
        if (m != kNegInf && !(sum < __builtin_huge_valf())) return true; // NaN / infinite scores
        const float inv = m == kNegInf ? 0.0f : __builtin_amdgcn_rcpf(sum);
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int cb = c * 512;
            const bool none = m == kNegInf || cb > hi || cb + 511 < lo;
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const int j0 = cb + hh * 256 + lane * 4;
                if (j0 >= kc) continue;
                Vec<ro, 4> o;
#pragma unroll
                for (int e = 0; e < 4; ++e) o.v[e] = none ? ro(0) : SO::enc_finite(r.v[c][4 * hh + e] * inv);
                if (vec && j0 + 4 <= kc) {
                    const Vec<uint32_t, 2> u = __builtin_bit_cast(Vec<uint32_t, 2>, o);
                    uint32_t *q = reinterpret_cast<uint32_t *>(yr + j0);
                    __builtin_nontemporal_store(u.v[0], q);
                    __builtin_nontemporal_store(u.v[1], q + 1);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (j0 + e < kc) yr[j0 + e] = o.v[e];
                }
            }
        }
        return false;
    }

    // One row per one-wave work-group. All of the row's loads are issued
    // before the first is used, and the compiler waits for each chunk's own.
    template <class SO, int CH, bool CAP, bool VEC>
    __global__ __launch_bounds__(64) void k_softmax_fast(const float *__restrict__ x,
                                                          typename SO::raw *__restrict__ y, SmArgs a, float c2)
    {
        const int lane = threadIdx.x & 63;
        const int64_t row = blockIdx.x;
        FastRow<CH> r;
        fast_load<CH, VEC>(a, x, row, lane, r);
        // a row with non-finite sums is redone on the accurate path
        if (fast_finish<SO, CH, CAP>(a, y, row, c2, VEC, lane, r))
            softmax_row_accurate<SF32, SO, CH, CAP>(a, x + row * a.ldx, y + row * a.ldy, r.lo64, r.hi64, VEC, lane);
    }

    // ------------------------------------------------------------- split rows
    MG_DEV float block_max_f32(float v, float *red)
    {
        v = wave_max(v);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
        __syncthreads();
        float t = red[0];
        for (int i = 1; i < int(blockDim.x >> 6); ++i) t = red[i] > t ? red[i] : t;
        __syncthreads();
        return t;
    }
    MG_DEV double block_sum_f64(double v, double *red)
    {
        v = wave_sum(v);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
        __syncthreads();
        double t = 0.0;
        for (int i = 0; i < int(blockDim.x >> 6); ++i) t += red[i];
        __syncthreads();
        return t;
    }

    // pass A: partial (max, sum exp(s - max)) of chunk blockIdx.x of row blockIdx.y
    template <class SI, bool CAP>
    __global__ __launch_bounds__(256) void k_softmax_partial(const typename SI::raw *__restrict__ x, SmArgs a,
                                                             bool vec, float2 *__restrict__ part)
    {
        __shared__ float red[4];
        __shared__ double redd[4];
        const int64_t row = blockIdx.y;
        int64_t lo, hi;
        row_range(a, row, lo, hi);
        const typename SI::raw *xr = x + row * a.ldx;
        const int64_t base = int64_t(blockIdx.x) * kSplitChunk;
        float s[2][8];
        float m = kNegInf;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            load_scores<SI, CAP>(a, xr, base + int64_t(threadIdx.x + 256 * c) * 8, lo, hi, vec, s[c]);
#pragma unroll
            for (int e = 0; e < 8; ++e) m = s[c][e] > m ? s[c][e] : m;
        }
        m = block_max_f32(m, red);
        double sum = 0.0;
        if (m != kNegInf)
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int e = 0; e < 8; ++e) sum += s[c][e] == kNegInf ? 0.0 : double(exp_diff(s[c][e], m));
        sum = block_sum_f64(sum, redd);
        if (threadIdx.x == 0) part[row * gridDim.x + blockIdx.x] = make_float2(m, float(sum));
    }

    // pass B: merge the row's partials, then write this chunk. Every work-group
    // of the row forms the same merge: max over the chunk maxima, then
    // sum_c l_c * exp(m_c - M) in f64 (FDLIBM exp), each thread over chunks
    // t, t+256, ... in order and the threads in a fixed tree.
    template <class SI, class SO, bool CAP>
    __global__ __launch_bounds__(256) void k_softmax_finish(const typename SI::raw *__restrict__ x,
                                                            typename SO::raw *__restrict__ y, SmArgs a,
                                                            bool vec, const float2 *__restrict__ part)
    {
        __shared__ float red[4];
        __shared__ double redd[4];
        const int64_t row = blockIdx.y;
        const int nch = int(gridDim.x);
        const float2 *pr = part + row * nch;
        // this chunk's scores first, so their latency overlaps the merge
        int64_t lo, hi;
        row_range(a, row, lo, hi);
        const typename SI::raw *xr = x + row * a.ldx;
        typename SO::raw *yr = y + row * a.ldy;
        const int64_t base = int64_t(blockIdx.x) * kSplitChunk;
        float s[2][8];
#pragma unroll
        for (int c = 0; c < 2; ++c)
            load_scores<SI, CAP>(a, xr, base + int64_t(threadIdx.x + 256 * c) * 8, lo, hi, vec, s[c]);
        float M = kNegInf;
        for (int i = threadIdx.x; i < nch; i += blockDim.x) M = pr[i].x > M ? pr[i].x : M;
        M = block_max_f32(M, red);
        double L = 0.0;
        if (M != kNegInf)
            for (int i = threadIdx.x; i < nch; i += blockDim.x)
                if (pr[i].x != kNegInf) L += double(pr[i].y) * mgm::exp(double(pr[i].x) - double(M));
        L = block_sum_f64(L, redd);
        const float inv = M == kNegInf ? 0.0f : float(1.0 / L);
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const int64_t j0 = base + int64_t(threadIdx.x + 256 * c) * 8;
#pragma unroll
            for (int e = 0; e < 8; ++e) s[c][e] = s[c][e] == kNegInf ? 0.0f : exp_diff(s[c][e], M) * inv;
            store_probs<SO>(a, yr, j0, vec, s[c]);
        }
    }

    // Long rows of f32 scores to 16-bit probabilities without softcap: the
    // log2-domain math of k_softmax_fast over 4096-key chunks (f32 partial
    // sums, merged as sum_c l_c * 2^(m_c - M)), with DPP reductions. A row
    // with NaN or +inf scores gets NaN sums and so NaN probabilities, as on
    // the accurate path; masked keys stay exactly 0.
    // STREAM: non-temporal loads (the first read of the scores); the second
    // pass reads them with ordinary loads (measured 6.4 us against 7.0 for the
    // decode row set of 40 x 131072)
    template <bool STREAM>
    MG_DEV void load_t8(const float *xr, int64_t j0, int64_t lo, int64_t hi, int64_t kc, bool vec, float c2,
                        float *t)
    {
        if (vec && j0 >= lo && j0 + 7 <= hi && j0 + 8 <= kc) {
            float v[8];
            if constexpr (STREAM) {
                load8_stream(xr + j0, v);
            } else {
                const Vec<float, 4> u0 = ld16<float, 4>(xr + j0), u1 = ld16<float, 4>(xr + j0 + 4);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[e] = u0.v[e];
                    v[e + 4] = u1.v[e];
                }
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) t[e] = v[e] * c2;
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int64_t j = j0 + e;
                t[e] = (j >= lo && j <= hi && j < kc) ? xr[j] * c2 : kNegInf;
            }
        }
    }
    MG_DEV float block_max_dpp(float v, float *red)
    {
        v = dpp_max(v);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
        __syncthreads();
        const float t = __builtin_fmaxf(__builtin_fmaxf(red[0], red[1]), __builtin_fmaxf(red[2], red[3]));
        __syncthreads();
        return t;
    }
    MG_DEV float block_sum_dpp(float v, float *red)
    {
        v = float(dpp_sum(double(v)));
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
        __syncthreads();
        const float t = (red[0] + red[1]) + (red[2] + red[3]);
        __syncthreads();
        return t;
    }

    __global__ __launch_bounds__(256) void k_softmax_partial_fast(const float *__restrict__ x, SmArgs a, float c2,
                                                                  bool vec, float2 *__restrict__ part)
    {
        __shared__ float red[4];
        const int64_t row = blockIdx.y;
        int64_t lo, hi;
        row_range(a, row, lo, hi);
        const float *xr = x + row * a.ldx;
        const int64_t base = int64_t(blockIdx.x) * kSplitChunk;
        float t[2][8];
        float m = kNegInf;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            load_t8<true>(xr, base + int64_t(threadIdx.x + 256 * c) * 8, lo, hi, a.kc, vec, c2, t[c]);
#pragma unroll
            for (int e = 0; e < 8; ++e) m = t[c][e] > m ? t[c][e] : m;
        }
        m = block_max_dpp(m, red);
        float sum = 0.0f;
        if (m != kNegInf)
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int e = 0; e < 8; ++e) sum += __builtin_amdgcn_exp2f(t[c][e] - m); // exp2(-inf) = 0
        sum = block_sum_dpp(sum, red);
        if (threadIdx.x == 0) part[row * gridDim.x + blockIdx.x] = make_float2(m, sum);
    }

    template <class SO>
    __global__ __launch_bounds__(256) void k_softmax_finish_fast(const float *__restrict__ x,
                                                                 typename SO::raw *__restrict__ y, SmArgs a,
                                                                 float c2, bool vec,
                                                                 const float2 *__restrict__ part)
    {
        __shared__ float red[4];
        const int64_t row = blockIdx.y;
        const int nch = int(gridDim.x);
        const float2 *pr = part + row * nch;
        int64_t lo, hi;
        row_range(a, row, lo, hi);
        const float *xr = x + row * a.ldx;
        typename SO::raw *yr = y + row * a.ldy;
        const int64_t base = int64_t(blockIdx.x) * kSplitChunk;
        // this chunk's scores first, so their latency overlaps the merge
        float t[2][8];
#pragma unroll
        for (int c = 0; c < 2; ++c) load_t8<false>(xr, base + int64_t(threadIdx.x + 256 * c) * 8, lo, hi, a.kc, vec, c2, t[c]);
        float M = kNegInf;
        for (int i = threadIdx.x; i < nch; i += blockDim.x) M = pr[i].x > M ? pr[i].x : M;
        M = block_max_dpp(M, red);
        float L = 0.0f;
        if (M != kNegInf)
            for (int i = threadIdx.x; i < nch; i += blockDim.x)
                if (pr[i].x != kNegInf) L += pr[i].y * __builtin_amdgcn_exp2f(pr[i].x - M);
        L = block_sum_dpp(L, red);
        const float inv = M == kNegInf ? 0.0f : 1.0f / L;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
#pragma unroll
            for (int e = 0; e < 8; ++e) t[c][e] = t[c][e] == kNegInf ? 0.0f : __builtin_amdgcn_exp2f(t[c][e] - M) * inv;
            store_probs<SO>(a, yr, base + int64_t(threadIdx.x + 256 * c) * 8, vec, t[c]);
        }
    }

    // The same two passes for rows of 16-byte-aligned, multiple-of-8 keys,
    // without a branch around any access: thread t holds keys base + 1024 c +
    // 4 t + e (each wave load covers 1 KiB contiguously), loaded through a
    // buffer resource over the row's keys [0, hi] (keys past hi read as zero
    // and are masked, keys below lo masked after the load), so all of a
    // thread's loads are in flight at once; the finishing pass stores through
    // one over the row's kc keys.
    __global__ __launch_bounds__(256) void k_softmax_partial_buf(const float *__restrict__ x, SmArgs a, float c2,
                                                                 float2 *__restrict__ part)
    {
        __shared__ float red[4];
        const int64_t row = blockIdx.y;
        int64_t lo64, hi64;
        row_range(a, row, lo64, hi64);
        const int lo = int(lo64), hi = int(hi64); // kc < 2^29: checked by the launcher
        const auto rs = buf_rsrc(x + row * a.ldx, (hi + 1) * 4);
        const int base = int(blockIdx.x) * kSplitChunk + 4 * int(threadIdx.x);
        Vec<float, 4> u[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) u[c] = buf_ld16<float, 4, kAuxNT>(rs, (base + 1024 * c) * 4);
        float t[4][4];
        float m = kNegInf;
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int j = base + 1024 * c + e;
                t[c][e] = (j >= lo && j <= hi) ? u[c].v[e] * c2 : kNegInf;
                m = __builtin_fmaxf(m, t[c][e]);
            }
        m = block_max_dpp(m, red);
        float sum = 0.0f;
        if (m != kNegInf)
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int e = 0; e < 4; ++e) sum += __builtin_amdgcn_exp2f(t[c][e] - m); // exp2(-inf) = 0
        sum = block_sum_dpp(sum, red);
        if (threadIdx.x == 0) part[row * gridDim.x + blockIdx.x] = make_float2(m, sum);
    }

    template <class SO>
    __global__ __launch_bounds__(256) void k_softmax_finish_buf(const float *__restrict__ x,
                                                                typename SO::raw *__restrict__ y, SmArgs a,
                                                                float c2, const float2 *__restrict__ part)
    {
        using ro = typename SO::raw;
        static_assert(sizeof(ro) == 2, "16-bit probabilities");
        __shared__ float red[4];
        const int64_t row = blockIdx.y;
        const int nch = int(gridDim.x);
        const float2 *pr = part + row * nch;
        int64_t lo64, hi64;
        row_range(a, row, lo64, hi64);
        const int lo = int(lo64), hi = int(hi64);
        const auto rs = buf_rsrc(x + row * a.ldx, (hi + 1) * 4);
        const auto ry = buf_rsrc(y + row * a.ldy, int(a.kc) * 2);
        const int base = int(blockIdx.x) * kSplitChunk + 4 * int(threadIdx.x);
        // the row's partials first (thread t takes partial t; rows of more
        // than 256 chunks loop over the rest), then the chunk's scores: loads
        // complete in order, so the merge waits only for the partials and runs
        // while the scores are in flight
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 pv = __builtin_amdgcn_raw_buffer_load_b64(buf_rsrc(pr, nch * 8), int(threadIdx.x) * 8, 0, 0);
        Vec<float, 4> u[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) u[c] = buf_ld16<float, 4, 0>(rs, (base + 1024 * c) * 4);
        const bool own = int(threadIdx.x) < nch;
        const float pm = own ? __builtin_bit_cast(float, uint32_t(pv[0])) : kNegInf;
        const float pl = __builtin_bit_cast(float, uint32_t(pv[1]));
        float M = pm;
        for (int i = threadIdx.x + blockDim.x; i < nch; i += blockDim.x) M = pr[i].x > M ? pr[i].x : M;
        M = block_max_dpp(M, red);
        float L = 0.0f;
        if (M != kNegInf) {
            if (pm != kNegInf) L = pl * __builtin_amdgcn_exp2f(pm - M);
            for (int i = threadIdx.x + blockDim.x; i < nch; i += blockDim.x)
                if (pr[i].x != kNegInf) L += pr[i].y * __builtin_amdgcn_exp2f(pr[i].x - M);
        }
        L = block_sum_dpp(L, red);
        const float inv = M == kNegInf ? 0.0f : 1.0f / L;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            Vec<ro, 8> o; // elements 0..3 stored (8 bytes), 4..7 unused
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int j = base + 1024 * c + e;
                const float p = (j >= lo && j <= hi) ? __builtin_amdgcn_exp2f(u[c].v[e] * c2 - M) * inv : 0.0f;
                o.v[e] = SO::enc32(p);
            }
            const Vec<uint32_t, 4> w = __builtin_bit_cast(Vec<uint32_t, 4>, o);
            typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
            u32x2 w2;
            w2[0] = w.v[0];
            w2[1] = w.v[1];
            __builtin_amdgcn_raw_buffer_store_b64(w2, ry, (base + 1024 * c) * 2, 0, kAuxNT);
        }
    }

    template <class SI, class SO, bool CAP>
    void launch_softmax_t(mg_ctx *c, const void *x, void *y, const SmArgs &a)
    {
        using ri = typename SI::raw;
        using ro = typename SO::raw;
        const bool vec = a.kc % 8 == 0 && a.ldx % 8 == 0 && a.ldy % 8 == 0 && aligned16(x) && aligned16(y);
        const ri *xi = static_cast<const ri *>(x);
        ro *yo = static_cast<ro *>(y);
        if (a.kc <= 2048) {
            const unsigned blocks = unsigned((a.nrows + 3) / 4);
            need(a.nrows < (int64_t(1) << 31), "softmax: too many rows");
            // the fast capped score takes 1 <= |cap| <= 2^20 (mg_softcap_fast.hpp,
            // the range its host checker sweeps); other caps take the accurate kernel
            const float acap = __builtin_fabsf(a.cap);
            const bool cap_ok = !CAP || (acap >= 1.0f && acap <= 0x1p20f);
            if constexpr (SI::dt == F32 && sizeof(ro) == 2) if (cap_ok && (CAP || a.scale > 0.0)) {
                // log2-domain factor: the scale folds in unless the cap comes after it
                const float c2 = float((CAP ? 1.0 : double(a.scale)) * 1.4426950408889634);
                const unsigned wgs = unsigned(a.nrows); // < 2^31: checked above
                // Without the cap the kernel needs few registers (8 waves per SIMD
                // would fit) but streams fastest at 4: the LDS each work-group
                // reserves (and never touches) holds a CU at 20 of them (measured
                // with four keys per lane and load: 110.5 us at 8 waves, 109.9 at
                // 4, 109.0 at 5, 126.4 at 3, config 4). With the cap its
                // registers allow 5, which the extra arithmetic uses.
                const unsigned lds = CAP ? 0u : kLdsPerCu / (4u * kFastWavesNoCap);
                auto go = [&](auto kern) {
                    hipLaunchKernelGGL(kern, dim3(wgs), dim3(64), lds, c->stream, xi, yo, a, c2);
                };
                if (a.kc <= 512)
                    vec ? go(k_softmax_fast<SO, 1, CAP, true>) : go(k_softmax_fast<SO, 1, CAP, false>);
                else if (a.kc <= 1024)
                    vec ? go(k_softmax_fast<SO, 2, CAP, true>) : go(k_softmax_fast<SO, 2, CAP, false>);
                else
                    vec ? go(k_softmax_fast<SO, 4, CAP, true>) : go(k_softmax_fast<SO, 4, CAP, false>);
                check_launch("k_softmax_fast");
                return;
            }
            if (a.kc <= 512)
                hipLaunchKernelGGL((k_softmax_wave<SI, SO, 1, CAP>), dim3(blocks), dim3(256), 0, c->stream, xi, yo, a, vec);
            else if (a.kc <= 1024)
                hipLaunchKernelGGL((k_softmax_wave<SI, SO, 2, CAP>), dim3(blocks), dim3(256), 0, c->stream, xi, yo, a, vec);
            else
                hipLaunchKernelGGL((k_softmax_wave<SI, SO, 4, CAP>), dim3(blocks), dim3(256), 0, c->stream, xi, yo, a, vec);
            check_launch("k_softmax_wave");
            return;
        }
        const int64_t nch = (a.kc + kSplitChunk - 1) / kSplitChunk;
        need(a.nrows <= 65535, "softmax: split path takes at most 65535 rows");
        need(a.nrows * nch * int64_t(sizeof(float2)) <= c->work_bytes,
             "softmax: partials exceed the context workspace (raise workspace_bytes at mg_open)");
        float2 *part = static_cast<float2 *>(c->work);
        const dim3 grid{unsigned(nch), unsigned(a.nrows), 1u};
        if constexpr (SI::dt == F32 && sizeof(ro) == 2 && !CAP) {
            const float c2 = float(double(a.scale) * 1.4426950408889634);
            if (vec && a.kc < (int64_t(1) << 28)) {
                hipLaunchKernelGGL(k_softmax_partial_buf, grid, dim3(256), 0, c->stream, xi, a, c2, part);
                check_launch("k_softmax_partial_buf");
                hipLaunchKernelGGL(k_softmax_finish_buf<SO>, grid, dim3(256), 0, c->stream, xi, yo, a, c2, part);
                check_launch("k_softmax_finish_buf");
                return;
            }
            hipLaunchKernelGGL(k_softmax_partial_fast, grid, dim3(256), 0, c->stream, xi, a, c2, vec, part);
            check_launch("k_softmax_partial_fast");
            hipLaunchKernelGGL(k_softmax_finish_fast<SO>, grid, dim3(256), 0, c->stream, xi, yo, a, c2, vec, part);
            check_launch("k_softmax_finish_fast");
            return;
        }
        hipLaunchKernelGGL((k_softmax_partial<SI, CAP>), grid, dim3(256), 0, c->stream, xi, a, vec, part);
        check_launch("k_softmax_partial");
        hipLaunchKernelGGL((k_softmax_finish<SI, SO, CAP>), grid, dim3(256), 0, c->stream, xi, yo, a, vec, part);
        check_launch("k_softmax_finish");
    }

    template <class SI>
    void launch_softmax_out(mg_ctx *c, const void *x, void *y, const SmArgs &a, int dt_out)
    {
        switch (dt_out) {
        case BF16: a.cap != 0.0f ? launch_softmax_t<SI, SBf16, true>(c, x, y, a) : launch_softmax_t<SI, SBf16, false>(c, x, y, a); break;
        case F16: a.cap != 0.0f ? launch_softmax_t<SI, SF16, true>(c, x, y, a) : launch_softmax_t<SI, SF16, false>(c, x, y, a); break;
        case F32: a.cap != 0.0f ? launch_softmax_t<SI, SF32, true>(c, x, y, a) : launch_softmax_t<SI, SF32, false>(c, x, y, a); break;
        default: fail("softmax: output dtype must be bf16, f16 or f32");
        }
    }

    void launch_softmax(mg_ctx *c, const void *x, int64_t ldx, void *y, int64_t ldy, int64_t heads, int64_t q,
                        int64_t kc, double scale, int mask, int64_t window, int64_t q_pos0, double softcap,
                        int dt_in, int dt_out)
    {
        need(heads >= 0 && q >= 0 && kc >= 0, "softmax: bad shape");
        ldx = ldx ? ldx : kc;
        ldy = ldy ? ldy : kc;
        need(ldx >= kc && ldy >= kc, "softmax: row strides smaller than the row length");
        need(x && y, "softmax: NULL tensor");
        need(mask >= 0 && mask <= 3, "softmax: unknown mask kind");
        need(mask < 2 || window > 0, "softmax: window masks need window > 0");
        if (heads == 0 || q == 0 || kc == 0) return;
        SmArgs a;
        a.nrows = heads * q;
        a.q = q;
        a.kc = kc;
        a.ldx = ldx;
        a.ldy = ldy;
        a.scale = float(scale);
        a.cap = float(softcap);
        a.rcap = a.cap != 0.0f ? recip_rn(a.cap) : 0.0f;
        a.mask = mask;
        a.window = window;
        a.q_pos0 = q_pos0;
        if (dt_in == F64 || dt_in == (F64 | kF32Compat)) {
            need(dt_out == F64, "softmax: f64 scores give f64 probabilities");
            launch_softmax_f64(c, x, ldx, y, ldy, heads * q, q, kc, scale, mask, window, q_pos0, softcap,
                               dt_in != F64);
            return;
        }
        switch (dt_in) {
        case F32: launch_softmax_out<SF32>(c, x, y, a, dt_out); break;
        case BF16: launch_softmax_out<SBf16>(c, x, y, a, dt_out); break;
        case F16: launch_softmax_out<SF16>(c, x, y, a, dt_out); break;
        default: fail("softmax: input dtype must be f32, bf16, f16 or f64");
        }
    }
} // namespace mg
