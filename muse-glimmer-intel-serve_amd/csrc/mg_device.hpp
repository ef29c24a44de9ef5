// Device-side helpers shared by the gfx950 kernels: storage formats, the
// twin's rounding chain, wave64 reductions, and an accurate f32 exp.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mg_fdlibm.hpp"
#include "mg_tanh_fast.hpp"

#define MG_DEV __device__ __forceinline__

namespace mg
{
    enum Dt : int { F64 = 0, BF16 = 1, F16 = 2, F32 = 3 };
    // OR-ed into an f64 dtype: the reference's --hf-f32-compat chains
    constexpr int kF32Compat = 0x100;
    constexpr int kBf16AsF32 = 4; // f32 words holding bf16 values (an output format of the mixed norm)

    // Visible keys [lo, hi] of a score row at position qpos over kc keys.
    // mask 1 causal: j <= qpos; 2 sliding window: qpos - window < j <= qpos
    // (src/muse_glimmer.hpp:838-843); 3 the drafter's bidirectional window:
    // qpos - window <= j <= qpos + window (src/dflash.hpp:339-344). A row that
    // sees no key gets the one canonical empty range lo = 0, hi = -1, so
    // 0 <= lo <= kc and hi - lo >= -1 always hold (kernels may take hi - lo as
    // an unsigned span and cast both to 32 bits for rows of < 2^31 keys).
    __host__ __device__ __forceinline__ void mask_range(int mask, int64_t qpos, int64_t kc, int64_t window,
                                                        int64_t &lo, int64_t &hi)
    {
        lo = 0;
        hi = kc - 1;
        if (mask == 3) {
            const int64_t l = qpos - window, h = qpos + window;
            lo = l > 0 ? l : 0;
            hi = h < hi ? h : hi;
        } else {
            if (mask >= 1) hi = qpos < hi ? qpos : hi;
            if (mask == 2) {
                const int64_t l = qpos - window + 1;
                lo = l > 0 ? l : 0;
            }
        }
        if (lo > hi) {
            lo = 0;
            hi = -1;
        }
    }

    // ------------------------------------------------------------ rounding
    // f32 -> bf16 bits, RNE (the gfx950 v_cvt_pk_bf16_f32 conversion), NaN
    // canonicalized to 0x7FC0 as c10 and the twin do (reference rounding.hpp:64-75).
    MG_DEV uint16_t bf16_bits(float f)
    {
        const uint16_t b = __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
        return f != f ? uint16_t(0x7fc0) : b;
    }
    // f32 -> f16 bits, RNE with subnormals (v_cvt_f16_f32), >= 65520 -> inf,
    // NaN -> sign | 0x7E00 (reference rounding.hpp:78-123)
    MG_DEV uint16_t f16_bits(float f)
    {
        const uint16_t h = __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
        return f != f ? uint16_t((h & 0x8000u) | 0x7e00u) : h;
    }
    // Opaque copy of an f32 value. Without it the backend may fold
    // f16(f32(a) * f32(b)) into v_fma_mixlo_f16 a, b, +0, which turns a -0
    // product into +0 (-0 + +0 = +0); the twin keeps the sign of zero.
    MG_DEV float opaque(float f)
    {
        __asm__("" : "+v"(f));
        return f;
    }
    MG_DEV float bf16_f32(uint32_t b) { return __builtin_bit_cast(float, b << 16); }
    MG_DEV float f16_f32(uint16_t h) { return float(__builtin_bit_cast(_Float16, h)); }

    // Storage formats. `comp` is the register type that holds a stored value
    // exactly (f32 for the 16-bit formats and f32, f64 for f64); `enc64`
    // rounds an f64 result to storage through f64 -> f32 -> storage RNE, the
    // twin's chain; `enc` rounds a comp value once.
    struct SBf16
    {
        using raw = uint16_t;
        using comp = float;
        static constexpr int dt = BF16;
        static MG_DEV float dec(raw r) { return bf16_f32(r); }
        static MG_DEV raw enc32(float f) { return bf16_bits(opaque(f)); }
        static MG_DEV raw enc64(double d) { return bf16_bits(float(d)); }
        static MG_DEV raw enc(comp c) { return bf16_bits(opaque(c)); }
        static MG_DEV raw enc_finite(float f) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(opaque(f))); }
    };
    struct SF16
    {
        using raw = uint16_t;
        using comp = float;
        static constexpr int dt = F16;
        static MG_DEV float dec(raw r) { return f16_f32(r); }
        static MG_DEV raw enc32(float f) { return f16_bits(opaque(f)); }
        static MG_DEV raw enc64(double d) { return f16_bits(float(d)); }
        static MG_DEV raw enc(comp c) { return f16_bits(opaque(c)); }
        static MG_DEV raw enc_finite(float f) { return __builtin_bit_cast(uint16_t, static_cast<_Float16>(opaque(f))); }
    };
    struct SF32
    {
        using raw = float;
        using comp = float;
        static constexpr int dt = F32;
        static MG_DEV float dec(raw r) { return r; }
        static MG_DEV raw enc32(float f) { return f; }
        static MG_DEV raw enc64(double d) { return float(d); }
        static MG_DEV raw enc(comp c) { return c; }
        static MG_DEV raw enc_finite(float f) { return f; }
    };
    struct SF64
    {
        using raw = double;
        using comp = double;
        static constexpr int dt = F64;
        static MG_DEV double dec(raw r) { return r; }
        static MG_DEV raw enc32(float f) { return double(f); }
        static MG_DEV raw enc64(double d) { return d; }
        static MG_DEV raw enc(comp c) { return c; }
    };

    // rnd(tanh(v)) for a stored value v, the step of apply_output_tail
    // (src/muse_glimmer.hpp:920-943) and of the score softcap: the short f64
    // evaluation of mg_tanh_fast.hpp, accepted when t(1 - m) and t(1 + m)
    // round to one stored value (FDLIBM's tanh, within that interval, rounds
    // to it too), else FDLIBM itself through an out-of-line call so the
    // unrolled per-key code that calls this stays small. NaN goes to FDLIBM.
    __attribute__((noinline)) static __device__ double tanh_fdlibm(double x)
    {
        return mgm::tanh(x);
    }
    template <class S>
    MG_DEV float tanh_stored(float v)
    {
        const double a = __builtin_fabs(double(v));
        if (a == a) {
            const double t = mgm::tanh_fast_abs(a);
            double tl, th;
            mgm::tanh_interval(t, tl, th);
            const auto lo = S::enc64(tl), hi = S::enc64(th);
            if (lo == hi) return __builtin_copysignf(S::dec(lo), v);
        }
        return S::dec(S::enc64(tanh_fdlibm(double(v))));
    }

    // --------------------------------------------------------- 16-byte vectors
    template <typename T, int N>
    struct alignas(sizeof(T) * N) Vec
    {
        T v[N];
    };
    template <typename T, int N>
    MG_DEV Vec<T, N> ld16(const T *p)
    {
        return *reinterpret_cast<const Vec<T, N> *>(p);
    }
    template <typename T, int N>
    MG_DEV void st16(T *p, const Vec<T, N> &v)
    {
        *reinterpret_cast<Vec<T, N> *>(p) = v;
    }
    // streaming variants: data touched once, keep it out of the caches' way
    template <typename T, int N>
    MG_DEV Vec<T, N> ld16_stream(const T *p)
    {
        using U = Vec<uint32_t, 4>;
        U u;
        const uint32_t *q = reinterpret_cast<const uint32_t *>(p);
#pragma unroll
        for (int i = 0; i < 4; ++i) u.v[i] = __builtin_nontemporal_load(q + i);
        return __builtin_bit_cast(Vec<T, N>, u);
    }
    template <typename T, int N>
    MG_DEV void st16_stream(T *p, const Vec<T, N> &v)
    {
        using U = Vec<uint32_t, 4>;
        const U u = __builtin_bit_cast(U, v);
        uint32_t *q = reinterpret_cast<uint32_t *>(p);
#pragma unroll
        for (int i = 0; i < 4; ++i) __builtin_nontemporal_store(u.v[i], q + i);
    }

    // Raw buffer accesses. A resource over [p, p + bytes): a 16-byte access
    // at a byte offset past the range reads zeros and writes nothing, without
    // touching memory, so a kernel can issue a fixed set of accesses with no
    // branch around them (and the compiler's wait counts stay exact). Word 3
    // is the gfx9 layout: 32-bit data format, no swizzle. AUX 2: non-temporal.
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    constexpr int kAuxNT = 2;
    MG_DEV __amdgpu_buffer_rsrc_t buf_rsrc(const void *p, int bytes)
    {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), short(0), bytes, 0x00020000);
    }
    template <class T, int N, int AUX>
    MG_DEV Vec<T, N> buf_ld16(__amdgpu_buffer_rsrc_t rs, int off)
    {
        const u32x4 u = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, AUX);
        Vec<uint32_t, 4> w;
        // (each element to a prvalue first: bit_cast of an ext_vector element
        // lvalue lowers to a read of element 0 in this compiler)
#pragma unroll
        for (int i = 0; i < 4; ++i) w.v[i] = uint32_t(u[i]);
        return __builtin_bit_cast(Vec<T, N>, w);
    }
    template <class T, int N, int AUX>
    MG_DEV void buf_st16(__amdgpu_buffer_rsrc_t rs, int off, const Vec<T, N> &v)
    {
        const Vec<uint32_t, 4> w = __builtin_bit_cast(Vec<uint32_t, 4>, v);
        u32x4 u;
#pragma unroll
        for (int i = 0; i < 4; ++i) u[i] = w.v[i];
        __builtin_amdgcn_raw_buffer_store_b128(u, rs, off, 0, AUX);
    }

    // N elements: one non-temporal 16-byte access when they fill 16 bytes,
    // plain element accesses otherwise (unaligned fallbacks)
    template <typename T, int N>
    MG_DEV Vec<T, N> ldv(const T *p)
    {
        if constexpr (sizeof(T) * N == 16)
            return ld16_stream<T, N>(p);
        else
            return *reinterpret_cast<const Vec<T, N> *>(p);
    }
    template <typename T, int N>
    MG_DEV void stv(T *p, const Vec<T, N> &v)
    {
        if constexpr (sizeof(T) * N == 16)
            st16_stream<T, N>(p, v);
        else
            *reinterpret_cast<Vec<T, N> *>(p) = v;
    }

    // RoPE rotate-half of one (lo, hi) pair (reference apply_rope,
    // src/muse_glimmer.hpp:681-705): x[j] = rnd(rnd(lo*c) + rnd(-hi*s)),
    // x[j+half] = rnd(rnd(hi*c) + rnd(lo*s)); for 16-bit and f32 storage the
    // products and sums of stored values in f32 equal the twin's f64 ones
    // rounded to storage, for f64 the plain f64 expression.
    template <class S>
    MG_DEV void rope_pair(typename S::raw &lo, typename S::raw &hi, typename S::raw c, typename S::raw s)
    {
        if (S::dt == F64) {
            const double l = double(S::dec(lo)), h = double(S::dec(hi));
            const double cc = double(S::dec(c)), ss = double(S::dec(s));
            lo = S::enc64(l * cc - h * ss);
            hi = S::enc64(h * cc + l * ss);
        } else {
            const float l = float(S::dec(lo)), h = float(S::dec(hi));
            const float cc = float(S::dec(c)), ss = float(S::dec(s));
            const float a = float(S::dec(S::enc32(l * cc))), b = float(S::dec(S::enc32(-(h * ss))));
            const float d = float(S::dec(S::enc32(h * cc))), e = float(S::dec(S::enc32(l * ss)));
            lo = S::enc32(a + b);
            hi = S::enc32(d + e);
        }
    }

    // ------------------------------------------------- packed 16-bit pairs
    // Two 16-bit values in one 32-bit word, element 0 in the low half: the
    // bf16 steps round two results with one v_cvt_pk_bf16_f32, and the
    // magnitude bounds take two halves per v_pk_max_u16 / v_pk_min_u16.
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    MG_DEV uint32_t pk_max_u16(uint32_t a, uint32_t b)
    {
        return __builtin_bit_cast(uint32_t,
                                  __builtin_elementwise_max(__builtin_bit_cast(u16x2, a), __builtin_bit_cast(u16x2, b)));
    }
    MG_DEV uint32_t pk_min_u16(uint32_t a, uint32_t b)
    {
        return __builtin_bit_cast(uint32_t,
                                  __builtin_elementwise_min(__builtin_bit_cast(u16x2, a), __builtin_bit_cast(u16x2, b)));
    }
    // each half minus one, modulo 2^16 (zero becomes 0xFFFF)
    MG_DEV uint32_t pk_dec_u16(uint32_t a)
    {
        return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, a) - u16x2{1, 1});
    }
    MG_DEV float bf_lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
    MG_DEV float bf_hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }
    // RNE of two f32 values into one word; a NaN stays a NaN of the
    // conversion's own pattern (bf_canon makes it 0x7FC0)
    MG_DEV uint32_t bf_pack(float a, float b)
    {
        typedef float f2 __attribute__((ext_vector_type(2)));
        typedef __bf16 h2 __attribute__((ext_vector_type(2)));
        const f2 v = {opaque(a), opaque(b)};
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, h2));
    }
    // RNE of one f32 value to bf16, returned as the f32 of the same value:
    // the conversion's high half with a zero low half, one instruction
    MG_DEV float bf_round(float x)
    {
        typedef float f2 __attribute__((ext_vector_type(2)));
        typedef __bf16 h2 __attribute__((ext_vector_type(2)));
        const f2 v = {0.0f, opaque(x)};
        return __builtin_bit_cast(float, __builtin_convertvector(v, h2));
    }
    MG_DEV uint32_t bf_canon(uint32_t w)
    {
        const uint32_t a = w & 0xffffu, b = w >> 16;
        return ((a & 0x7fffu) > 0x7f80u ? 0x7fc0u : a) | ((b & 0x7fffu) > 0x7f80u ? 0x7fc0u : b) << 16;
    }

    // -------------------------------------------------------- wave64 reductions
    template <typename T>
    MG_DEV T wave_sum(T v)
    {
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
        return v;
    }
    template <typename T>
    MG_DEV T wave_max(T v)
    {
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
            const T o = __shfl_xor(v, m, 64);
            v = o > v ? o : v;
        }
        return v;
    }

    // DPP wave64 reductions (all 64 lanes active): swap within quads, mirror
    // within half-rows and rows, then broadcast lane 15 of each row into the
    // next row and lane 31 into the upper half; lane 63 ends with the result
    // and readlane hands it to every lane as a uniform value. No LDS traffic,
    // and a fixed combination order, so floating-point results are
    // deterministic.
    template <int CTRL, int ROWS, int BANKS = 0xf>
    MG_DEV uint32_t dpp32(uint32_t old, uint32_t v)
    {
        return uint32_t(__builtin_amdgcn_update_dpp(int(old), int(v), CTRL, ROWS, BANKS, false));
    }
    // inclusive prefix sum over the lanes (all active): shifts by 1, 2, 3
    // within rows of 16, then 4 and 8 into the upper banks, then the row
    // broadcasts of lanes 15 and 31
    MG_DEV int wave_prefix_sum(int v)
    {
        const uint32_t u = uint32_t(v);
        uint32_t t = u;
        t += dpp32<0x111, 0xf>(0u, u);      // row_shr:1
        t += dpp32<0x112, 0xf>(0u, u);      // row_shr:2
        t += dpp32<0x113, 0xf>(0u, u);      // row_shr:3
        t += dpp32<0x114, 0xf, 0xe>(0u, t); // row_shr:4, banks 1-3
        t += dpp32<0x118, 0xf, 0xc>(0u, t); // row_shr:8, banks 2-3
        t += dpp32<0x142, 0xa>(0u, t);      // row_bcast:15 into rows 1, 3
        t += dpp32<0x143, 0xc>(0u, t);      // row_bcast:31 into rows 2, 3
        return int(t);
    }
    template <int CTRL, int ROWS, typename T>
    MG_DEV T dpp_mov(T old, T v)
    {
        if constexpr (sizeof(T) == 4) {
            return __builtin_bit_cast(T, dpp32<CTRL, ROWS>(__builtin_bit_cast(uint32_t, old), __builtin_bit_cast(uint32_t, v)));
        } else {
            using U2 = Vec<uint32_t, 2>;
            const U2 o = __builtin_bit_cast(U2, old), x = __builtin_bit_cast(U2, v);
            U2 r;
            r.v[0] = dpp32<CTRL, ROWS>(o.v[0], x.v[0]);
            r.v[1] = dpp32<CTRL, ROWS>(o.v[1], x.v[1]);
            return __builtin_bit_cast(T, r);
        }
    }
    template <typename T>
    MG_DEV T readlane63(T v)
    {
        if constexpr (sizeof(T) == 4) {
            return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
        } else {
            using U2 = Vec<int, 2>;
            U2 x = __builtin_bit_cast(U2, v);
            x.v[0] = __builtin_amdgcn_readlane(x.v[0], 63);
            x.v[1] = __builtin_amdgcn_readlane(x.v[1], 63);
            return __builtin_bit_cast(T, x);
        }
    }
    template <typename T, class OP>
    MG_DEV T dpp_reduce(T v, T id, OP op)
    {
        v = op(v, dpp_mov<0xB1, 0xf>(id, v));  // quad_perm [1,0,3,2]
        v = op(v, dpp_mov<0x4E, 0xf>(id, v));  // quad_perm [2,3,0,1]
        v = op(v, dpp_mov<0x141, 0xf>(id, v)); // row_half_mirror
        v = op(v, dpp_mov<0x140, 0xf>(id, v)); // row_mirror
        v = op(v, dpp_mov<0x142, 0xa>(id, v)); // row_bcast:15 into rows 1, 3
        v = op(v, dpp_mov<0x143, 0xc>(id, v)); // row_bcast:31 into rows 2, 3
        return readlane63(v);
    }
    MG_DEV float dpp_max(float v)
    {
        return dpp_reduce(v, -__builtin_huge_valf(), [](float a, float b) { return __builtin_fmaxf(a, b); });
    }
    MG_DEV double dpp_sum(double v)
    {
        return dpp_reduce(v, 0.0, [](double a, double b) { return a + b; });
    }
    MG_DEV float dpp_sum_f32(float v)
    {
        return dpp_reduce(v, 0.0f, [](float a, float b) { return a + b; });
    }
    MG_DEV uint32_t dpp_min_u32(uint32_t v)
    {
        return dpp_reduce(v, 0xffffffffu, [](uint32_t a, uint32_t b) { return a < b ? a : b; });
    }
    MG_DEV uint32_t dpp_max_u32(uint32_t v)
    {
        return dpp_reduce(v, 0u, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
    }
    // number of lanes for which p holds (uniform)
    MG_DEV int wave_count(bool p)
    {
        return __builtin_popcountll(__builtin_amdgcn_ballot_w64(p));
    }

    // LDS writes of one wave made visible to the same wave's later reads
    MG_DEV void wave_lds_sync()
    {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }

    // ------------------------------------------------------------ matrix cores
    // v_mfma_f32_16x16x32_bf16: lane l = 16c + n holds row n of A (column n of
    // B) and its k-elements 8c..8c+7; C lane l holds rows 4c..4c+3 of column n
    typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
    typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    typedef short i16x4 __attribute__((ext_vector_type(4)));

    MG_DEV f32x4 mfma_bf16(bf16x8 a, bf16x8 b, f32x4 c)
    {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
    MG_DEV bf16x8 ld_bf16x8(const uint16_t *p)
    {
        return __builtin_bit_cast(bf16x8, *reinterpret_cast<const Vec<uint32_t, 4> *>(p));
    }
    // ds_read_b64_tr_b16: within each 16-lane group, lane i receives element
    // i % 4 of the 8-byte pieces addressed by lanes 4j + i / 4, j = 0..3
    MG_DEV bf16x4 lds_read_tr(const uint16_t *p)
    {
        typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
        return __builtin_bit_cast(bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(p)));
    }

    // x combined with the value of lane ^ 16 (XOR16) or lane ^ 32 (XOR32) by a
    // commutative op, through v_permlane16_swap / v_permlane32_swap: with the
    // same register as both operands, the pair returned holds, in every lane,
    // its own value and its partner's (no LDS traffic)
    template <int XOR, class OP>
    MG_DEV float lane_pair(float x, OP op)
    {
        const uint32_t u = __builtin_bit_cast(uint32_t, x);
        if constexpr (XOR == 16) {
            const auto p = __builtin_amdgcn_permlane16_swap(u, u, false, false);
            return op(__builtin_bit_cast(float, uint32_t(p[0])), __builtin_bit_cast(float, uint32_t(p[1])));
        } else {
            static_assert(XOR == 32, "lane_pair: XOR 16 or 32");
            const auto p = __builtin_amdgcn_permlane32_swap(u, u, false, false);
            return op(__builtin_bit_cast(float, uint32_t(p[0])), __builtin_bit_cast(float, uint32_t(p[1])));
        }
    }
    // the max / sum over the four 16-lane rows (lanes n, n+16, n+32, n+48)
    MG_DEV float rows4_max(float x)
    {
        auto mx = [](float a, float b) { return __builtin_fmaxf(a, b); };
        return lane_pair<32>(lane_pair<16>(x, mx), mx);
    }
    MG_DEV float rows4_sum(float x)
    {
        auto add = [](float a, float b) { return a + b; };
        return lane_pair<32>(lane_pair<16>(x, add), add);
    }

    MG_DEV int lane_rank(uint64_t mask)
    {
        return int(__builtin_amdgcn_mbcnt_hi(uint32_t(mask >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(mask), 0u)));
    }

    // ---------------------------------------------------------------- f32 exp
    // e^(x + lo) for the f32 reductions, lo a small correction term (|lo| <=
    // ulp(x)/2): Cody–Waite reduction x = n·ln2 + r with the Cephes
    // two-constant split of ln2, r += lo, then 2^(r·log2 e) on the hardware exp2
    // (|r| <= ln2/2, so the f32 product adds < 2^-25 relative), scaled by 2^n.
    // Relative error ~1.5 ulp; underflows smoothly through subnormals to 0.
    MG_DEV float exp_f32(float x, float lo = 0.0f)
    {
        if (x < -104.0f) return 0.0f;
        x = x > 88.72f ? 88.72f : x;
        const float n = __builtin_rintf(x * 1.44269504088896341f);
        float r = __builtin_fmaf(-n, 0.693359375f, x);
        r = __builtin_fmaf(n, 2.12194440e-4f, r) + lo;
        return __builtin_ldexpf(__builtin_amdgcn_exp2f(r * 1.44269504088896341f), int(n));
    }
    // e^(s - m) with the subtraction made exact (Knuth's TwoSum: d + err = s - m
    // exactly), so scores far from the row max lose nothing to the f32 rounding
    // of s - m (up to 2^-19 absolute at |s| ~ 30, a softcapped score's range).
    MG_DEV float exp_diff(float s, float m)
    {
        const float d = s - m;
        const float bp = d - s;
        const float err = (s - (d - bp)) + (-m - bp);
        return exp_f32(d, err);
    }

    // order-preserving map of an f32 to u32 (larger float -> larger key)
    MG_DEV uint32_t f32_key(float f)
    {
        const uint32_t u = __builtin_bit_cast(uint32_t, f);
        return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    }
    MG_DEV float key_f32(uint32_t k)
    {
        return __builtin_bit_cast(float, (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
    }
} // namespace mg
