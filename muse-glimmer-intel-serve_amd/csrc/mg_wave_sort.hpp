// Sorting networks over the words a wave holds in registers (gfx950): lane
// exchanges by DPP and v_permlane16/32_swap, no LDS traffic. Used by the
// vocab pass (csrc/k_vocab.hip) and the full-row sampler (csrc/k_sample.hip).
#pragma once

#include "mg_device.hpp"

namespace mg
{
    // ------------------------------------------------ wave bitonic networks
    // A 32-bit word and its copy from lane ^ J, in either order (the
    // compare-exchange below is symmetric in them). J = 1, 2: quad
    // permutes; J = 4: within each row of 16, rotations by 12 on the banks
    // whose lane bit 2 is clear and by 4 on the others; J = 8: rotation by 8;
    // J = 16, 32: v_permlane16_swap / v_permlane32_swap, whose two results hold
    // own and partner word in every lane. No LDS traffic.
    template <int J>
    MG_DEV void xor_pair(uint32_t v, uint32_t &a, uint32_t &b)
    {
        if constexpr (J == 1) {
            a = v;
            b = dpp32<0xB1, 0xf>(0u, v);
        } else if constexpr (J == 2) {
            a = v;
            b = dpp32<0x4E, 0xf>(0u, v);
        } else if constexpr (J == 4) {
            a = v;
            b = dpp32<0x124, 0xf, 0xa>(dpp32<0x12C, 0xf, 0x5>(0u, v), v);
        } else if constexpr (J == 8) {
            a = v;
            b = dpp32<0x128, 0xf>(0u, v);
        } else if constexpr (J == 16) {
            const auto q = __builtin_amdgcn_permlane16_swap(v, v, false, false);
            a = uint32_t(q[0]);
            b = uint32_t(q[1]);
        } else {
            static_assert(J == 32, "xor_pair: J in 1 .. 32");
            const auto q = __builtin_amdgcn_permlane32_swap(v, v, false, false);
            a = uint32_t(q[0]);
            b = uint32_t(q[1]);
        }
    }
    // compare-exchange of v with lane ^ J: the larger of the two if keep_max,
    // else the smaller (32- or 64-bit unsigned words)
    template <int J, typename T>
    MG_DEV T cx(T v, bool keep_max)
    {
        T a, b;
        if constexpr (sizeof(T) == 4) {
            xor_pair<J>(v, a, b);
        } else {
            uint32_t al, bl, ah, bh;
            xor_pair<J>(uint32_t(v), al, bl);
            xor_pair<J>(uint32_t(v >> 32), ah, bh);
            a = (uint64_t(ah) << 32) | al;
            b = (uint64_t(bh) << 32) | bl;
        }
        return (a > b) == keep_max ? a : b;
    }
    template <typename T>
    MG_DEV T cx_j(int j, T v, bool keep_max)
    {
        switch (j) {
        case 1: return cx<1>(v, keep_max);
        case 2: return cx<2>(v, keep_max);
        case 4: return cx<4>(v, keep_max);
        case 8: return cx<8>(v, keep_max);
        case 16: return cx<16>(v, keep_max);
        default: return cx<32>(v, keep_max);
        }
    }

    // Bitonic sort of the 64*R words a wave holds in a[0..R-1], slot 64*r +
    // lane in a[r], descending (DESC) or ascending. Runs of the network ascend
    // or descend by slot; partners 64 or more slots apart sit in the same
    // lane. TOP64 (descending only): only the largest 64 are wanted, in a[0],
    // sorted: the last merge stage, after its cross-register step, sorts a[0]
    // alone.
    template <typename T, int R, bool DESC, bool TOP64 = false>
    MG_DEV void wave_bitonic(T (&a)[R])
    {
        static_assert(DESC || !TOP64, "wave_bitonic: TOP64 sorts descending");
        const int lane = threadIdx.x & 63;
        constexpr int N = 64 * R;
#pragma unroll
        for (int k = 2; k <= N; k <<= 1) {
#pragma unroll
            for (int j = k >> 1; j > 0; j >>= 1) {
                if (j >= 64) {
                    const int rj = j / 64;
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const int p = r ^ rj;
                        if (p > r) {
                            const bool desc = (((64 * r) & k) == 0) == DESC;
                            const T x = a[r], y = a[p];
                            const bool sw = desc ? (x < y) : (x > y);
                            a[r] = sw ? y : x;
                            a[p] = sw ? x : y;
                        }
                    }
                } else {
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        if (TOP64 && k == N && N > 64 && r > 0) continue;
                        const bool desc = (((64 * r + lane) & k) == 0) == DESC;
                        a[r] = cx_j<T>(j, a[r], ((lane & j) == 0) == desc);
                    }
                }
            }
        }
    }
    template <typename T, int R, bool TOP64 = false>
    MG_DEV void wave_bitonic_desc(T (&a)[R])
    {
        wave_bitonic<T, R, true, TOP64>(a);
    }

    // top: the 64 largest of two sorted runs, a (descending) and b
    // (ascending): their slot-wise maxima form a bitonic sequence holding the
    // 64 largest, which the half-cleaners sort (descending)
    MG_DEV uint64_t top64_merge(uint64_t a, uint64_t b)
    {
        const int lane = threadIdx.x & 63;
        uint64_t v = a > b ? a : b;
#pragma unroll
        for (int j = 32; j > 0; j >>= 1) v = cx_j<uint64_t>(j, v, (lane & j) == 0);
        return v;
    }

    // Bitonic merge of a bitonic sequence of the 64*R words a wave holds
    // (slot 64*r + lane in a[r]) into order, descending if desc: the
    // half-cleaners of strides 32*R .. 1 (the last stage of wave_bitonic)
    template <typename T, int R>
    MG_DEV void wave_bitonic_merge(T (&a)[R], bool desc)
    {
        const int lane = threadIdx.x & 63;
#pragma unroll
        for (int j = 32 * R; j > 0; j >>= 1) {
            if (j >= 64) {
                const int rj = j / 64;
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const int p = r ^ rj;
                    if (p > r) {
                        const T x = a[r], y = a[p];
                        const bool sw = desc ? (x < y) : (x > y);
                        a[r] = sw ? y : x;
                        a[p] = sw ? x : y;
                    }
                }
            } else {
#pragma unroll
                for (int r = 0; r < R; ++r) a[r] = cx_j<T>(j, a[r], ((lane & j) == 0) == desc);
            }
        }
    }
} // namespace mg
