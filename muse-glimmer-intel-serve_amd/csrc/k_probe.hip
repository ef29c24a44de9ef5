// HBM stream probes: the access patterns of the primitives with no arithmetic,
// so each primitive's time can be read against what the same traffic costs on
// its own (a measurement aid; nothing in the reference corresponds to it).
//
//   kind 0  copy   b = a                        1 read, 1 write per word
//   kind 1  read   xor-fold of a (one word out)   1 read
//   kind 2  write  b = constant                 1 write
//   kind 3  2r2w   a = a + c, d = a' ^ c       2 reads, 2 writes (the
//                                               residual-add + norm shape)
//
// One 16-byte word per lane per step, non-temporal loads and stores (the
// primitives' own policy), a one-shot grid of 256-thread work-groups, one
// word per thread per operand (no loop), so the probe measures the memory
// system under the primitives' launch shape rather than a tuned copy.
// Three other forms of the copy show what the primitives' pattern is worth
// against the alternatives:
//   kind 4  copy with ordinary (cached) loads and stores, one word a thread
//   kind 5  copy, four words a thread (each wave on 4 contiguous KiB, its
//           four loads issued before its four stores)
//   kind 6  copy by a persistent grid of 2048 work-groups, grid-stride, two
//           words in flight a thread
#include "mg_device.hpp"
#include "mg_internal.hpp"

namespace mg
{
    using U4 = Vec<uint32_t, 4>;

    // one kernel per kind, so profiles tell the patterns apart
    template <int KIND>
    __global__ __launch_bounds__(256) void k_probe(uint32_t *__restrict__ a, uint32_t *__restrict__ b,
                                                   const uint32_t *__restrict__ c, uint32_t *__restrict__ d,
                                                   int64_t words)
    {
        const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
        if (i >= words) return;
        if constexpr (KIND == 0) {
            st16_stream<uint32_t, 4>(b + 4 * i, ld16_stream<uint32_t, 4>(a + 4 * i));
        } else if constexpr (KIND == 1) {
            const U4 v = ld16_stream<uint32_t, 4>(a + 4 * i);
            // never true for the probe's inputs: keeps the load live
            if ((v.v[0] ^ v.v[1] ^ v.v[2] ^ v.v[3]) == 0x9e3779b9u) b[0] = uint32_t(i);
        } else if constexpr (KIND == 2) {
            st16_stream<uint32_t, 4>(b + 4 * i, U4{{uint32_t(i), 1u, 2u, 3u}});
        } else if constexpr (KIND == 4) {
            *reinterpret_cast<U4 *>(b + 4 * i) = *reinterpret_cast<const U4 *>(a + 4 * i);
        } else {
            const U4 x = ld16_stream<uint32_t, 4>(a + 4 * i), y = ld16_stream<uint32_t, 4>(c + 4 * i);
            U4 s, t;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                s.v[e] = x.v[e] + y.v[e];
                t.v[e] = s.v[e] ^ y.v[e];
            }
            st16_stream<uint32_t, 4>(a + 4 * i, s);
            st16_stream<uint32_t, 4>(d + 4 * i, t);
        }
    }

    // kind 5: four words a thread, wave w of the grid on words 256 w .. 256 w + 255
    __global__ __launch_bounds__(256) void k_probe_4vec(const uint32_t *__restrict__ a, uint32_t *__restrict__ b,
                                                       int64_t words)
    {
        const int64_t base = (int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6)) * 256 + (threadIdx.x & 63);
        U4 t[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
            if (base + 64 * k < words) t[k] = ld16_stream<uint32_t, 4>(a + 4 * (base + 64 * k));
#pragma unroll
        for (int k = 0; k < 4; ++k)
            if (base + 64 * k < words) st16_stream<uint32_t, 4>(b + 4 * (base + 64 * k), t[k]);
    }

    // kind 6: a persistent grid, grid-stride, two words in flight a thread
    __global__ __launch_bounds__(256) void k_probe_persist(const uint32_t *__restrict__ a, uint32_t *__restrict__ b,
                                                          int64_t words)
    {
        const int64_t stride = int64_t(gridDim.x) * 256;
        for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < words; i += 2 * stride) {
            const U4 x = ld16_stream<uint32_t, 4>(a + 4 * i);
            const bool two = i + stride < words;
            U4 y{};
            if (two) y = ld16_stream<uint32_t, 4>(a + 4 * (i + stride));
            st16_stream<uint32_t, 4>(b + 4 * i, x);
            if (two) st16_stream<uint32_t, 4>(b + 4 * (i + stride), y);
        }
    }

    void launch_probe(mg_ctx *ctx, int kind, void *a, void *b, const void *c, void *d, int64_t bytes)
    {
        need(kind >= 0 && kind <= 6,
             "probe: kind must be 0 (copy), 1 (read), 2 (write), 3 (2r2w), 4 (cached copy), 5 (copy, four "
             "words a thread) or 6 (persistent copy)");
        need(bytes >= 0 && bytes % 16 == 0, "probe: bytes must be a multiple of 16");
        need(bytes / 16 / 256 < (int64_t(1) << 31), "probe: too many bytes");
        const bool need_a = kind != 2, need_b = kind != 3, need_cd = kind == 3;
        need((!need_a || (a && aligned16(a))) && (!need_b || (b && aligned16(b))) &&
                 (!need_cd || (c && d && aligned16(c) && aligned16(d))),
             "probe: NULL or misaligned buffer");
        if (bytes == 0) return;
        const int64_t words = bytes / 16;
        auto go = [&](auto kern) {
            hipLaunchKernelGGL(kern, dim3(unsigned((words + 255) / 256)), dim3(256), 0, ctx->stream,
                               static_cast<uint32_t *>(a), static_cast<uint32_t *>(b),
                               static_cast<const uint32_t *>(c), static_cast<uint32_t *>(d), words);
        };
        const auto *ua = static_cast<const uint32_t *>(a);
        auto *ub = static_cast<uint32_t *>(b);
        switch (kind) {
        case 0: go(k_probe<0>); break;
        case 1: go(k_probe<1>); break;
        case 2: go(k_probe<2>); break;
        case 3: go(k_probe<3>); break;
        case 4: go(k_probe<4>); break;
        case 5:
            hipLaunchKernelGGL(k_probe_4vec, dim3(unsigned((words + 1023) / 1024)), dim3(256), 0, ctx->stream, ua, ub,
                               words);
            break;
        default: {
            const int64_t g = (words + 255) / 256 < 2048 ? (words + 255) / 256 : 2048;
            hipLaunchKernelGGL(k_probe_persist, dim3(unsigned(g)), dim3(256), 0, ctx->stream, ua, ub, words);
            break;
        }
        }
        check_launch("k_probe");
    }
} // namespace mg
