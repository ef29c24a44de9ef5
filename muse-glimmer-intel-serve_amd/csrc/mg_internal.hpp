// Host-side internals of libmgprims: the context and the kernel launchers each
// kernel file provides. Launchers validate shapes before they launch and throw
// std::runtime_error; the C ABI turns that into -1 + mg_last_error().
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <stdexcept>
#include <cmath>
#include <string>

#include "mg_softcap_fast.hpp"

struct mg_ctx
{
    int device = 0;
    hipStream_t stream = nullptr; // where every call launches (NULL: the default stream)
    int num_cus = 256;
    // silu/sigmoid of every 16-bit input, as output bits:
    // [0] silu bf16, [1] sigmoid bf16, [2] silu f16, [3] sigmoid f16 (65536 each)
    uint16_t *lut = nullptr;
    void *work = nullptr; // reduction partials (softmax split rows, vocab chunks)
    int64_t work_bytes = 0;
    hipEvent_t handoff = nullptr; // orders a new stream after the old one (mg_set_stream)
};

namespace mg
{
    [[noreturn]] inline void fail(const std::string &m) { throw std::runtime_error(m); }
    inline void check(hipError_t e, const char *what)
    {
        if (e != hipSuccess) fail(std::string(what) + ": " + hipGetErrorString(e));
    }
    inline void check_launch(const char *what) { check(hipGetLastError(), what); }
    inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
    using mgm::recip_rn; // RN(1 / c), mg_softcap_fast.hpp (shared with its host checker)
    inline int dt_size(int dt)
    {
        switch (dt) {
        case 0: return 8;
        case 1: case 2: return 2;
        case 3: return 4;
        default: fail("unknown dtype " + std::to_string(dt));
        }
    }
    inline void need(bool ok, const std::string &m)
    {
        if (!ok) fail(m);
    }

    // lookup tables, built at mg_open (k_elementwise.hip)
    void build_luts(mg_ctx *c);

    // k_norm.hip
    void launch_norm(mg_ctx *c, int kind, void *h, const void *x, int64_t ldh, int64_t ldx,
                     const void *w, double eps, void *y, int64_t ldy, int64_t rows, int64_t dim,
                     int dt);
    void launch_norm_mixed(mg_ctx *c, int kind, const void *x, int64_t ldx, int dtx, const void *w, int dtw,
                           double eps, void *y, int64_t ldy, int dty, int64_t rows, int64_t dim);
    // k_elementwise.hip
    void launch_residual_add(mg_ctx *c, void *h, const void *x, int64_t n, int dt);
    void launch_swiglu(mg_ctx *c, const void *g, const void *u, void *out, int64_t n, int dt,
                       bool sigmoid_gate);
    void launch_scale(mg_ctx *c, void *x, int64_t n, double s, int dt);
    void launch_softcap(mg_ctx *c, void *z, int64_t n, double mult, double cap, int dt);
    // k_rope.hip
    void launch_rope_table(mg_ctx *c, double theta, int64_t dim, int64_t T, int dt, void *co,
                           void *si);
    void launch_qk_norm_rope(mg_ctx *c, void *q, int64_t nq, int64_t ldq, void *k, int64_t nkv, int64_t ldk,
                             int64_t T, int64_t D, double eps, double qk_scale, const void *co, const void *si,
                             int64_t table_rows, const int64_t *pos, int64_t pos0, const void *v, int64_t ldv,
                             void *kc, void *vc, int64_t slots, int dt);
    void launch_rope(mg_ctx *c, void *q, int64_t qh, int64_t ldq, void *k, int64_t kh,
                     int64_t ldk, int64_t tokens, int64_t dim, const void *co, const void *si,
                     int64_t table_rows, const int64_t *pos, int64_t pos0, int dt);
    // k_softmax.hip
    void launch_softmax(mg_ctx *c, const void *x, int64_t ldx, void *y, int64_t ldy, int64_t heads, int64_t q,
                        int64_t kc, double scale, int mask, int64_t window, int64_t q_pos0, double softcap,
                        int dt_in, int dt_out);
    // k_softmax64.hip (f64 scores: the pure f64 and the f32-compat chains)
    void launch_softmax_f64(mg_ctx *c, const void *x, int64_t ldx, void *y, int64_t ldy, int64_t rows, int64_t q,
                            int64_t kc, double scale, int mask, int64_t window, int64_t q_pos0, double softcap,
                            bool compat);
    // k_q8.hip
    void launch_dequant_q8_0(mg_ctx *c, const int8_t *qs, const uint16_t *d, void *out,
                             int64_t rows, int64_t in, int dt_out);
    // k_vocab.hip
    // mg_npy.cpp (host: .npy files to and from device tensors)
    void npy_info(const char *path, char *descr, int64_t *shape, int max_ndim, int *ndim);
    void npy_load(mg_ctx *c, const char *path, void *dst, int64_t n, int dt);
    void npy_save(mg_ctx *c, const char *path, const void *src, int dt, const int64_t *shape, int ndim);
    void npy_save_i64(mg_ctx *c, const char *path, const int64_t *src, int64_t n);
    // k_sample.hip
    void launch_sample_dist(mg_ctx *c, const int64_t *top_idx, const float *top_val, const int64_t *amax,
                            const int64_t *raw_amax, int64_t rows, int64_t K, double temperature, double top_p,
                            double min_p, int64_t *out_ids, float *out_p, int64_t *out_n);
    void launch_sample_rows(mg_ctx *c, const float *lg, int64_t ld, int64_t rows, int64_t V,
                            const int64_t *raw_amax, int64_t top_k, double temperature, double top_p, double min_p,
                            int64_t *out_ids, float *out_p, int64_t *out_n);
    void launch_quantize_q8_0(mg_ctx *c, const uint16_t *w, int64_t rows, int64_t in, int8_t *qs, uint16_t *d);
    void launch_gemv_q8_0(mg_ctx *c, const int8_t *qs, const uint16_t *d, const uint16_t *x, int64_t batch,
                          int64_t rows, int64_t in, int64_t ldx, float *y, int64_t ldy, bool blockdot);
    void launch_attn_prefill(mg_ctx *c, const uint16_t *q, int64_t ldq, const uint16_t *kc, const uint16_t *vc,
                             int64_t T, int64_t nq, int64_t nkv, int64_t D, int64_t slots, int64_t pos0,
                             int64_t window, double scaling, float *out, int64_t ldo);
    void launch_attn_decode(mg_ctx *c, const uint16_t *q, const uint16_t *kc, const uint16_t *vc, int64_t nq,
                            int64_t nkv, int64_t D, int64_t slots, int64_t qpos, int64_t window, double scaling,
                            float *out);
    void launch_vocab(mg_ctx *c, const void *logits, int64_t ld, int64_t rows, int64_t V, int dt_in, int64_t K,
                      double *lse, int64_t *amax, int64_t *top_idx, float *top_val, bool tail_on, double mult,
                      double cap, void *logits_out);
    // the vocab pass without a context: partials in a fixed device array of
    // kVocabScratchBytes (k_vocab.hip), on `stream` of the current device
    constexpr int64_t kVocabScratchBytes = int64_t(16) << 20;
    // HBM stream probes (k_probe.hip): kind 0 copy, 1 read, 2 write, 3 2r2w
    void launch_probe(mg_ctx *ctx, int kind, void *a, void *b, const void *c, void *d, int64_t bytes);
    void launch_vocab_noalloc(hipStream_t stream, const void *logits, int64_t ld, int64_t rows, int64_t V,
                              int dt_in, int64_t K, double *lse, int64_t *amax, int64_t *top_idx, float *top_val);
} // namespace mg
