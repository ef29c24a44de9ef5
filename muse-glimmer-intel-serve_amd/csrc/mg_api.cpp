// C ABI of libmgprims (include/mg_prims.h).
//
// The boundary follows the reference's C ABI over its GPU engine
// (src/gpu/c_api.cpp): no exception crosses it (each entry point catches and
// stores the message in a thread-local string read by mg_last_error,
// c_api.cpp:15-17, 35, 170-188) and nothing allocates device memory after
// mg_open returns (c_api.cpp:9-14): the lookup tables and the reduction
// workspace are allocated there, and a call whose partials would not fit the
// workspace fails instead of growing it. mg_vocab_reduce_noalloc takes no
// context and allocates nothing at all (its partials live in a fixed device
// array, k_vocab.hip).
#include "mg_prims.h"

#include "mg_internal.hpp"

#include <exception>
#include <string>

namespace
{
    thread_local std::string g_err;
    constexpr int64_t kDefaultWorkspace = int64_t(64) << 20;
}

namespace
{
    // The caller's current HIP device, put back when an entry point returns:
    // a call switches to its context's device (or its stream's) for its own
    // work and leaves the caller's choice as it found it.
    struct DeviceRestore
    {
        int dev = -1;
        DeviceRestore()
        {
            if (hipGetDevice(&dev) != hipSuccess) dev = -1;
        }
        ~DeviceRestore()
        {
            int now = -1;
            if (dev >= 0 && hipGetDevice(&now) == hipSuccess && now != dev) (void)hipSetDevice(dev);
        }
    };
}

// one shape for every entry point: BODY may return; a throw becomes FAIL
#define MG_GUARD(FAIL, BODY)                         \
    do {                                             \
        DeviceRestore restore_device_;               \
        g_err.clear();                               \
        try {                                        \
            BODY                                     \
        } catch (const std::exception &ex) {         \
            g_err = ex.what();                       \
            return FAIL;                             \
        } catch (...) {                              \
            g_err = "unknown error";                 \
            return FAIL;                             \
        }                                            \
    } while (0)

namespace
{
    mg_ctx *ctx_of(mg_ctx *c)
    {
        if (!c) mg::fail("NULL context");
        int cur = -1;
        mg::check(hipGetDevice(&cur), "hipGetDevice");
        if (cur != c->device) mg::check(hipSetDevice(c->device), "hipSetDevice");
        return c;
    }

    // Frees everything the context owns, whatever fails on the way; returns
    // the first failure (a failed wait reports an error of earlier work).
    hipError_t release(mg_ctx *c)
    {
        if (!c) return hipSuccess;
        hipError_t first = hipSuccess;
        auto note = [&](hipError_t e) {
            if (first == hipSuccess) first = e;
        };
        note(hipSetDevice(c->device));
        note(hipStreamSynchronize(c->stream));
        if (c->lut) note(hipFree(c->lut));
        if (c->work) note(hipFree(c->work));
        if (c->handoff) note(hipEventDestroy(c->handoff));
        delete c;
        return first;
    }
}

extern "C" {

const char *mg_last_error(void) { return g_err.c_str(); }

int mg_open(int device, void *stream, int64_t workspace_bytes, mg_ctx **out)
{
    MG_GUARD(-1, {
        if (!out) mg::fail("mg_open: NULL out pointer");
        *out = nullptr;
        int n = 0;
        mg::check(hipGetDeviceCount(&n), "hipGetDeviceCount");
        if (device < 0 || device >= n) mg::fail("mg_open: no HIP device " + std::to_string(device));
        mg_ctx *c = new mg_ctx();
        try {
            c->device = device;
            mg::check(hipSetDevice(device), "hipSetDevice");
            hipDeviceProp_t prop;
            mg::check(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
            c->num_cus = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
            c->stream = static_cast<hipStream_t>(stream);
            c->work_bytes = workspace_bytes > 0 ? workspace_bytes : kDefaultWorkspace;
            mg::check(hipMalloc(&c->work, size_t(c->work_bytes)), "hipMalloc(workspace)");
            mg::check(hipMalloc(reinterpret_cast<void **>(&c->lut), 4 * 65536 * sizeof(uint16_t)), "hipMalloc(lut)");
            mg::check(hipEventCreateWithFlags(&c->handoff, hipEventDisableTiming), "hipEventCreate");
            mg::build_luts(c);
            mg::check(hipStreamSynchronize(c->stream), "building lookup tables");
        } catch (...) {
            (void)release(c); // the original error is the one reported
            throw;
        }
        *out = c;
        return 0;
    });
}

int mg_close(mg_ctx *ctx)
{
    MG_GUARD(-1, {
        mg::check(release(ctx), "mg_close");
        return 0;
    });
}

int mg_sync(mg_ctx *ctx)
{
    MG_GUARD(-1, {
        mg::check(hipStreamSynchronize(ctx_of(ctx)->stream), "hipStreamSynchronize");
        return 0;
    });
}

// Work queued on the old stream may still use the context's workspace, which
// the next call on the new stream reuses: the new stream waits for the old
// one's queued work (an event, no host wait) before anything runs on it.
int mg_set_stream(mg_ctx *ctx, void *stream)
{
    MG_GUARD(-1, {
        mg_ctx *c = ctx_of(ctx);
        const hipStream_t next = static_cast<hipStream_t>(stream);
        if (next != c->stream) {
            mg::check(hipEventRecord(c->handoff, c->stream), "mg_set_stream: hipEventRecord");
            mg::check(hipStreamWaitEvent(next, c->handoff, 0), "mg_set_stream: hipStreamWaitEvent");
            c->stream = next;
        }
        return 0;
    });
}

void *mg_get_stream(mg_ctx *ctx) { return ctx ? static_cast<void *>(ctx->stream) : nullptr; }

int mg_rmsnorm_rows(mg_ctx *ctx, int kind, const void *x, int64_t ldx, const void *w, double eps,
                    void *y, int64_t ldy, int64_t rows, int64_t dim, int dtype)
{
    MG_GUARD(-1, {
        mg::launch_norm(ctx_of(ctx), kind, const_cast<void *>(x), nullptr, ldx ? ldx : dim, 0, w, eps, y,
                        ldy ? ldy : dim, rows, dim, dtype);
        return 0;
    });
}

int mg_norm_rows_mixed(mg_ctx *ctx, int kind, const void *x, int64_t ldx, int x_dtype, const void *w, int w_dtype,
                       double eps, void *y, int64_t ldy, int y_dtype, int64_t rows, int64_t dim)
{
    MG_GUARD(-1, {
        mg::launch_norm_mixed(ctx_of(ctx), kind, x, ldx, x_dtype, w, w_dtype, eps, y, ldy, y_dtype, rows, dim);
        return 0;
    });
}

int mg_residual_rmsnorm(mg_ctx *ctx, int kind, void *h, int64_t ldh, const void *x, int64_t ldx, const void *w,
                        double eps, void *y, int64_t ldy, int64_t rows, int64_t dim, int dtype)
{
    MG_GUARD(-1, {
        if (!x) mg::fail("residual_rmsnorm: NULL residual operand");
        mg::launch_norm(ctx_of(ctx), kind, h, x, ldh ? ldh : dim, ldx ? ldx : dim, w, eps, y, ldy ? ldy : dim, rows,
                        dim, dtype);
        return 0;
    });
}

int mg_residual_add(mg_ctx *ctx, void *h, const void *x, int64_t n, int dtype)
{
    MG_GUARD(-1, {
        mg::launch_residual_add(ctx_of(ctx), h, x, n, dtype);
        return 0;
    });
}

int mg_swiglu(mg_ctx *ctx, const void *gate, const void *up, void *out, int64_t n, int dtype)
{
    MG_GUARD(-1, {
        mg::launch_swiglu(ctx_of(ctx), gate, up, out, n, dtype, false);
        return 0;
    });
}

int mg_sigmoid_gate(mg_ctx *ctx, const void *pv, const void *gate, void *out, int64_t n, int dtype)
{
    MG_GUARD(-1, {
        mg::launch_swiglu(ctx_of(ctx), gate, pv, out, n, dtype, true);
        return 0;
    });
}

int mg_scale(mg_ctx *ctx, void *x, int64_t n, double s, int dtype)
{
    MG_GUARD(-1, {
        mg::launch_scale(ctx_of(ctx), x, n, s, dtype);
        return 0;
    });
}

int mg_rope_table(mg_ctx *ctx, double theta, int64_t head_dim, int64_t positions, int dtype,
                  void *cos_out, void *sin_out)
{
    MG_GUARD(-1, {
        mg::launch_rope_table(ctx_of(ctx), theta, head_dim, positions, dtype, cos_out, sin_out);
        return 0;
    });
}

int mg_rope(mg_ctx *ctx, void *q, int64_t q_heads, int64_t ldq, void *k, int64_t k_heads,
            int64_t ldk, int64_t tokens, int64_t head_dim, const void *cos_t, const void *sin_t,
            int64_t table_rows, const int64_t *positions, int64_t pos0, int dtype)
{
    MG_GUARD(-1, {
        if (!positions && (pos0 < 0 || pos0 + tokens > table_rows))
            mg::fail("rope: positions pos0..pos0+tokens-1 fall outside the table");
        mg::launch_rope(ctx_of(ctx), q, q_heads, ldq, k, k_heads, ldk, tokens, head_dim, cos_t, sin_t,
                        table_rows, positions, pos0, dtype);
        return 0;
    });
}

int mg_qk_norm_rope(mg_ctx *ctx, void *q, int64_t q_heads, int64_t ldq, void *k, int64_t k_heads,
                    int64_t ldk, int64_t tokens, int64_t head_dim, double eps, double qk_scale,
                    const void *cos_t, const void *sin_t, int64_t table_rows, const int64_t *positions,
                    int64_t pos0, const void *v, int64_t ldv, void *k_cache, void *v_cache,
                    int64_t cache_slots, int dtype)
{
    MG_GUARD(-1, {
        mg::launch_qk_norm_rope(ctx_of(ctx), q, q_heads, ldq, k, k_heads, ldk, tokens, head_dim, eps, qk_scale,
                                cos_t, sin_t, table_rows, positions, pos0, v, ldv, k_cache, v_cache,
                                cache_slots, dtype);
        return 0;
    });
}

int mg_softmax_rows(mg_ctx *ctx, const void *x, int64_t ldx, void *y, int64_t ldy, int64_t heads, int64_t q_rows,
                    int64_t k_cols, double scale, int mask, int64_t window, int64_t q_pos0,
                    double softcap, int dtype_in, int dtype_out)
{
    MG_GUARD(-1, {
        mg::launch_softmax(ctx_of(ctx), x, ldx, y, ldy, heads, q_rows, k_cols, scale, mask, window, q_pos0, softcap,
                           dtype_in, dtype_out);
        return 0;
    });
}

int mg_softcap(mg_ctx *ctx, void *z, int64_t n, double mult, double cap, int dtype)
{
    MG_GUARD(-1, {
        mg::launch_softcap(ctx_of(ctx), z, n, mult, cap, dtype);
        return 0;
    });
}

int mg_dequant_q8_0(mg_ctx *ctx, const int8_t *qs, const uint16_t *d, void *out, int64_t rows,
                    int64_t in, int dtype_out)
{
    MG_GUARD(-1, {
        mg::launch_dequant_q8_0(ctx_of(ctx), qs, d, out, rows, in, dtype_out);
        return 0;
    });
}

int mg_probe_stream(mg_ctx *ctx, int kind, void *a, void *b, const void *c, void *d, int64_t bytes)
{
    MG_GUARD(-1, {
        mg::launch_probe(ctx_of(ctx), kind, a, b, c, d, bytes);
        return 0;
    });
}

int mg_vocab_reduce(mg_ctx *ctx, const void *logits, int64_t ld, int64_t rows, int64_t V, int dtype_in,
                    int64_t K, double *lse, int64_t *argmax, int64_t *top_idx, float *top_val)
{
    MG_GUARD(-1, {
        mg::launch_vocab(ctx_of(ctx), logits, ld, rows, V, dtype_in, K, lse, argmax, top_idx, top_val, false, 1.0, 0.0,
                         nullptr);
        return 0;
    });
}

int mg_vocab_reduce_tail(mg_ctx *ctx, const void *logits, int64_t ld, int64_t rows, int64_t V, int dtype_in,
                         double mult, double cap, int64_t K, double *lse, int64_t *argmax, int64_t *top_idx,
                         float *top_val, void *logits_out)
{
    MG_GUARD(-1, {
        mg::launch_vocab(ctx_of(ctx), logits, ld, rows, V, dtype_in, K, lse, argmax, top_idx, top_val, true, mult, cap,
                         logits_out);
        return 0;
    });
}

int mg_vocab_reduce_noalloc(void *stream, const void *logits, int64_t ld, int64_t rows, int64_t V, int dtype_in,
                            int64_t K, double *lse, int64_t *argmax, int64_t *top_idx, float *top_val)
{
    MG_GUARD(-1, {
        mg::launch_vocab_noalloc(static_cast<hipStream_t>(stream), logits, ld, rows, V, dtype_in, K, lse, argmax,
                                 top_idx, top_val);
        return 0;
    });
}

int mg_sample_dist(mg_ctx *ctx, const int64_t *top_idx, const float *top_val, const int64_t *argmax,
                   const int64_t *raw_argmax, int64_t rows, int64_t K, double temperature, double top_p, double min_p,
                   int64_t *cand_ids, float *cand_probs, int64_t *cand_count)
{
    MG_GUARD(-1, {
        mg::launch_sample_dist(ctx_of(ctx), top_idx, top_val, argmax, raw_argmax, rows, K, temperature, top_p, min_p,
                               cand_ids, cand_probs, cand_count);
        return 0;
    });
}

int mg_sample_rows(mg_ctx *ctx, const float *logits, int64_t ld, int64_t rows, int64_t V, const int64_t *raw_argmax,
                   int64_t top_k, double temperature, double top_p, double min_p, int64_t *cand_ids,
                   float *cand_probs, int64_t *cand_count)
{
    MG_GUARD(-1, {
        mg::launch_sample_rows(ctx_of(ctx), logits, ld, rows, V, raw_argmax, top_k, temperature, top_p, min_p,
                               cand_ids, cand_probs, cand_count);
        return 0;
    });
}

int mg_npy_info(const char *path, char *descr, int64_t *shape, int max_ndim, int *ndim)
{
    MG_GUARD(-1, {
        mg::npy_info(path, descr, shape, max_ndim, ndim);
        return 0;
    });
}

int mg_npy_load(mg_ctx *ctx, const char *path, void *dst, int64_t n, int dtype)
{
    MG_GUARD(-1, {
        mg::npy_load(ctx_of(ctx), path, dst, n, dtype);
        return 0;
    });
}

int mg_npy_save(mg_ctx *ctx, const char *path, const void *src, int dtype, const int64_t *shape, int ndim)
{
    MG_GUARD(-1, {
        mg::npy_save(ctx_of(ctx), path, src, dtype, shape, ndim);
        return 0;
    });
}

int mg_npy_save_i64(mg_ctx *ctx, const char *path, const int64_t *src, int64_t n)
{
    MG_GUARD(-1, {
        mg::npy_save_i64(ctx_of(ctx), path, src, n);
        return 0;
    });
}

int mg_quantize_q8_0(mg_ctx *ctx, const uint16_t *w, int64_t rows, int64_t in, int8_t *qs, uint16_t *d)
{
    MG_GUARD(-1, {
        mg::launch_quantize_q8_0(ctx_of(ctx), w, rows, in, qs, d);
        return 0;
    });
}

int mg_gemv_q8_0(mg_ctx *ctx, const int8_t *qs, const uint16_t *d, const uint16_t *x, int64_t batch, int64_t rows,
                 int64_t in, int64_t ldx, float *y, int64_t ldy, int blockdot)
{
    MG_GUARD(-1, {
        mg::launch_gemv_q8_0(ctx_of(ctx), qs, d, x, batch, rows, in, ldx, y, ldy, blockdot != 0);
        return 0;
    });
}

int mg_attn_prefill(mg_ctx *ctx, const uint16_t *q, int64_t ldq, const uint16_t *k_cache, const uint16_t *v_cache,
                    int64_t tokens, int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t cache_slots,
                    int64_t pos0, int64_t window, double scaling, float *out, int64_t ldo)
{
    MG_GUARD(-1, {
        mg::launch_attn_prefill(ctx_of(ctx), q, ldq, k_cache, v_cache, tokens, q_heads, kv_heads, head_dim,
                                cache_slots, pos0, window, scaling, out, ldo);
        return 0;
    });
}

int mg_attn_decode(mg_ctx *ctx, const uint16_t *q, const uint16_t *k_cache, const uint16_t *v_cache, int64_t q_heads,
                   int64_t kv_heads, int64_t head_dim, int64_t cache_slots, int64_t q_pos, int64_t window,
                   double scaling, float *out)
{
    MG_GUARD(-1, {
        mg::launch_attn_decode(ctx_of(ctx), q, k_cache, v_cache, q_heads, kv_heads, head_dim, cache_slots, q_pos,
                               window, scaling, out);
        return 0;
    });
}

} // extern "C"
