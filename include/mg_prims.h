/* mg_prims.h — C ABI of the MI355X (gfx950) non-GEMM tensor primitives.
 *
 * One library (libmgprims.so), HIP kernels only; no CPU fallback. Conventions
 * follow the reference's C ABI over its GPU engine (src/gpu/c_api.cpp):
 *   - an opaque context created once; every device buffer the library needs
 *     (lookup tables, reduction partials) is allocated in mg_open, and no entry
 *     point allocates device memory afterwards (c_api.cpp:9-14);
 *   - no exception crosses the boundary: every entry point returns 0 on success
 *     and -1 on failure, with the message readable from mg_last_error() on the
 *     same thread (c_api.cpp:15-17, 170-188);
 *   - a context is not thread-safe; calls are asynchronous on the context's
 *     stream, and mg_sync() waits for them;
 *   - a call runs on its context's device (mg_vocab_reduce_noalloc: on its
 *     stream's) and leaves the calling thread's current HIP device as it was;
 *   - all tensor pointers are DEVICE pointers, row-major and contiguous unless
 *     a leading dimension argument says otherwise; counts are int64.
 *
 * Storage dtypes (the reference's prec::Dtype order, src/rounding.hpp:31-36,
 * plus f32): bf16 and f16 travel as their 16-bit patterns.
 *
 * Numerics: each op's result is the reference's f64 oracle / bf16-f16 twin
 * value (src/muse_glimmer.hpp) rounded to the output dtype through
 * f64 -> f32 -> storage RNE (src/rounding.hpp:64-166). Elementwise ops are
 * bit-exact against the twin; norms use f64 internals; the softmax and vocab
 * reductions compute in f32 with f64 merges. */
#ifndef MG_PRIMS_H
#define MG_PRIMS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mg_ctx mg_ctx;

enum mg_dtype { MG_F64 = 0, MG_BF16 = 1, MG_F16 = 2, MG_F32 = 3 };

/* An output format of mg_norm_rows_mixed only: f32 words holding bf16 values
 * (the value rounded f64 -> f32 -> bf16, then widened), the layout of
 * bf16exec's norm_rows_f32 (src/bf16exec.hpp:422-442) and of the GPU engine's
 * k_rmsnorm_f32 (src/gpu/gpu_engine.cpp:392-415), the embedding norm. */
enum { MG_BF16_AS_F32 = 4 };

/* Flag OR-ed into a dtype argument, together with MG_F64 only: the reference's
 * --hf-f32-compat mode (src/main.cpp:164-165; f64 runs only,
 * src/muse_glimmer.hpp:951-955), which places stock HF's f32 upcasts inside an
 * f64 run, bit for bit. Taken by mg_rmsnorm_rows, mg_residual_rmsnorm and
 * mg_qk_norm_rope (rmsnorm_rows's f32 chain with mean_sq_f32,
 * src/muse_glimmer.hpp:530-556, 581-594; 799-803 for the QK-norm), by
 * mg_rope_table (the f32 inverse-frequency chain stored as double(float(v)),
 * 634-657) and by mg_softmax_rows as dtype_in (the f32 softmax, 856-870). */
enum { MG_F32_COMPAT = 0x100 };

/* muse::NormKind (src/muse_glimmer.hpp:558-563) */
enum mg_norm_kind { MG_NORM_CENTERED = 0, MG_NORM_PLAIN = 1, MG_NORM_WEIGHTLESS = 2 };

/* mask of a [heads, q, k] score block; qpos = q_pos0 + row.
 * causal: key j visible iff j <= qpos; window: qpos - window < j <= qpos
 * (src/muse_glimmer.hpp:838-843, the sliding-window rule); biwindow: the
 * drafter's bidirectional window, qpos - window <= j <= qpos + window
 * (src/dflash.hpp:339-344). */
enum mg_mask { MG_MASK_NONE = 0, MG_MASK_CAUSAL = 1, MG_MASK_WINDOW = 2, MG_MASK_BIWINDOW = 3 };

/* Thread-local message of the last failing call on this thread
 * (muse_last_error, src/gpu/c_api.cpp:35, 170-188). */
const char *mg_last_error(void);

/* Create a context on HIP device `device`. `stream` is the hipStream_t every
 * call launches on; NULL is the device's default (null) stream.
 * `workspace_bytes` sizes the reduction-partials buffer (0 = 64 MiB); calls
 * whose partials would not fit fail with an error instead of allocating.
 * (muse_open, src/gpu/c_api.cpp:88-168) */
int mg_open(int device, void *stream, int64_t workspace_bytes, mg_ctx **out);
/* Wait for the context's stream, then free the context (always, also when the
 * wait fails); -1 reports the first failure, e.g. an error of earlier work.
 * (muse_close, src/gpu/c_api.cpp:163-166) */
int mg_close(mg_ctx *ctx);
/* Wait for all work queued on the context's stream. */
int mg_sync(mg_ctx *ctx);
/* Point the context at another stream (hipStream_t; NULL = the default stream).
 * The new stream first waits (on the device, through an event) for the work
 * already queued on the old one, since both use the context's workspace. */
int mg_set_stream(mg_ctx *ctx, void *stream);
void *mg_get_stream(mg_ctx *ctx);

/* y[r,:] = norm(x[r,:]) — replaces muse::rmsnorm_rows (src/muse_glimmer.hpp:572-608)
 * and bf16exec norm_rows (src/bf16exec.hpp:398-421); GPU k_rmsnorm_auto
 * (src/gpu/gpu_engine.cpp:285-390). Centered: x*rs*(1+w); Plain: x*rs*w;
 * Weightless: x*rs (w may be NULL); rs = 1/sqrt(mean(x^2)+eps), f64 internals,
 * one rounding to `dtype`. MG_F64 | MG_F32_COMPAT: the reference's f32 chain
 * (mean_sq_f32, rs = 1.0f/sqrtf(ms + float(eps)), f32 products, y = double(v)).
 * ldx/ldy: row strides in elements (0 = dim). In place (y == x) is allowed. */
int mg_rmsnorm_rows(mg_ctx *ctx, int kind, const void *x, int64_t ldx, const void *w,
                    double eps, void *y, int64_t ldy, int64_t rows, int64_t dim, int dtype);

/* The same norm with each operand at its own storage format — the bf16exec
 * candidate's norm_rows (src/bf16exec.hpp:398-421: x f32 rows, w bf16, y bf16):
 * f64 internals, one rounding to y_dtype. y_dtype MG_BF16_AS_F32 is its
 * norm_rows_f32 (422-442; the embedding norm, 469, and the GPU engine's
 * k_rmsnorm_f32, src/gpu/gpu_engine.cpp:392-415, 4283): y f32 holding the
 * bf16-rounded values, in place on f32 rows allowed, and, as there, the
 * weight applied for MG_NORM_PLAIN only (a Centered call is weight-less,
 * 437-438). The sum of squares runs in a fixed parallel order, not bf16exec's
 * sequential one (within 1e-16 relative). ldx/ldy: row strides in elements
 * (0 = dim); in place only with one element size and one stride. */
int mg_norm_rows_mixed(mg_ctx *ctx, int kind, const void *x, int64_t ldx, int x_dtype, const void *w, int w_dtype,
                       double eps, void *y, int64_t ldy, int y_dtype, int64_t rows, int64_t dim);

/* Fused residual add + norm: h[r,:] = rnd(h[r,:] + x[r,:]) (updated in place),
 * then y[r,:] = norm(h[r,:]). Replaces the residual loop
 * (src/muse_glimmer.hpp:1023-1024, 1048-1049; src/bf16exec.hpp:608-610, 641-643;
 * GPU k_residual src/gpu/gpu_engine.cpp:1886-1893) followed by the next
 * rmsnorm_rows call on the updated stream (src/muse_glimmer.hpp:1028-1031).
 * ldh/ldx/ldy: row strides in elements (0 = dim). */
int mg_residual_rmsnorm(mg_ctx *ctx, int kind, void *h, int64_t ldh, const void *x, int64_t ldx, const void *w,
                        double eps, void *y, int64_t ldy, int64_t rows, int64_t dim, int dtype);

/* h = rnd(h + x), elementwise (src/muse_glimmer.hpp:1023-1024). */
int mg_residual_add(mg_ctx *ctx, void *h, const void *x, int64_t n, int dtype);

/* out = rnd(rnd(silu(gate)) * up) — the SwiGLU loop (src/muse_glimmer.hpp:1036-1039;
 * src/bf16exec.hpp:626-631; GPU k_swiglu src/gpu/gpu_engine.cpp:1895-1904).
 * silu is the twin's f64 FDLIBM form (src/muse_glimmer.hpp:493). */
int mg_swiglu(mg_ctx *ctx, const void *gate, const void *up, void *out, int64_t n, int dtype);

/* out = rnd(pv * rnd(sigmoid(gate))) — attention output gate
 * (src/muse_glimmer.hpp:896-906; GPU k_out_gate src/gpu/gpu_engine.cpp:1873-1883). */
int mg_sigmoid_gate(mg_ctx *ctx, const void *pv, const void *gate, void *out, int64_t n,
                    int dtype);

/* x = rnd(x * s), s taken as an f32 opmath scalar for bf16/f16/f32 — the q-only
 * qk_scale (src/muse_glimmer.hpp:803-807; GPU k_scale_bf16 gpu_engine.cpp:433-440). */
int mg_scale(mg_ctx *ctx, void *x, int64_t n, double s, int dtype);

/* RoPE table [positions, head_dim/2] of cos and sin, stored at `dtype` —
 * muse::build_rope_table (src/muse_glimmer.hpp:625-674): f32 inverse-frequency
 * chain for bf16/f16/f32, f64 chain for f64; FDLIBM pow/cos/sin on the device.
 * MG_F64 | MG_F32_COMPAT: the f32 chain, entries stored as double(float(v)). */
int mg_rope_table(mg_ctx *ctx, double theta, int64_t head_dim, int64_t positions, int dtype,
                  void *cos_out, void *sin_out);

/* Rotate-half RoPE in place on q [tokens, q_heads, head_dim] and (optionally,
 * k may be NULL) k [tokens, k_heads, head_dim]; token t uses table row
 * positions[t] (device int64 array) or, when positions is NULL, pos0 + t.
 * Row strides between tokens: ldq/ldk elements (0 = heads*head_dim).
 * Replaces muse::apply_rope over (t, head) (src/muse_glimmer.hpp:681-705, 809-819)
 * and GPU k_rope (src/gpu/gpu_engine.cpp:444-476). `table_rows` bounds positions. */
int mg_rope(mg_ctx *ctx, void *q, int64_t q_heads, int64_t ldq, void *k, int64_t k_heads,
            int64_t ldk, int64_t tokens, int64_t head_dim, const void *cos_t, const void *sin_t,
            int64_t table_rows, const int64_t *positions, int64_t pos0, int dtype);

/* The caller sequence around RoPE in one pass (src/muse_glimmer.hpp:799-819;
 * GPU src/gpu/gpu_engine.cpp:4339-4350 and k_kv_append 481-492), in place on
 * q [tokens, q_heads, head_dim] and k [tokens, k_heads, head_dim]:
 *   weight-less RMSNorm of every head row over head_dim (eps),
 *   q = rnd(q * qk_scale) (q only; qk_scale taken as an f32 value outside f64),
 *   rotate-half RoPE with table row positions[t] or pos0 + t, when cos_t/sin_t
 *   are given (NULL for NoPE layers; rows outside the table stay unrotated),
 *   and, when k_cache is given, k_cache[p % cache_slots, g, :] = k and (with
 *   v/v_cache) v_cache[p % cache_slots, g, :] = v for token position p >= 0;
 *   the caches are [cache_slots, k_heads, head_dim] (the ring of k_kv_append);
 *   two tokens of one call that map to one slot race, as in the reference.
 * Each step rounds to `dtype` exactly as mg_rmsnorm_rows, mg_scale and mg_rope
 * do, so the result is bit-identical to running them in sequence
 * (MG_F64 | MG_F32_COMPAT: the QK-norm takes the f32 chain, 801-803).
 * ldq/ldk/ldv: token strides in elements (0 = heads*head_dim). */
int mg_qk_norm_rope(mg_ctx *ctx, void *q, int64_t q_heads, int64_t ldq, void *k, int64_t k_heads,
                    int64_t ldk, int64_t tokens, int64_t head_dim, double eps, double qk_scale,
                    const void *cos_t, const void *sin_t, int64_t table_rows, const int64_t *positions,
                    int64_t pos0, const void *v, int64_t ldv, void *k_cache, void *v_cache,
                    int64_t cache_slots, int dtype);

/* Scaled, masked row softmax over a [heads, q, k] score block — the
 * softmax of attention_forward (src/muse_glimmer.hpp:828-885) as a row operator:
 * s = x*scale (f32 opmath), optional tanh softcap s = cap*tanh(s/cap) in
 * apply_output_tail's op order (src/muse_glimmer.hpp:920-943; cap 0 = off),
 * masked keys get probability exactly 0, p = exp(s - max)/sum.
 * dtype_in: f32, bf16 or f16 scores; dtype_out: bf16, f16 or f32 probs.
 * f64 scores (dtype_in MG_F64, dtype_out MG_F64): the twin's f64 softmax
 * (845-848, 871-880), scale and softcap in f64, the sum in a fixed parallel
 * order (within 1e-12 relative of the ascending loop). dtype_in
 * MG_F64 | MG_F32_COMPAT: the f32 softmax of 856-870 bit for bit (f32 max,
 * float(exp(double(float(s) - m))), the f32 sum in ascending key order,
 * double(float(e) / sum)); no softcap.
 * Rows longer than one work-group's registers are split across work-groups
 * and merged in chunk order (the k_attn_decode_combine rule,
 * src/gpu/gpu_engine.cpp:1816-1857). Row r of the block (r = head * q_rows +
 * query) starts at x + r * ldx and y + r * ldy; ldx/ldy are row strides in
 * elements (0 = k_cols, the contiguous block). */
int mg_softmax_rows(mg_ctx *ctx, const void *x, int64_t ldx, void *y, int64_t ldy, int64_t heads, int64_t q_rows,
                    int64_t k_cols, double scale, int mask, int64_t window, int64_t q_pos0,
                    double softcap, int dtype_in, int dtype_out);

/* Output tail z = rnd(z*mult); z = rnd(cap*rnd(tanh(rnd(z/cap)))) in place
 * (muse::apply_output_tail src/muse_glimmer.hpp:920-943; GPU k_softcap
 * src/gpu/gpu_engine.cpp:1906-1919). mult 1 / cap 0 skip their steps. */
int mg_softcap(mg_ctx *ctx, void *z, int64_t n, double mult, double cap, int dtype);

/* Q8_0 dequantize: out[r,i] = rnd(f32(qs[r,i]) * f32(d[r,i/32])) with the
 * reference's separate-arrays layout (QW, src/gpu/gpu_engine.cpp:120-141):
 * qs int8 [rows, in], d f16 bits [rows, in/32]; `in` must be a multiple of 32.
 * Replaces k_dequant_q8 (src/gpu/gpu_engine.cpp:1117-1171). dtype_out bf16/f16/f32. */
int mg_dequant_q8_0(mg_ctx *ctx, const int8_t *qs, const uint16_t *d, void *out, int64_t rows,
                    int64_t in, int dtype_out);

/* Prefill attention over the KV ring — the GPU engine's --flash-prefill tier
 * (attention_flash with k_flash_softmax and k_flash_finish,
 * src/gpu/gpu_engine.cpp:3292-3372, 1481-1560): q bf16 [tokens, q_heads,
 * head_dim] (token stride ldq, 0 = q_heads*head_dim) after QK-norm, scale and
 * RoPE; row t, at position pos0 + t, attends keys lo_t..pos0 + t (lo_t =
 * window > 0 ? max(0, pos0 + t - window + 1) : 0) of the caches bf16
 * [cache_slots, kv_heads, head_dim] (key j in slot j % cache_slots, all of
 * them appended before the call); query head h reads kv head
 * h / (q_heads / kv_heads). out f32 [tokens, q_heads, head_dim] (token stride
 * ldo, 0 = q_heads*head_dim). Tile-wise online softmax with bf16
 * probabilities in the p.v product, the reference tier's contract: a
 * numerical envelope, not bits. head_dim 64 or 128; any number of query heads
 * per kv head (groups of more than 8 are served by several work-groups). */
int mg_attn_prefill(mg_ctx *ctx, const uint16_t *q, int64_t ldq, const uint16_t *k_cache, const uint16_t *v_cache,
                    int64_t tokens, int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t cache_slots,
                    int64_t pos0, int64_t window, double scaling, float *out, int64_t ldo);

/* Decode attention, the softmax's caller at one query token — the GPU
 * engine's split-K flash decode (k_attn_decode_split + k_attn_decode_combine,
 * src/gpu/gpu_engine.cpp:1690-1857) over the KV ring of k_kv_append:
 * q bf16 [q_heads, head_dim] (after QK-norm, scale and RoPE), caches bf16
 * [cache_slots, kv_heads, head_dim] with key position j in slot j % cache_slots;
 * keys lo..q_pos, lo = window > 0 ? max(0, q_pos - window + 1) : 0 (at most
 * cache_slots of them); query head h reads kv head h / (q_heads / kv_heads).
 * out f32 [q_heads, head_dim] = softmax(q.k * scaling) v. head_dim 64 or 128;
 * any number of query heads per kv head (one wave serves up to 16). Like the
 * reference's split-K path, a
 * numerical envelope rather than bits (f32 online softmax, split merge). */
int mg_attn_decode(mg_ctx *ctx, const uint16_t *q, const uint16_t *k_cache, const uint16_t *v_cache, int64_t q_heads,
                   int64_t kv_heads, int64_t head_dim, int64_t cache_slots, int64_t q_pos, int64_t window,
                   double scaling, float *out);

/* Q8_0 quantizer, the step before dequant — up_w (src/gpu/gpu_engine.cpp:2722-2755,
 * llama.cpp's quantize_row_q8_0 rule): w bf16 bits [rows, in] (in % 32 == 0) ->
 * qs int8 [rows, in] and d f16 bits [rows, in/32]; per 32-block d = amax/127 in
 * f32 stored as f16 (RNE, subnormals kept), q = lround(x * (d ? 1/d : 0)). */
int mg_quantize_q8_0(mg_ctx *ctx, const uint16_t *w, int64_t rows, int64_t in, int8_t *qs, uint16_t *d);

/* Q8_0 GEMV, the step after — k_gemv_q8 (src/gpu/gpu_engine.cpp:815-889):
 * y[b, o] = sum_i w[o, i] * x[b, i] for b < batch (1..8), x bf16 bits
 * [batch, in] (row stride ldx, 0 = in), y f32 [batch, rows] (row stride ldy,
 * 0 = rows). blockdot = 0: every weight is bf16(q * d) first (the engine's
 * default, consistent with a prefill that dequantizes); blockdot = 1:
 * sum over blocks of d * sum(q * x) (llama.cpp's dot). f32 accumulation. */
int mg_gemv_q8_0(mg_ctx *ctx, const int8_t *qs, const uint16_t *d, const uint16_t *x, int64_t batch, int64_t rows,
                 int64_t in, int64_t ldx, float *y, int64_t ldy, int blockdot);

/* HBM stream probe: NO COUNTERPART in the reference; a measurement aid that
 * moves `bytes` (a multiple of 16) through the primitives' access pattern
 * (16-byte non-temporal loads and stores, one-shot grid) with no arithmetic:
 * kind 0 copies a to b; 1 reads a (b receives at most one word); 2 writes b;
 * 3 reads a and c and writes a = a + c and d = (a + c) ^ c, 32-bit words (the
 * residual-add + RMSNorm traffic shape); 4, 5 and 6 copy a to b in other forms
 * (ordinary cached accesses; four words a thread; a persistent grid-stride
 * loop) to compare the pattern against. Buffers 16-byte aligned. */
int mg_probe_stream(mg_ctx *ctx, int kind, void *a, void *b, const void *c, void *d, int64_t bytes);

/* Per row of logits [rows, V] (dtype_in f32 or bf16; row r at logits + r * ld,
 * ld the row stride in elements, 0 = V), one fused pass:
 *   lse[r]     = m + log(sum exp(x - m)) over finite entries, m their max
 *                (serve/sampler.py:168-171); -inf for a row with none
 *   argmax[r]  = first index of the maximum, the strict '>' scan from index 0
 *                (src/main.cpp:475-483; src/bf16exec.hpp:686-693)
 *   top_idx/top_val [rows, K] = the K largest by value, ties by lower index
 *                (src/main.cpp:604-615 and serve/sampler.py:84-89, whose tie
 *                order is unspecified; this one is total), 0 < K <= 256.
 * Any output pointer may be NULL to skip it (all device pointers). */
int mg_vocab_reduce(mg_ctx *ctx, const void *logits, int64_t ld, int64_t rows, int64_t V, int dtype_in,
                    int64_t K, double *lse, int64_t *argmax, int64_t *top_idx, float *top_val);

/* mg_vocab_reduce without a context, allocating nothing: NO COUNTERPART in the
 * reference. For callers that cannot allocate device memory or hold a context
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Same kernels and results as mg_vocab_reduce (dtype_in f32 or
 * bf16, 0 < K <= 256, ld the row stride (0 = V), any output pointer may be
 * NULL), launched on `stream` (hipStream_t; NULL = the default stream of the
 * current HIP device) on that stream's device, whose own copy of the array it
 * uses. The reduction partials live in a fixed 16 MiB device
 * array (one per GPU, held until the process ends; its address is looked up
 * once per device, which allocates nothing): a call needs
 * rows * ceil(V / 4096) * 2216 bytes of it, e.g. 64 rows x V = 201088 take
 * 7.1 MB, and a call needing more fails with an error before launching
 * anything. Every call on one GPU shares that array: calls that overlap on
 * one GPU (concurrent streams) race; serialize them. */
int mg_vocab_reduce_noalloc(void *stream, const void *logits, int64_t ld, int64_t rows, int64_t V, int dtype_in,
                            int64_t K, double *lse, int64_t *argmax, int64_t *top_idx, float *top_val);

/* The output tail fused into the vocab pass: every logit first becomes
 * apply_output_tail's value (z = rnd(z*mult); z = rnd(cap*rnd(tanh(rnd(z/cap)))),
 * rounded to dtype_in at each step, FDLIBM tanh; src/muse_glimmer.hpp:920-943,
 * GPU k_softcap src/gpu/gpu_engine.cpp:1906-1919), then lse / argmax / top-K are
 * taken over the transformed logits exactly as mg_vocab_reduce does; top_val
 * holds transformed values. logits_out (optional, contiguous [rows, V] at
 * dtype_in) receives the transformed logits; the input (row stride ld,
 * 0 = V) is not modified. */
int mg_vocab_reduce_tail(mg_ctx *ctx, const void *logits, int64_t ld, int64_t rows, int64_t V, int dtype_in,
                         double mult, double cap, int64_t K, double *lse, int64_t *argmax, int64_t *top_idx,
                         float *top_val, void *logits_out);

/* The sampler's final candidate distribution from a vocab pass's output
 * (serve/sampler.py:43-112, Sampler._transformed / dist after the logit edits):
 * top_idx/top_val [rows, K] sorted as mg_vocab_reduce writes them over the
 * edited logits (K = the sampler's top_k, 1..256; other top_k:
 * mg_sample_rows), argmax [rows] of the edited logits, raw_argmax [rows] of
 * the logits before the edits (NULL: argmax; serve/sampler.py:70-74 falls
 * back to np.argmax of the raw logits). Per row: no finite candidate (the
 * edited row has no finite value) gives the point mass on raw_argmax (the
 * reference's "masked" fallback); temperature <= 0 the point mass on argmax
 * (greedy); otherwise -inf candidates are dropped, probs = softmax(values),
 * top_p < 1 keeps the first searchsorted(cumsum, top_p)+1, min_p > 0 keeps
 * probs >= min_p*max(probs), and the kept candidates get softmax(values /
 * temperature). Writes cand_count[r] candidates, in order, to
 * cand_ids/cand_probs [rows, K]. Probabilities match the reference's numpy
 * float32 arithmetic to a few ulp (f32 exp, f64 sums); a cut whose cumulative
 * sum lies within that distance of top_p may fall one candidate apart. */
int mg_sample_dist(mg_ctx *ctx, const int64_t *top_idx, const float *top_val, const int64_t *argmax,
                   const int64_t *raw_argmax, int64_t rows, int64_t K, double temperature, double top_p, double min_p,
                   int64_t *cand_ids, float *cand_probs, int64_t *cand_count);

/* The same filter chain on full rows of edited logits, for any top_k
 * (serve/sampler.py:43-112 with top_k <= 0 keeping every token, 80-95):
 * logits f32 [rows, V] (row stride ld, 0 = V), raw_argmax [rows] as in
 * mg_sample_dist (NULL: the row's own argmax). Greedy takes np.argmax of the
 * edited row (first maximum, NaN counting as the largest). top_k in (0, V)
 * keeps the top_k largest finite-or-+inf values (ties by lower index), top_k
 * <= 0 every value > -inf. Candidates come out in value order (ties by
 * index) when top_k > 0 or top_p < 1, as the reference sorts them, else in
 * index order. cand_ids/cand_probs are [rows, V]; cand_count[r] is the
 * number written, or -1 for a row left to the host: one whose kept prefix in
 * value order (after the top_p and min_p cuts) exceeds 4096 candidates, or one
 * holding +inf (the reference's probabilities are NaN there and its draw
 * raises). Rows with value-order outputs and no top_k cut use the context's
 * workspace for per-slice counts and gathered keys when they fit it. */
int mg_sample_rows(mg_ctx *ctx, const float *logits, int64_t ld, int64_t rows, int64_t V, const int64_t *raw_argmax,
                   int64_t top_k, double temperature, double top_p, double min_p, int64_t *cand_ids,
                   float *cand_probs, int64_t *cand_count);

/* .npy files to and from device tensors — oracle::Tensor's I/O
 * (src/tensor.h:11-48, src/tensor.cpp:13-224), the format of the reference's
 * fixtures and of its --dump-hidden / --trace-dir dumps (src/main.cpp:55-76).
 * Synchronous: file I/O on the host, one copy on the context's stream, waited
 * for. mg_npy_info needs no context or GPU: the stored descr ('<f8', '<f4',
 * '<i8', '<i4', '|u1', ...) into descr (at least 16 bytes, NULL to skip) and
 * the shape into shape[0..*ndim) (at most max_ndim dimensions). */
int mg_npy_info(const char *path, char *descr, int64_t *shape, int max_ndim, int *ndim);

/* load_npy (tensor.cpp:91-224): version 1-3 headers, C order, '<f8', '<f4',
 * '<i8', '<i4' or '|u1' data, every value widened to f64 as there (u1 stays
 * 0..255), then stored to the device buffer dst at `dtype` (MG_F64, MG_F32,
 * MG_BF16, MG_F16) with the twin's rounding (prec::round_act,
 * src/rounding.hpp:64-166). n must equal the file's element count. */
int mg_npy_load(mg_ctx *ctx, const char *path, void *dst, int64_t n, int dtype);

/* save_npy (tensor.cpp:62-76): the device tensor src at `dtype`, widened to f64
 * (exact), written as '<f8' with shape[0..ndim), header padded to 64 bytes as
 * write_npy_header does (13-38). */
int mg_npy_save(mg_ctx *ctx, const char *path, const void *src, int dtype, const int64_t *shape, int ndim);

/* save_npy_i64 (tensor.cpp:78-89): n int64 device values as a 1-d '<i8' file. */
int mg_npy_save_i64(mg_ctx *ctx, const char *path, const int64_t *src, int64_t n);

#ifdef __cplusplus
}
#endif

#endif /* MG_PRIMS_H */
