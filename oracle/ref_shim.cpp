// ORACLE CHECKER — test infrastructure only; built into oracle/_ref/ from the
// reference's own headers where they lie under /root/reference/src (nothing is
// copied). It exports the reference functions that have no C entry point in
// the reference's own referee library (tools/oracle_kernels.cpp, built beside
// it): storage rounding, rmsnorm_rows, the RoPE table and its application, the
// output tail, the exact f16 decode, and the .npy writer and reader of
// src/tensor.cpp (compiled beside this file from where it lies). Used only to pin oracle/oracle.cpp
// (tests/golden/make_golden.py and the CPU tests).
#include <cstdint>
#include <exception>
#include <vector>

#include "bf16exec.hpp"
#include "muse_glimmer.hpp"
#include "rounding.hpp"
#include "safetensors.hpp"
#include "tensor.h"

extern "C"
{
    // prec::round_act (rounding.hpp:155-166); dt = 0 f64, 1 bf16, 2 f16
    void rs_round(int dt, const double *x, double *y, int64_t n)
    {
        for (int64_t i = 0; i < n; ++i)
            y[i] = prec::round_act(prec::Dtype(dt), x[i]);
    }

    // st::f16_to_f64 (safetensors.hpp:100-130)
    void rs_f16_to_f64(const uint16_t *h, double *y, int64_t n)
    {
        for (int64_t i = 0; i < n; ++i)
            y[i] = st::f16_to_f64(h[i]);
    }

    // bf16exec Engine::norm_rows (bf16exec.hpp:398-420): f32 rows, bf16 weights,
    // bf16 out; and Engine::norm_rows_f32 (422-442): the same rounding stored
    // back in f32, weight applied for Plain only. Neither reads engine state,
    // so a default-constructed engine serves.
    void rs_bf16exec_norm_rows(int kind, const float *X, const uint16_t *wt, double eps, uint16_t *out,
                               int64_t rows, int64_t dim)
    {
        const muse::bf16::Engine e{};
        e.norm_rows(muse::NormKind(kind), X, wt, eps, out, rows, dim);
    }
    void rs_bf16exec_norm_rows_f32(int kind, const float *X, const uint16_t *wt, double eps, float *out,
                                   int64_t rows, int64_t dim)
    {
        const muse::bf16::Engine e{};
        e.norm_rows_f32(muse::NormKind(kind), X, wt, eps, out, rows, dim);
    }

    // muse::rmsnorm_rows (muse_glimmer.hpp:572-608)
    void rs_rmsnorm_rows(int kind, const double *X, const double *w, double eps, double *Y,
                         int64_t rows, int64_t dim, int f32_compat, int dt)
    {
        muse::rmsnorm_rows(muse::NormKind(kind), X, w, eps, Y, rows, dim, f32_compat != 0,
                           prec::Dtype(dt));
    }

    // muse::build_rope_table (muse_glimmer.hpp:625-674)
    void rs_rope_table(double theta, int64_t head_dim, int64_t T, int f32_compat, int dt,
                       double *cos_out, double *sin_out)
    {
        muse::Config c;
        c.head_dim = head_dim;
        c.rope_theta = theta;
        muse::RopeTable rt = muse::build_rope_table(c, T, f32_compat != 0, prec::Dtype(dt));
        for (size_t i = 0; i < rt.cos.size(); ++i)
        {
            cos_out[i] = rt.cos[i];
            sin_out[i] = rt.sin[i];
        }
    }

    // muse::apply_rope (muse_glimmer.hpp:681-705) on one head vector at `pos`,
    // with a caller-supplied table of T rows
    void rs_apply_rope(double *x, int64_t head_dim, const double *cos_t, const double *sin_t,
                       int64_t T, int64_t pos, int dt)
    {
        muse::RopeTable rt;
        rt.dim = head_dim;
        rt.cos.assign(cos_t, cos_t + T * (head_dim / 2));
        rt.sin.assign(sin_t, sin_t + T * (head_dim / 2));
        muse::apply_rope(x, rt, pos, prec::Dtype(dt));
    }

    // oracle::save_npy (tensor.cpp:59-73): an f64 tensor of `ndim` dims
    int rs_save_npy_f64(const char *path, const double *data, const int64_t *shape, int ndim)
    {
        try {
            oracle::Tensor t(std::vector<int64_t>(shape, shape + ndim));
            for (size_t i = 0; i < t.data.size(); ++i) t.data[i] = data[i];
            oracle::save_npy(path, t);
            return 0;
        } catch (const std::exception &) {
            return -2;
        }
    }

    // oracle::save_npy_i64 (tensor.cpp:75-89)
    int rs_save_npy_i64(const char *path, const int64_t *data, int64_t n)
    {
        try {
            oracle::save_npy_i64(path, std::vector<int64_t>(data, data + n));
            return 0;
        } catch (const std::exception &) {
            return -2;
        }
    }

    // oracle::load_npy (tensor.cpp:91-222): the widened values into out[n];
    // -1 when n is not the file's element count, -2 when load_npy throws
    int rs_load_npy(const char *path, double *out, int64_t n)
    {
        try {
            const oracle::Tensor t = oracle::load_npy(path);
            if (t.numel() != n) return -1;
            for (int64_t i = 0; i < n; ++i) out[i] = t.data[size_t(i)];
            return 0;
        } catch (const std::exception &) {
            return -2;
        }
    }

    // muse::apply_output_tail (muse_glimmer.hpp:920-943)
    void rs_output_tail(double mult, double cap, double *z, int64_t n, int dt)
    {
        muse::Config c;
        c.output_multiplier = mult;
        c.final_logit_softcapping = cap;
        muse::apply_output_tail(c, z, n, prec::Dtype(dt));
    }
}
