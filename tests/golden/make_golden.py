"""Write the golden fixtures in this directory from the reference's own code.

    make -C oracle ref && python tests/golden/make_golden.py [part ...]

Every expected output below is computed by the reference's C++ sources,
compiled from /root/reference by oracle/Makefile into oracle/_ref:
tools/oracle_kernels.cpp (the reference's referee library: fmath exp/tanh/
sin/cos/pow, silu, sigmoid, the blocked-8 mean of squares) and
oracle/ref_shim.cpp over src/rounding.hpp, src/safetensors.hpp,
src/muse_glimmer.hpp (round_act, f16_to_f64, rmsnorm_rows, build_rope_table,
apply_rope, apply_output_tail; rmsnorm_rows and build_rope_table also in
their --hf-f32-compat branches) and src/bf16exec.hpp (norm_rows,
norm_rows_f32) and src/tensor.cpp (save_npy, save_npy_i64,
load_npy: the .npy files under npy/ and what the reference reads from numpy's). Inputs come from the oracle's portable seeded
generator (splitmix64 + Box-Muller), stored in the fixtures as well, so the
tests never regenerate them. Loops the reference writes inline (the residual
add, SwiGLU) are composed here from its round_act and ok_siluv exactly as
src/muse_glimmer.hpp:1023-1024 and 1036-1039 write them.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import oracle as O  # noqa: E402  (generator and storage conversions only)

R = O.Ref()
F64, BF16, F16, F32 = O.F64, O.BF16, O.F16, O.F32


def save(name, **arrays):
    np.savez_compressed(os.path.join(HERE, name), **arrays)
    print("wrote", name, sum(a.nbytes for a in arrays.values()), "bytes (uncompressed)")


def rounding():
    # crafted f64 values: ties and near-ties of the f32 and bf16/f16 grids,
    # f16 subnormal/overflow boundaries, specials
    rng = np.random.default_rng(7)
    base = rng.normal(0, 1, 2000) * np.exp2(rng.integers(-30, 30, 2000))
    f32 = base.astype(np.float32)
    u = f32.view(np.uint32)
    bf_mid = ((u & 0xffff0000) | 0x8000).view(np.float32).astype(np.float64)   # bf16 ties
    f16_mid = ((u & 0xffffe000) | 0x1000).view(np.float32).astype(np.float64)  # f16 ties
    nudge = np.concatenate([bf_mid * (1 + 2.0**-40), bf_mid * (1 - 2.0**-40), f16_mid * (1 + 2.0**-35)])
    special = np.array([0.0, -0.0, np.inf, -np.inf, 65504.0, 65519.99, 65520.0, 2.0**-24, 2.0**-25,
                        2.0**-25 * 1.0000001, 3 * 2.0**-26, 6.1e-5, 5.96e-8, 1e-45, 3.4e38, -3.4e38])
    x = np.concatenate([base, bf_mid, f16_mid, nudge, special])
    h = np.arange(65536, dtype=np.uint16)
    save("rounding.npz", x=x, bf16=R.round(x, BF16), f16=R.round(x, F16),
         f16_decode=R.f16_to_f64(h))


def fmath():
    rng = np.random.default_rng(11)
    x = np.concatenate([rng.uniform(-745, 709, 3000), rng.uniform(-30, 0, 3000),
                        rng.uniform(-8, 8, 3000), rng.normal(0, 3, 3000), [0.0, -0.0, 1e-300, -1e-30]])
    xt = np.concatenate([rng.uniform(-30, 30, 3000), rng.uniform(-1, 1, 3000), [0.0, 50.0, -50.0, 22.0, 1e-20]])
    xs = np.concatenate([rng.uniform(0, 1.6e6, 3000), rng.uniform(-8, 8, 3000), [0.0, 1e-30, np.pi / 4]])
    e = -np.arange(0, 256, 2) / 256.0
    save("fmath.npz", x=x, exp=R.vec("ok_expv", x), silu=R.vec("ok_siluv", x), sigmoid=R.vec("ok_sigmoidv", x),
         xt=xt, tanh=R.vec("ok_tanhv", xt), xs=xs, sin=R.vec("ok_sinv", xs), cos=R.vec("ok_cosv", xs),
         pow_e=e, pow_1e6=R.pow_(1e6, e), pow_5e5=R.pow_(5e5, e), pow_1e4=R.pow_(1e4, e))


def config1():
    """f32 x, residual [16, 64] ~ N(0,1), w [64] ~ N(1, 0.1), eps 1e-6;
    gate/up f32 [16, 256] ~ N(0,1). Reference outputs in f64 and in the bf16 twin."""
    out = {}
    x32 = O.to_f64(O.normal(1, (16, 64), 0, 1, F32), F32)
    r32 = O.to_f64(O.normal(2, (16, 64), 0, 1, F32), F32)
    w32 = O.to_f64(O.normal(3, (64,), 1, 0.1, F32), F32)
    g32 = O.to_f64(O.normal(4, (16, 256), 0, 1, F32), F32)
    u32 = O.to_f64(O.normal(5, (16, 256), 0, 1, F32), F32)
    out.update(x=x32, residual=r32, w=w32, gate=g32, up=u32)
    for dt, tag in ((F64, "f64"), (BF16, "bf16")):
        x, r, w, g, u = (R.round(a, dt) for a in (x32, r32, w32, g32, u32))
        h = R.round(x + r, dt)                       # muse_glimmer.hpp:1023-1024
        for kind, kn in ((0, "centered"), (1, "plain"), (2, "weightless")):
            out[f"{tag}_{kn}_y"] = R.rmsnorm_rows(kind, h, None if kind == 2 else w, 1e-6, dt)
        out[f"{tag}_h"] = h
        s = R.vec("ok_siluv", g)
        out[f"{tag}_swiglu"] = s * u if dt == F64 else R.round(R.round(s, dt) * u, dt)  # :1036-1039
    save("config1.npz", **out)


def norms():
    """rmsnorm_rows at the ordered (dim <= 128) and larger dims, all kinds and twin dtypes."""
    out = {}
    for dim in (13, 128, 640):
        x = O.to_f64(O.normal(20 + dim, (9, dim), 0, 2, F64), F64)
        w = O.to_f64(O.normal(21 + dim, (dim,), 1, 0.05, F64), F64)
        out[f"x{dim}"], out[f"w{dim}"] = x, w
        for dt in (F64, BF16, F16):
            xr, wr = R.round(x, dt), R.round(w, dt)
            for kind in (0, 1, 2):
                out[f"y{dim}_k{kind}_d{dt}"] = R.rmsnorm_rows(kind, xr, None if kind == 2 else wr, 1e-6, dt)
        for kind in (0, 1, 2):  # the --hf-f32-compat branch (f64 storage)
            out[f"y{dim}_k{kind}_compat"] = R.rmsnorm_rows(kind, x, None if kind == 2 else w, 1e-6, F64,
                                                           f32_compat=True)
    save("norms.npz", **out)


def bf16exec():
    """The bf16exec candidate's norm_rows (bf16 out) and norm_rows_f32 (bf16 values kept in
    f32, the embedding norm; weight for Plain only) over f32 rows and bf16 weights, every kind."""
    out = {}
    for dim in (13, 640, 6656):
        x = O.from_f64(O.to_f64(O.normal(60 + dim, (6, dim), 0, 1, F32), F32), F32).view(np.float32)
        wb = O.normal(61 + dim, (dim,), 1, 0.05, BF16)
        out[f"x{dim}"], out[f"w{dim}"] = x, wb
        for kind in (0, 1, 2):
            out[f"y{dim}_k{kind}"] = R.bf16exec_norm_rows(kind, x, None if kind == 2 else wb, 1e-6)
            out[f"f{dim}_k{kind}"] = R.bf16exec_norm_rows_f32(kind, x, None if kind == 2 else wb, 1e-6)
    save("bf16exec.npz", **out)


def rope():
    out = {}
    for theta, dim, T in ((1e6, 128, 64), (5e5, 128, 48), (1e4, 64, 40)):
        tag = f"{int(theta)}_{dim}"
        for dt in (F64, BF16, F16):
            c, s = R.rope_table(theta, dim, T, dt)
            out[f"cos_{tag}_d{dt}"], out[f"sin_{tag}_d{dt}"] = c, s
            x = R.round(O.to_f64(O.normal(30 + dt, (T, dim), 0, 1, F64), F64), dt)
            out[f"x_{tag}_d{dt}"] = x
            out[f"rot_{tag}_d{dt}"] = np.stack([R.apply_rope_vec(x[t], c, s, t, dt) for t in range(T)])
        c, s = R.rope_table(theta, dim, T, F64, f32_compat=True)  # the --hf-f32-compat table
        out[f"cos_{tag}_compat"], out[f"sin_{tag}_compat"] = c, s
    save("rope.npz", **out)


def tail():
    out = {}
    for dt in (F64, BF16, F16):
        z = R.round(O.to_f64(O.normal(40 + dt, (4096,), 0, 40 if dt != F16 else 20, F64), F64), dt)
        out[f"z_d{dt}"] = z
        for mult, cap in ((1.0, 30.0), (0.5, 30.0), (2.0, 0.0)):
            out[f"tail_d{dt}_m{mult}_c{cap}"] = R.output_tail(z, mult, cap, dt)
    save("tail.npz", **out)


def npy():
    """.npy files written by the reference's own save_npy / save_npy_i64
    (src/tensor.cpp), and the reference's load_npy of files numpy wrote in every
    element type it reads ('<f8', '<f4', '<i8', '<i4', '|u1')."""
    d = os.path.join(HERE, "npy")
    os.makedirs(d, exist_ok=True)
    # tests/test_npy.cpp:13-17's tensor: [2, 3], 0.1 i - 0.25
    R.save_npy(os.path.join(d, "ref_f64_2x3.npy"), (0.1 * np.arange(6.0) - 0.25).reshape(2, 3))
    R.save_npy(os.path.join(d, "ref_f64_2x1x5.npy"), O.to_f64(O.normal(50, (2, 1, 5), 0, 1, F64), F64))
    R.save_npy(os.path.join(d, "ref_f64_7.npy"), O.to_f64(O.normal(51, (7,), 0, 1e10, F64), F64))
    R.save_npy(os.path.join(d, "ref_i64_3.npy"), np.array([5, -1, 262143], np.int64))  # test_npy.cpp:26
    rng = np.random.default_rng(52)
    written = {
        "np_f4": rng.normal(0, 3, (3, 4)).astype("<f4"),
        "np_i4": rng.integers(-2**31, 2**31, (5,), dtype=np.int64).astype("<i4"),
        "np_i8": rng.integers(-2**62, 2**62, (2, 2), dtype=np.int64).astype("<i8"),
        "np_u1": rng.integers(0, 256, (4, 2, 2), dtype=np.int64).astype("|u1"),
        "np_f8": rng.normal(0, 1, (3,)).astype("<f8"),
    }
    loaded = {}
    for name, a in written.items():
        path = os.path.join(d, name + ".npy")
        np.save(path, a, allow_pickle=False)
        loaded[name] = R.load_npy(path, a.shape)
    save("npy.npz", **loaded)


if __name__ == "__main__":
    if not O.Ref.available():
        sys.exit("oracle/_ref is not built (make -C oracle ref)")
    parts = {"rounding": rounding, "fmath": fmath, "config1": config1, "norms": norms, "rope": rope,
             "tail": tail, "npy": npy, "bf16exec": bf16exec}
    for name in sys.argv[1:] or parts:
        parts[name]()
