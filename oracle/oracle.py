"""ORACLE — test infrastructure only.

ctypes bindings over ``oracle/liboracle.so`` (the CPU restatement of the
reference's CPU tensor path, ``oracle/oracle.cpp``) and, where it was built in
this container, over ``oracle/_ref`` (the reference's own sources compiled by
``oracle/Makefile``).  Only tests/, ``__graft_entry__.smoke()`` and bench.py's
``cpu_baseline`` leg import this module, and only as the checker or the timed
CPU baseline.

Arrays cross the boundary as numpy arrays.  Oracle ops run on float64 arrays
that hold storage-rounded values, exactly as the reference's twin does
(``src/muse_glimmer.hpp`` keeps every tensor as f64).  Storage dtypes:
0 f64, 1 bf16, 2 f16 (``prec::Dtype`` order, ``src/rounding.hpp:31-36``),
3 f32.  bf16/f16 storage is carried as uint16 bit patterns.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
F64, BF16, F16, F32 = 0, 1, 2, 3
F32_COMPAT = 0x100  # OR-ed into F64: the --hf-f32-compat chains (norm, RoPE table, softmax)
CENTERED, PLAIN, WEIGHTLESS = 0, 1, 2
MASK_NONE, MASK_CAUSAL, MASK_WINDOW, MASK_BIWINDOW = 0, 1, 2, 3

_P = ctypes.c_void_p
_I = ctypes.c_int64
_D = ctypes.c_double
_INT = ctypes.c_int
_U64 = ctypes.c_uint64

_SIGS = {
    "or_to_f64": [_P, _INT, _P, _I],
    "or_from_f64": [_P, _INT, _P, _I],
    "or_round": [_INT, _P, _I],
    "or_fill_normal": [_U64, _D, _D, _INT, _P, _I],
    "or_fill_uniform": [_U64, _D, _D, _INT, _P, _I],
    "or_fill_int8": [_U64, _INT, _INT, _P, _I],
    "or_expv": [_P, _P, _I], "or_logv": [_P, _P, _I], "or_expm1v": [_P, _P, _I],
    "or_tanhv": [_P, _P, _I], "or_sinv": [_P, _P, _I], "or_cosv": [_P, _P, _I],
    "or_powv": [_D, _P, _P, _I], "or_siluv": [_P, _P, _I], "or_sigmoidv": [_P, _P, _I],
    "or_meansq": [_P, _P, _I, _I],
    "or_rmsnorm_rows": [_INT, _P, _P, _D, _P, _I, _I, _INT],
    "or_residual_rmsnorm": [_INT, _P, _P, _P, _D, _P, _I, _I, _INT],
    "or_norm_rows_mixed": [_INT, _P, _P, _D, _P, _I, _I, _INT],
    "or_residual_add": [_P, _P, _I, _INT],
    "or_swiglu": [_P, _P, _P, _I, _INT],
    "or_sigmoid_gate": [_P, _P, _P, _I, _INT],
    "or_scale": [_P, _I, _D, _INT],
    "or_rope_table": [_D, _I, _I, _INT, _P, _P],
    "or_apply_rope": [_P, _I, _I, _I, _I, _P, _P, _P, _INT],
    "or_softcap": [_P, _I, _D, _D, _INT],
    "or_softmax_rows": [_P, _P, _I, _I, _I, _D, _INT, _I, _I, _D, _INT, _INT],
    "or_dequant_q8_0": [_P, _P, _P, _I, _I, _INT],
    "or_quantize_q8_0": [_P, _P, _P, _I, _I],
    "or_vocab_reduce": [_P, _I, _I, _I, _P, _P, _P, _P],
    "or_sample_dist": [_P, _P, _P, _I, _I, _D, _D, _D, _P, _P, _P],
    "or_norm_rows_f32": [_INT, _P, _P, _D, _P, _I, _I],
    "or_save_npy_f64": [ctypes.c_char_p, _P, _P, _INT],
    "or_save_npy_i64": [ctypes.c_char_p, _P, _I],
    "or_npy_info": [ctypes.c_char_p, ctypes.c_char_p, _P, ctypes.POINTER(_INT)],
    "or_load_npy": [ctypes.c_char_p, _P, _I],
    "or_num_threads": [],
}

_INT_RESULT = ("or_num_threads", "or_save_npy_f64", "or_save_npy_i64", "or_npy_info", "or_load_npy")
_lib = None


def lib():
    global _lib
    if _lib is None:
        path = os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is not built (run `make -C oracle`)")
        L = ctypes.CDLL(path)
        for name, args in _SIGS.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int if name in _INT_RESULT else None
        L.or_last_error.argtypes = []
        L.or_last_error.restype = ctypes.c_char_p
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def _c(a, dtype=np.float64):
    return np.ascontiguousarray(a, dtype=dtype)


def storage_np_dtype(dt):
    return {F64: np.float64, F32: np.float32, BF16: np.uint16, F16: np.uint16}[dt]


# ------------------------------------------------------------------ storage
def to_f64(a, dt):
    a = np.ascontiguousarray(a)
    out = np.empty(a.shape, np.float64)
    lib().or_to_f64(_p(a), dt, _p(out), a.size)
    return out


def from_f64(x, dt):
    x = _c(x)
    out = np.empty(x.shape, storage_np_dtype(dt))
    lib().or_from_f64(_p(x), dt, _p(out), x.size)
    return out


def rnd(x, dt):
    y = _c(x).copy()
    lib().or_round(dt, _p(y), y.size)
    return y


# --------------------------------------------------------------- generators
def normal(seed, shape, mean=0.0, std=1.0, dt=F64):
    n = int(np.prod(shape))
    out = np.empty(n, storage_np_dtype(dt))
    lib().or_fill_normal(seed, mean, std, dt, _p(out), n)
    return out.reshape(shape)


def uniform(seed, shape, lo, hi, dt=F64):
    n = int(np.prod(shape))
    out = np.empty(n, storage_np_dtype(dt))
    lib().or_fill_uniform(seed, lo, hi, dt, _p(out), n)
    return out.reshape(shape)


def int8_uniform(seed, shape, lo=-127, hi=127):
    n = int(np.prod(shape))
    out = np.empty(n, np.int8)
    lib().or_fill_int8(seed, lo, hi, _p(out), n)
    return out.reshape(shape)


# -------------------------------------------------------------------- fmath
def _vec(name, x, *pre):
    x = _c(x)
    y = np.empty_like(x)
    getattr(lib(), name)(*pre, _p(x), _p(y), x.size)
    return y


def exp(x): return _vec("or_expv", x)
def log(x): return _vec("or_logv", x)
def expm1(x): return _vec("or_expm1v", x)
def tanh(x): return _vec("or_tanhv", x)
def sin(x): return _vec("or_sinv", x)
def cos(x): return _vec("or_cosv", x)
def silu(x): return _vec("or_siluv", x)
def sigmoid(x): return _vec("or_sigmoidv", x)
def pow_(base, e): return _vec("or_powv", e, base)


def mean_sq(X):
    X = _c(X)
    rows, dim = X.shape
    out = np.empty(rows)
    lib().or_meansq(_p(X), _p(out), rows, dim)
    return out


# ---------------------------------------------------------------------- ops
def rmsnorm_rows(kind, X, w, eps, dt):
    X = _c(X)
    rows, dim = X.shape
    Y = np.empty_like(X)
    w = _c(w) if w is not None else None
    lib().or_rmsnorm_rows(kind, _p(X), _p(w), eps, _p(Y), rows, dim, dt)
    return Y


def norm_rows_mixed(kind, X, w, eps, dt):
    """bf16exec's norm_rows (src/bf16exec.hpp:398-421): X, w storage-valued f64; output rounded to dt."""
    X = _c(X)
    rows, dim = X.shape
    Y = np.empty_like(X)
    w = _c(w) if w is not None else None
    lib().or_norm_rows_mixed(kind, _p(X), _p(w), eps, _p(Y), rows, dim, dt)
    return Y


def norm_rows_f32(kind, X, w, eps):
    """bf16exec's norm_rows_f32 (src/bf16exec.hpp:422-442): X f32-valued f64, w bf16-valued
    (read for Plain only); the output bf16-rounded values as f64."""
    X = _c(X)
    rows, dim = X.shape
    Y = np.empty_like(X)
    w = _c(w) if w is not None else None
    lib().or_norm_rows_f32(kind, _p(X), _p(w), eps, _p(Y), rows, dim)
    return Y


def residual_rmsnorm(kind, h, x, w, eps, dt):
    """Returns (y, h_new)."""
    h = _c(h).copy()
    x = _c(x)
    rows, dim = h.shape
    Y = np.empty_like(h)
    w = _c(w) if w is not None else None
    lib().or_residual_rmsnorm(kind, _p(h), _p(x), _p(w), eps, _p(Y), rows, dim, dt)
    return Y, h


def residual_add(h, x, dt):
    h = _c(h).copy()
    lib().or_residual_add(_p(h), _p(_c(x)), h.size, dt)
    return h


def swiglu(g, u, dt):
    g, u = _c(g), _c(u)
    out = np.empty_like(g)
    lib().or_swiglu(_p(g), _p(u), _p(out), g.size, dt)
    return out


def sigmoid_gate(pv, gate, dt):
    pv, gate = _c(pv), _c(gate)
    out = np.empty_like(pv)
    lib().or_sigmoid_gate(_p(pv), _p(gate), _p(out), pv.size, dt)
    return out


def scale(x, s, dt):
    x = _c(x).copy()
    lib().or_scale(_p(x), x.size, s, dt)
    return x


def rope_table(theta, dim, T, dt):
    c = np.empty((T, dim // 2))
    s = np.empty((T, dim // 2))
    lib().or_rope_table(theta, dim, T, dt, _p(c), _p(s))
    return c, s


def apply_rope(x, cos_t, sin_t, pos, dt):
    """x: [tokens, heads, dim] float64 (a copy is rotated and returned)."""
    x = _c(x).copy()
    tokens, heads, dim = x.shape
    pos = _c(pos, np.int64)
    lib().or_apply_rope(_p(x), tokens, heads, dim, heads * dim, _p(_c(cos_t)), _p(_c(sin_t)), _p(pos), dt)
    return x


def softcap(z, mult, cap, dt):
    z = _c(z).copy()
    lib().or_softcap(_p(z), z.size, mult, cap, dt)
    return z


def softmax_rows(x, scale, mask=MASK_NONE, window=0, q_pos0=0, softcap=0.0, dt_in=F32, dt_out=BF16):
    """x: [heads, q, k] float64 holding dt_in values.  Returns f64 values rounded to dt_out."""
    x = _c(x)
    heads, q, k = x.shape
    y = np.empty_like(x)
    lib().or_softmax_rows(_p(x), _p(y), heads, q, k, scale, mask, window, q_pos0, softcap, dt_in, dt_out)
    return y


def dequant_q8_0(qs, d, dt_out=BF16):
    qs = _c(qs, np.int8)
    d = _c(d, np.uint16)
    rows, n_in = qs.shape
    out = np.empty((rows, n_in))
    lib().or_dequant_q8_0(_p(qs), _p(d), _p(out), rows, n_in, dt_out)
    return out


def quantize_q8_0(w_bf16_bits):
    w = _c(w_bf16_bits, np.uint16)
    rows, n_in = w.shape
    qs = np.empty((rows, n_in), np.int8)
    d = np.empty((rows, n_in // 32), np.uint16)
    lib().or_quantize_q8_0(_p(w), _p(qs), _p(d), rows, n_in)
    return qs, d


def vocab_reduce(L, K):
    """Returns (lse f64 [rows], argmax i64 [rows], top_idx i64 [rows,K], top_val f64 [rows,K])."""
    L = _c(L)
    rows, V = L.shape
    lse = np.empty(rows)
    am = np.empty(rows, np.int64)
    ti = np.empty((rows, K), np.int64)
    tv = np.empty((rows, K))
    lib().or_vocab_reduce(_p(L), rows, V, K, _p(lse), _p(am), _p(ti), _p(tv))
    return lse, am, ti, tv


def sample_dist(top_idx, top_val, argmax, temperature, top_p, min_p):
    """Sampler._transformed's final distribution (serve/sampler.py:85-112) from a row's
    top-K candidates (value desc, index asc). Returns (ids i64 [rows,K], probs f64
    [rows,K], n i64 [rows]); slots past n[r] hold -1 / 0."""
    ti = _c(top_idx, np.int64)
    tv = _c(top_val)
    am = _c(argmax, np.int64)
    rows, K = ti.shape
    ids = np.full((rows, K), -1, np.int64)
    p = np.zeros((rows, K))
    n = np.zeros(rows, np.int64)
    lib().or_sample_dist(_p(ti), _p(tv), _p(am), rows, K, temperature, top_p, min_p, _p(ids), _p(p), _p(n))
    return ids, p, n


def sample_rows(lg, raw_argmax, top_k, temperature, top_p, min_p):
    """Sampler._transformed's final distribution (serve/sampler.py:43-112) on rows of
    already-edited f32 logits, for any top_k, in numpy float32 as the reference computes
    it (its steps in its order: finite check 70-74, greedy 76-78, candidates 80-95, the
    -inf drop 97-98, softmax 104, top_p 104-106, min_p 107-109, final softmax 111-112).
    The one choice the reference leaves open, which of several values tied at the
    top_k-th place argpartition keeps and their order, is fixed here as lower index
    first (numpy's stable lexsort). Returns one (ids int64, probs float32) pair per row;
    the probabilities follow the reference's float32 operations, so cuts at top_p and
    min_p fall exactly where the reference's fall."""
    lg = np.asarray(lg, dtype=np.float32)
    out = []
    f32 = np.float32
    for r in range(lg.shape[0]):
        x = lg[r]
        V = x.size
        if not np.isfinite(x).any():          # fully masked: the raw logits' argmax
            out.append((np.array([int(raw_argmax[r])], np.int64), np.ones(1, f32)))
            continue
        if not temperature > 0:               # greedy: first maximum (NaN counts as largest)
            out.append((np.array([int(np.argmax(x))], np.int64), np.ones(1, f32)))
            continue
        # value-descending order, ties by index (NaN last, -inf before it)
        order = np.lexsort((np.arange(V), -x))
        kk = min(top_k, V) if top_k > 0 else 0
        if kk:
            ids = order[:kk]
        elif top_p < 1.0:
            ids = order
        else:
            ids = np.arange(V)
        vals = x[ids]
        live = vals > -np.inf
        ids, vals = ids[live], vals[live]
        ex = np.exp(vals - vals.max())
        p = ex / ex.sum()
        if top_p < 1.0:
            cut = int(np.searchsorted(np.cumsum(p), top_p)) + 1
            ids, vals, p = ids[:cut], vals[:cut], p[:cut]
        if min_p > 0.0:
            sel = p >= min_p * p.max()
            ids, vals = ids[sel], vals[sel]
        y = vals / f32(temperature)
        ey = np.exp(y - y.max())
        q = ey / ey.sum()
        out.append((ids.astype(np.int64), (q / q.sum()).astype(f32)))
    return out


class NpyError(RuntimeError):
    pass


def _npy_check(rc):
    if rc != 0:
        raise NpyError(lib().or_last_error().decode())


def save_npy(path, arr):
    """save_npy / save_npy_i64 (src/tensor.cpp): float arrays as '<f8', int arrays
    as a '<i8' vector (.npy v1.0, header padded to 64 bytes)."""
    a = np.asarray(arr)
    if a.dtype.kind in "iu":
        a = np.ascontiguousarray(a.reshape(-1), np.int64)
        _npy_check(lib().or_save_npy_i64(os.fsencode(path), _p(a), a.size))
    else:
        a = np.array(a, np.float64, order="C")  # keeps a 0-d shape (ascontiguousarray would not)
        shape = np.array(a.shape, np.int64)
        _npy_check(lib().or_save_npy_f64(os.fsencode(path), _p(a), _p(shape), a.ndim))


def load_npy(path):
    """load_npy (src/tensor.cpp): returns (f64 array of the file's shape, descr)."""
    descr = ctypes.create_string_buffer(8)
    shape = np.zeros(8, np.int64)
    nd = _INT(0)
    _npy_check(lib().or_npy_info(os.fsencode(path), descr, _p(shape), ctypes.byref(nd)))
    shp = tuple(int(v) for v in shape[:nd.value])
    out = np.empty(shp, np.float64)
    _npy_check(lib().or_load_npy(os.fsencode(path), _p(out), out.size))
    return out, descr.value.decode()


def num_threads():
    return lib().or_num_threads()


# ---------------------------------------------------------- oracle/_ref
class Ref:
    """The reference's own code, compiled from /root/reference by oracle/Makefile."""

    def __init__(self):
        d = os.path.join(HERE, "_ref")
        self.k = ctypes.CDLL(os.path.join(d, "libmuse_refkernels.so"))
        self.s = ctypes.CDLL(os.path.join(d, "libref_shim.so"))
        for n in ("ok_expv", "ok_tanhv", "ok_sinv", "ok_cosv", "ok_siluv", "ok_sigmoidv"):
            getattr(self.k, n).argtypes = [_P, _P, _I]
            getattr(self.k, n).restype = None
        self.k.ok_powv.argtypes = [_D, _P, _P, _I]
        self.k.ok_meansq.argtypes = [_P, _P, _I, _I]
        self.s.rs_round.argtypes = [_INT, _P, _P, _I]
        self.s.rs_f16_to_f64.argtypes = [_P, _P, _I]
        self.s.rs_rmsnorm_rows.argtypes = [_INT, _P, _P, _D, _P, _I, _I, _INT, _INT]
        self.s.rs_bf16exec_norm_rows.argtypes = [_INT, _P, _P, _D, _P, _I, _I]
        self.s.rs_bf16exec_norm_rows_f32.argtypes = [_INT, _P, _P, _D, _P, _I, _I]
        self.s.rs_bf16exec_norm_rows.restype = None
        self.s.rs_bf16exec_norm_rows_f32.restype = None
        self.s.rs_rope_table.argtypes = [_D, _I, _I, _INT, _INT, _P, _P]
        self.s.rs_apply_rope.argtypes = [_P, _I, _P, _P, _I, _I, _INT]
        self.s.rs_output_tail.argtypes = [_D, _D, _P, _I, _INT]
        self.s.rs_save_npy_f64.argtypes = [ctypes.c_char_p, _P, _P, _INT]
        self.s.rs_save_npy_i64.argtypes = [ctypes.c_char_p, _P, _I]
        self.s.rs_load_npy.argtypes = [ctypes.c_char_p, _P, _I]
        for f in (self.s.rs_save_npy_f64, self.s.rs_save_npy_i64, self.s.rs_load_npy):
            f.restype = _INT
        for f in (self.k.ok_powv, self.k.ok_meansq, self.s.rs_round, self.s.rs_f16_to_f64,
                  self.s.rs_rmsnorm_rows, self.s.rs_rope_table, self.s.rs_apply_rope,
                  self.s.rs_output_tail):
            f.restype = None

    @staticmethod
    def available():
        d = os.path.join(HERE, "_ref")
        return all(os.path.exists(os.path.join(d, f)) for f in ("libmuse_refkernels.so", "libref_shim.so"))

    def vec(self, name, x):
        x = _c(x)
        y = np.empty_like(x)
        getattr(self.k, name)(_p(x), _p(y), x.size)
        return y

    def pow_(self, base, e):
        e = _c(e)
        y = np.empty_like(e)
        self.k.ok_powv(base, _p(e), _p(y), e.size)
        return y

    def mean_sq(self, X):
        X = _c(X)
        out = np.empty(X.shape[0])
        self.k.ok_meansq(_p(X), _p(out), X.shape[0], X.shape[1])
        return out

    def round(self, x, dt):
        x = _c(x)
        y = np.empty_like(x)
        self.s.rs_round(dt, _p(x), _p(y), x.size)
        return y

    def f16_to_f64(self, h):
        h = _c(h, np.uint16)
        y = np.empty(h.shape)
        self.s.rs_f16_to_f64(_p(h), _p(y), h.size)
        return y

    def rmsnorm_rows(self, kind, X, w, eps, dt, f32_compat=False):
        X = _c(X)
        Y = np.empty_like(X)
        w = _c(w) if w is not None else None
        self.s.rs_rmsnorm_rows(kind, _p(X), _p(w), eps, _p(Y), X.shape[0], X.shape[1], int(f32_compat), dt)
        return Y

    def bf16exec_norm_rows(self, kind, X, wt, eps):
        """Engine::norm_rows (bf16exec.hpp:398-420): X f32 [rows, dim], wt bf16 bits -> bf16 bits"""
        X = np.ascontiguousarray(X, np.float32)
        wt = None if wt is None else np.ascontiguousarray(wt, np.uint16)
        out = np.empty(X.shape, np.uint16)
        self.s.rs_bf16exec_norm_rows(kind, _p(X), _p(wt), eps, _p(out), X.shape[0], X.shape[1])
        return out

    def bf16exec_norm_rows_f32(self, kind, X, wt, eps):
        """Engine::norm_rows_f32 (bf16exec.hpp:422-442): X f32 [rows, dim] -> f32 holding bf16 values"""
        X = np.ascontiguousarray(X, np.float32)
        wt = None if wt is None else np.ascontiguousarray(wt, np.uint16)
        out = np.empty(X.shape, np.float32)
        self.s.rs_bf16exec_norm_rows_f32(kind, _p(X), _p(wt), eps, _p(out), X.shape[0], X.shape[1])
        return out

    def rope_table(self, theta, dim, T, dt, f32_compat=False):
        c = np.empty((T, dim // 2))
        s = np.empty((T, dim // 2))
        self.s.rs_rope_table(theta, dim, T, int(f32_compat), dt, _p(c), _p(s))
        return c, s

    def apply_rope_vec(self, x, cos_t, sin_t, pos, dt):
        x = _c(x).copy()
        cos_t, sin_t = _c(cos_t), _c(sin_t)
        self.s.rs_apply_rope(_p(x), x.size, _p(cos_t), _p(sin_t), cos_t.shape[0], pos, dt)
        return x

    def save_npy(self, path, arr):
        """the reference's save_npy ('<f8' tensor) or save_npy_i64 ('<i8' vector)"""
        a = np.asarray(arr)
        if a.dtype.kind in "iu":
            a = np.ascontiguousarray(a.reshape(-1), np.int64)
            rc = self.s.rs_save_npy_i64(os.fsencode(path), _p(a), a.size)
        else:
            a = np.array(a, np.float64, order="C")
            shape = np.array(a.shape, np.int64)
            rc = self.s.rs_save_npy_f64(os.fsencode(path), _p(a), _p(shape), a.ndim)
        if rc != 0:
            raise NpyError(f"reference save_npy failed on {path}")

    def load_npy(self, path, shape):
        """the reference's load_npy, widened to f64, for a file of `shape`"""
        out = np.empty(shape, np.float64)
        if self.s.rs_load_npy(os.fsencode(path), _p(out), out.size) != 0:
            raise NpyError(f"reference load_npy failed on {path}")
        return out

    def output_tail(self, z, mult, cap, dt):
        z = _c(z).copy()
        self.s.rs_output_tail(mult, cap, _p(z), z.size, dt)
        return z
