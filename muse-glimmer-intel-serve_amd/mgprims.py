"""Python binding of libmgprims (include/mg_prims.h) over ctypes.

The host-side mirror of the reference's primitive interface for callers that
hold device tensors in PyTorch: the names and argument meanings follow the
reference's functions (``muse::rmsnorm_rows``, ``apply_rope``,
``build_rope_table``, ``apply_output_tail`` in src/muse_glimmer.hpp, the
residual / SwiGLU / output-gate loops of the layer body, the Q8_0 dequantize of
src/gpu/gpu_engine.cpp, and the sampler's logsumexp / argmax / top-k), and
errors surface as exceptions carrying ``mg_last_error()``, as the reference's
host functions throw ``std::runtime_error``.

PyTorch only supplies device memory and the stream: every op runs a HIP kernel
of libmgprims.so on the context's stream (by default torch's current stream).
There is no CPU fallback: constructing ``Prims`` fails if the library is not
built or no GPU is visible.
"""
from __future__ import annotations

import ctypes
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB_PATH = os.path.join(HERE, "libmgprims.so")
HEADER = os.path.join(ROOT, "include", "mg_prims.h")

F64, BF16, F16, F32 = 0, 1, 2, 3
BF16_AS_F32 = 4  # f32 words holding bf16 values (an output format of norm_rows_mixed)
F32_COMPAT = 0x100  # with F64: the reference's --hf-f32-compat chains
CENTERED, PLAIN, WEIGHTLESS = 0, 1, 2
MASK_NONE, MASK_CAUSAL, MASK_WINDOW, MASK_BIWINDOW = 0, 1, 2, 3

_P = ctypes.c_void_p
_I = ctypes.c_int64
_D = ctypes.c_double
_INT = ctypes.c_int

_SIGS = {
    "mg_last_error": ([], ctypes.c_char_p),
    "mg_open": ([_INT, _P, _I, ctypes.POINTER(_P)], _INT),
    "mg_close": ([_P], _INT),
    "mg_sync": ([_P], _INT),
    "mg_set_stream": ([_P, _P], _INT),
    "mg_get_stream": ([_P], _P),
    "mg_rmsnorm_rows": ([_P, _INT, _P, _I, _P, _D, _P, _I, _I, _I, _INT], _INT),
    "mg_norm_rows_mixed": ([_P, _INT, _P, _I, _INT, _P, _INT, _D, _P, _I, _INT, _I, _I], _INT),
    "mg_residual_rmsnorm": ([_P, _INT, _P, _I, _P, _I, _P, _D, _P, _I, _I, _I, _INT], _INT),
    "mg_residual_add": ([_P, _P, _P, _I, _INT], _INT),
    "mg_swiglu": ([_P, _P, _P, _P, _I, _INT], _INT),
    "mg_sigmoid_gate": ([_P, _P, _P, _P, _I, _INT], _INT),
    "mg_scale": ([_P, _P, _I, _D, _INT], _INT),
    "mg_rope_table": ([_P, _D, _I, _I, _INT, _P, _P], _INT),
    "mg_rope": ([_P, _P, _I, _I, _P, _I, _I, _I, _I, _P, _P, _I, _P, _I, _INT], _INT),
    "mg_qk_norm_rope": ([_P, _P, _I, _I, _P, _I, _I, _I, _I, _D, _D, _P, _P, _I, _P, _I, _P, _I, _P, _P, _I, _INT],
                        _INT),
    "mg_softmax_rows": ([_P, _P, _I, _P, _I, _I, _I, _I, _D, _INT, _I, _I, _D, _INT, _INT], _INT),
    "mg_softcap": ([_P, _P, _I, _D, _D, _INT], _INT),
    "mg_dequant_q8_0": ([_P, _P, _P, _P, _I, _I, _INT], _INT),
    "mg_vocab_reduce": ([_P, _P, _I, _I, _I, _INT, _I, _P, _P, _P, _P], _INT),
    "mg_quantize_q8_0": ([_P, _P, _I, _I, _P, _P], _INT),
    "mg_gemv_q8_0": ([_P, _P, _P, _P, _I, _I, _I, _I, _P, _I, _INT], _INT),
    "mg_attn_decode": ([_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _D, _P], _INT),
    "mg_attn_prefill": ([_P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _I, _I, _D, _P, _I], _INT),
    "mg_sample_dist": ([_P, _P, _P, _P, _P, _I, _I, _D, _D, _D, _P, _P, _P], _INT),
    "mg_sample_rows": ([_P, _P, _I, _I, _I, _P, _I, _D, _D, _D, _P, _P, _P], _INT),
    "mg_vocab_reduce_tail": ([_P, _P, _I, _I, _I, _INT, _D, _D, _I, _P, _P, _P, _P, _P], _INT),
    "mg_vocab_reduce_noalloc": ([_P, _P, _I, _I, _I, _INT, _I, _P, _P, _P, _P], _INT),
    "mg_probe_stream": ([_P, _INT, _P, _P, _P, _P, _I], _INT),
    "mg_npy_info": ([ctypes.c_char_p, ctypes.c_char_p, _P, _INT, ctypes.POINTER(_INT)], _INT),
    "mg_npy_load": ([_P, ctypes.c_char_p, _P, _I, _INT], _INT),
    "mg_npy_save": ([_P, ctypes.c_char_p, _P, _INT, _P, _INT], _INT),
    "mg_npy_save_i64": ([_P, ctypes.c_char_p, _P, _I], _INT),
}

_lib = None


def header_symbols():
    """Every function the public header declares."""
    with open(HEADER) as f:
        text = f.read()
    return sorted(set(re.findall(r"\b(mg_[a-z0-9_]+)\s*\(", text)))


def load_library(path: str = LIB_PATH):
    """dlopen libmgprims.so and bind every exported signature (no GPU needed)."""
    global _lib
    if _lib is None:
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is not built: run `python muse-glimmer-intel-serve_amd/build.py`")
        L = ctypes.CDLL(path)
        for name, (args, res) in _SIGS.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


class MgError(RuntimeError):
    pass


def npy_info(path):
    """(descr, shape) of an .npy file, read by the library (mg_npy_info; no GPU needed)"""
    L = load_library()
    descr = ctypes.create_string_buffer(16)
    shape = (ctypes.c_int64 * 32)()
    nd = _INT(0)
    if L.mg_npy_info(os.fsencode(path), descr, ctypes.cast(shape, _P), 32, ctypes.byref(nd)) != 0:
        raise MgError(L.mg_last_error().decode())
    return descr.value.decode(), tuple(shape[i] for i in range(nd.value))


def _dtype_code(t):
    import torch
    return {torch.float64: F64, torch.bfloat16: BF16, torch.float16: F16, torch.float32: F32}[t.dtype]


def _code(t, f32_compat=False):
    """dtype code of t, with the f32-compat flag when asked (the library
    accepts it with f64 storage only and raises otherwise)"""
    return _dtype_code(t) | (F32_COMPAT if f32_compat else 0)


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


class Prims:
    """A libmgprims context bound to one device and stream."""

    def __init__(self, device: int = 0, stream=None, workspace_bytes: int = 0):
        import torch
        self.lib = load_library()
        if stream is None:
            stream = torch.cuda.current_stream(device).cuda_stream
        h = _P()
        self._check(self.lib.mg_open(device, ctypes.c_void_p(stream), workspace_bytes, ctypes.byref(h)))
        self.h = h
        self.device = device

    def _check(self, rc):
        if rc != 0:
            raise MgError(self.lib.mg_last_error().decode())

    def close(self):
        if getattr(self, "h", None):
            self._check(self.lib.mg_close(self.h))
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def sync(self):
        self._check(self.lib.mg_sync(self.h))

    def set_stream(self, stream):
        self._check(self.lib.mg_set_stream(self.h, ctypes.c_void_p(stream)))

    def stream(self):
        return self.lib.mg_get_stream(self.h)

    # ------------------------------------------------------------ checks
    # The ABI takes raw device pointers with element counts or row strides; these
    # checks keep a view the kernels cannot read that way (a transposed or sliced
    # tensor, another device, an undersized output) from reaching them.
    def _dev(self, *ts):
        for t in ts:
            if t is not None and (t.device.type != "cuda" or t.device.index != self.device):
                raise MgError(f"tensor on {t.device}, context on cuda:{self.device}")

    @staticmethod
    def _contig(name, *ts):
        for t in ts:
            if t is not None and not t.is_contiguous():
                raise MgError(f"{name}: tensors must be contiguous")

    @staticmethod
    def _rows(name, t, ndim=2):
        """a [.., rows, cols] view with unit inner stride and one row stride; returns it"""
        if t.dim() != ndim:
            raise MgError(f"{name}: expected a {ndim}-d tensor, got shape {tuple(t.shape)}")
        if t.stride(-1) != 1 and t.shape[-1] > 1:
            raise MgError(f"{name}: the last dimension must have stride 1")
        ld = t.stride(-2) if t.shape[-2] > 1 else t.shape[-1]
        if ndim == 3 and t.shape[0] > 1 and t.stride(0) != t.shape[1] * ld:
            raise MgError(f"{name}: rows of consecutive heads must share one row stride")
        return max(ld, t.shape[-1])

    @staticmethod
    def _same(name, a, b, what="dtype"):
        if a is not None and b is not None and getattr(a, what) != getattr(b, what):
            raise MgError(f"{name}: {what} {getattr(a, what)} and {getattr(b, what)} differ")

    @staticmethod
    def _numel(name, t, n):
        if t is not None and t.numel() < n:
            raise MgError(f"{name}: tensor of {t.numel()} elements, {n} needed")

    # ------------------------------------------------------------- norms
    def rmsnorm_rows(self, kind, X, w, eps, Y, f32_compat=False):
        """muse::rmsnorm_rows (src/muse_glimmer.hpp:572-608); X, Y: [rows, dim].
        f32_compat (f64 tensors): the --hf-f32-compat f32 chain."""
        self._dev(X, w, Y)
        ldx, ldy = self._rows("rmsnorm_rows", X), self._rows("rmsnorm_rows", Y)
        self._same("rmsnorm_rows", X, Y)
        self._same("rmsnorm_rows", X, Y, "shape")
        self._same("rmsnorm_rows", X, w)
        self._contig("rmsnorm_rows", w)
        rows, dim = X.shape
        self._numel("rmsnorm_rows weight", w, dim)
        self._check(self.lib.mg_rmsnorm_rows(self.h, kind, _ptr(X), ldx, _ptr(w), eps, _ptr(Y), ldy, rows, dim,
                                             _code(X, f32_compat)))

    def norm_rows_mixed(self, kind, X, w, eps, Y, bf16_as_f32=False):
        """bf16exec's norm_rows (src/bf16exec.hpp:398-421) generalised: X, w and Y each
        at its own dtype (f32 rows, bf16 weights, bf16 output there); X, Y: [rows, dim].
        bf16_as_f32 (Y float32): its norm_rows_f32 (422-442), Y holding the bf16-rounded
        values, the weight applied for PLAIN only; Y may be X (the embedding norm in place)."""
        self._dev(X, w, Y)
        ldx, ldy = self._rows("norm_rows_mixed", X), self._rows("norm_rows_mixed", Y)
        self._same("norm_rows_mixed", X, Y, "shape")
        self._contig("norm_rows_mixed", w)
        rows, dim = X.shape
        self._numel("norm_rows_mixed weight", w, dim)
        ycode = _dtype_code(Y)
        if bf16_as_f32:
            if ycode != F32:
                raise MgError("norm_rows_mixed: bf16_as_f32 needs a float32 output")
            ycode = BF16_AS_F32
        self._check(self.lib.mg_norm_rows_mixed(self.h, kind, _ptr(X), ldx, _dtype_code(X), _ptr(w),
                                                _dtype_code(w) if w is not None else 0, eps, _ptr(Y), ldy,
                                                ycode, rows, dim))

    def residual_rmsnorm(self, kind, h, x, w, eps, y, f32_compat=False):
        """h = rnd(h + x) in place, then y = norm(h); h, x, y: [rows, dim] with unit
        inner stride (each its own row stride)."""
        self._dev(h, x, w, y)
        ldh, ldx, ldy = (self._rows("residual_rmsnorm", t) for t in (h, x, y))
        for t in (x, y):
            self._same("residual_rmsnorm", h, t)
            self._same("residual_rmsnorm", h, t, "shape")
        self._same("residual_rmsnorm", h, w)
        self._contig("residual_rmsnorm", w)
        rows, dim = h.shape
        self._numel("residual_rmsnorm weight", w, dim)
        self._check(self.lib.mg_residual_rmsnorm(self.h, kind, _ptr(h), ldh, _ptr(x), ldx, _ptr(w), eps, _ptr(y),
                                                 ldy, rows, dim, _code(h, f32_compat)))

    def residual_add(self, h, x):
        self._dev(h, x)
        self._contig("residual_add", h, x)
        self._same("residual_add", h, x)
        self._numel("residual_add", x, h.numel())
        self._check(self.lib.mg_residual_add(self.h, _ptr(h), _ptr(x), h.numel(), _dtype_code(h)))

    # ------------------------------------------------------- elementwise
    def _gate(self, name, fn, a, b, out):
        self._dev(a, b, out)
        self._contig(name, a, b, out)
        self._same(name, a, b)
        self._same(name, a, out)
        self._numel(name, b, a.numel())
        self._numel(name, out, a.numel())
        self._check(fn(self.h, _ptr(a), _ptr(b), _ptr(out), a.numel(), _dtype_code(a)))

    def swiglu(self, gate, up, out):
        """out = rnd(rnd(silu(gate)) * up) (src/muse_glimmer.hpp:1036-1039)"""
        self._gate("swiglu", self.lib.mg_swiglu, gate, up, out)

    def sigmoid_gate(self, pv, gate, out):
        """out = rnd(pv * rnd(sigmoid(gate))) (src/muse_glimmer.hpp:896-906)"""
        self._gate("sigmoid_gate", self.lib.mg_sigmoid_gate, pv, gate, out)

    def scale(self, x, s):
        self._dev(x)
        self._contig("scale", x)
        self._check(self.lib.mg_scale(self.h, _ptr(x), x.numel(), s, _dtype_code(x)))

    # --------------------------------------------------------------- rope
    def build_rope_table(self, theta, head_dim, positions, dtype, f32_compat=False):
        """muse::build_rope_table (src/muse_glimmer.hpp:625-674) -> (cos, sin) [positions, head_dim/2].
        f32_compat (torch.float64): the f32 chain stored as double(float(v))."""
        import torch
        co = torch.empty((positions, head_dim // 2), dtype=dtype, device=f"cuda:{self.device}")
        si = torch.empty_like(co)
        self._check(self.lib.mg_rope_table(self.h, theta, head_dim, positions, _code(co, f32_compat), _ptr(co),
                                           _ptr(si)))
        return co, si

    def _heads(self, name, t):
        """[T, heads, D] with each token's heads contiguous; returns the token stride"""
        if t.dim() != 3 or t.stride(2) != 1 or (t.shape[1] > 1 and t.stride(1) != t.shape[2]):
            raise MgError(f"{name}: expected [T, heads, D] with each token's heads contiguous")
        return t.stride(0)

    def _table(self, name, q, cos, sin, positions):
        self._dev(cos, sin, positions)
        self._contig(name, cos, sin, positions)
        self._same(name, q, cos)
        self._same(name, q, sin)
        self._same(name, cos, sin, "shape")
        if cos is not None and cos.shape[-1] != q.shape[2] // 2:
            raise MgError(f"{name}: table rows of {cos.shape[-1]}, head_dim / 2 = {q.shape[2] // 2} needed")
        if positions is not None:
            import torch
            if positions.dtype != torch.int64:
                raise MgError(f"{name}: positions must be int64")
            self._numel(name + " positions", positions, q.shape[0])

    def apply_rope(self, q, k, cos, sin, positions=None, pos0=0):
        """In-place rotate-half RoPE (src/muse_glimmer.hpp:681-705) on q [T, Hq, D] and k [T, Hk, D]."""
        self._dev(q, k)
        ldq = self._heads("apply_rope", q)
        ldk = self._heads("apply_rope", k) if k is not None else 0
        self._same("apply_rope", q, k)
        self._table("apply_rope", q, cos, sin, positions)
        T, qh, D = q.shape
        kh = k.shape[1] if k is not None else 0
        self._check(self.lib.mg_rope(self.h, _ptr(q), qh, ldq, _ptr(k), kh, ldk, T, D, _ptr(cos), _ptr(sin),
                                     cos.shape[0], _ptr(positions), pos0, _dtype_code(q)))

    def qk_norm_rope(self, q, k, eps, qk_scale, cos=None, sin=None, positions=None, pos0=0, v=None,
                     k_cache=None, v_cache=None, f32_compat=False):
        """The sequence around RoPE in one pass (src/muse_glimmer.hpp:799-819): weight-less
        QK-norm over head_dim, q *= qk_scale, RoPE (when a table is given), and the KV-cache
        append k_cache/v_cache [slots, Hk, D] at row position % slots (k_kv_append)."""
        self._dev(q, k, v, k_cache, v_cache)
        ldq = self._heads("qk_norm_rope", q)
        ldk = self._heads("qk_norm_rope", k) if k is not None else 0
        ldv = self._heads("qk_norm_rope", v) if v is not None else 0
        for t in (k, v, k_cache, v_cache):
            self._same("qk_norm_rope", q, t)
        self._contig("qk_norm_rope", k_cache, v_cache)
        self._table("qk_norm_rope", q, cos, sin, positions)
        T, qh, D = q.shape
        kh = k.shape[1] if k is not None else 0
        slots = k_cache.shape[0] if k_cache is not None else 0
        for c in (k_cache, v_cache):
            if c is not None and tuple(c.shape[1:]) != (kh, D):
                raise MgError(f"qk_norm_rope: caches must be [slots, {kh}, {D}], got {tuple(c.shape)}")
        self._check(self.lib.mg_qk_norm_rope(
            self.h, _ptr(q), qh, ldq, _ptr(k), kh, ldk, T, D, eps, qk_scale, _ptr(cos), _ptr(sin),
            cos.shape[0] if cos is not None else 0, _ptr(positions), pos0, _ptr(v), ldv, _ptr(k_cache),
            _ptr(v_cache), slots, _code(q, f32_compat)))

    def attn_prefill(self, q, k_cache, v_cache, pos0, scaling, window=0, out=None):
        """Attention of a prompt chunk over the KV ring (the flash-prefill tier,
        src/gpu/gpu_engine.cpp:3292-3372): q [T, Hq, D] bf16, caches [slots, Hk, D]
        bf16 holding keys up to pos0 + T - 1 -> out [T, Hq, D] f32."""
        import torch
        T, hq, D = q.shape
        slots, hk, _ = k_cache.shape
        if out is None:
            out = torch.empty((T, hq, D), dtype=torch.float32, device=q.device)
        self._dev(q, k_cache, v_cache, out)
        ldq, ldo = self._heads("attn_prefill", q), self._heads("attn_prefill", out)
        self._contig("attn_prefill", k_cache, v_cache)
        self._same("attn_prefill", k_cache, v_cache, "shape")
        self._same("attn_prefill", q, out, "shape")
        self._check(self.lib.mg_attn_prefill(self.h, _ptr(q), ldq, _ptr(k_cache), _ptr(v_cache), T, hq, hk,
                                             D, slots, pos0, window, scaling, _ptr(out), ldo))
        return out

    def attn_decode(self, q, k_cache, v_cache, q_pos, scaling, window=0, out=None):
        """One query token's attention over the KV ring (split-K flash decode):
        q [Hq, D] bf16, caches [slots, Hk, D] bf16 -> out [Hq, D] f32."""
        import torch
        hq, D = q.shape
        slots, hk, _ = k_cache.shape
        if out is None:
            out = torch.empty((hq, D), dtype=torch.float32, device=q.device)
        self._dev(q, k_cache, v_cache, out)
        self._contig("attn_decode", q, k_cache, v_cache, out)
        self._same("attn_decode", k_cache, v_cache, "shape")
        self._numel("attn_decode out", out, hq * D)
        self._check(self.lib.mg_attn_decode(self.h, _ptr(q), _ptr(k_cache), _ptr(v_cache), hq, hk, D, slots, q_pos,
                                            window, scaling, _ptr(out)))
        return out

    # ------------------------------------------------------------ softmax
    def softmax_rows(self, x, y, scale, mask=MASK_NONE, window=0, q_pos0=0, softcap=0.0, f32_compat=False):
        """x [heads, q, k] scores -> y probabilities (attention_forward's softmax, src/muse_glimmer.hpp:828-885).
        f64 x and y: the twin's f64 softmax, or with f32_compat its --hf-f32-compat f32 chain (856-870).
        x and y may be row-strided views (unit inner stride, one row stride each)."""
        self._dev(x, y)
        ldx, ldy = self._rows("softmax_rows", x, 3), self._rows("softmax_rows", y, 3)
        self._same("softmax_rows", x, y, "shape")
        heads, q, kc = x.shape
        self._check(self.lib.mg_softmax_rows(self.h, _ptr(x), ldx, _ptr(y), ldy, heads, q, kc, scale, mask, window,
                                             q_pos0, softcap, _code(x, f32_compat), _dtype_code(y)))

    def apply_output_tail(self, z, mult, cap):
        """muse::apply_output_tail (src/muse_glimmer.hpp:920-943), in place."""
        self._dev(z)
        self._contig("apply_output_tail", z)
        self._check(self.lib.mg_softcap(self.h, _ptr(z), z.numel(), mult, cap, _dtype_code(z)))

    # --------------------------------------------------------------- Q8_0
    def _q8(self, name, qs, d, w):
        import torch
        self._dev(qs, d, w)
        self._contig(name, qs, d, w)
        if qs.dtype != torch.int8 or d.element_size() != 2:
            raise MgError(f"{name}: quants must be int8 and scales 16-bit (f16 bits)")
        rows, n_in = qs.shape
        self._numel(name + " scales", d, rows * (n_in // 32))
        self._numel(name, w, rows * n_in)
        return rows, n_in

    def dequant_q8_0(self, qs, d, out):
        """qs int8 [rows, in], d f16 scales [rows, in/32] -> out [rows, in] (k_dequant_q8)."""
        rows, n_in = self._q8("dequant_q8_0", qs, d, out)
        self._check(self.lib.mg_dequant_q8_0(self.h, _ptr(qs), _ptr(d), _ptr(out), rows, n_in, _dtype_code(out)))

    def quantize_q8_0(self, w, qs, d):
        """w bf16 [rows, in] -> qs int8 [rows, in], d f16 [rows, in/32] (up_w, llama.cpp Q8_0 rule)."""
        import torch
        if w.dtype != torch.bfloat16:
            raise MgError("quantize_q8_0: weights must be bf16")
        rows, n_in = self._q8("quantize_q8_0", qs, d, w)
        self._check(self.lib.mg_quantize_q8_0(self.h, _ptr(w), rows, n_in, _ptr(qs), _ptr(d)))

    def gemv_q8_0(self, qs, d, x, y, blockdot=False):
        """y[b, o] = sum_i W[o, i] x[b, i] over a Q8_0 weight (k_gemv_q8); x bf16 [B, in], y f32 [B, rows]."""
        rows, n_in = self._q8("gemv_q8_0", qs, d, None)
        self._dev(x, y)
        ldx, ldy = self._rows("gemv_q8_0", x), self._rows("gemv_q8_0", y)
        B = x.shape[0]
        if x.shape[1] != n_in or tuple(y.shape) != (B, rows):
            raise MgError(f"gemv_q8_0: x must be [B, {n_in}] and y [B, {rows}]")
        self._check(self.lib.mg_gemv_q8_0(self.h, _ptr(qs), _ptr(d), _ptr(x), B, rows, n_in, ldx, _ptr(y), ldy,
                                          int(blockdot)))

    # -------------------------------------------------------------- vocab
    def _vocab_outs(self, name, rows, K, lse, argmax, top_idx, top_val):
        import torch
        self._dev(lse, argmax, top_idx, top_val)
        self._contig(name, lse, argmax, top_idx, top_val)
        for t, dt, n in ((lse, torch.float64, rows), (argmax, torch.int64, rows), (top_idx, torch.int64, rows * K),
                         (top_val, torch.float32, rows * K)):
            if t is not None and t.dtype != dt:
                raise MgError(f"{name}: output of dtype {t.dtype}, {dt} needed")
            self._numel(name, t, n)

    def vocab_reduce(self, logits, K, lse=None, argmax=None, top_idx=None, top_val=None):
        """Per row: logsumexp, first argmax, top-K (value desc, index asc)."""
        import torch
        self._dev(logits)
        ld = self._rows("vocab_reduce", logits)
        rows, V = logits.shape
        dev = logits.device
        if lse is None:
            lse = torch.empty(rows, dtype=torch.float64, device=dev)
        if argmax is None:
            argmax = torch.empty(rows, dtype=torch.int64, device=dev)
        if K > 0 and top_idx is None:
            top_idx = torch.empty((rows, K), dtype=torch.int64, device=dev)
        if K > 0 and top_val is None:
            top_val = torch.empty((rows, K), dtype=torch.float32, device=dev)
        self._vocab_outs("vocab_reduce", rows, K, lse, argmax, top_idx, top_val)
        self._check(self.lib.mg_vocab_reduce(self.h, _ptr(logits), ld, rows, V, _dtype_code(logits), K, _ptr(lse),
                                             _ptr(argmax), _ptr(top_idx) if K > 0 else None,
                                             _ptr(top_val) if K > 0 else None))
        return lse, argmax, top_idx, top_val

    def vocab_reduce_noalloc(self, logits, K, lse, argmax, top_idx, top_val, stream=None):
        """vocab_reduce through mg_vocab_reduce_noalloc: no context workspace, the
        library's fixed scratch array instead; outputs must be given (nothing is
        allocated). `stream` defaults to this context's stream."""
        self._dev(logits)
        ld = self._rows("vocab_reduce_noalloc", logits)
        rows, V = logits.shape
        self._vocab_outs("vocab_reduce_noalloc", rows, K, lse, argmax, top_idx, top_val)
        s = self.stream() if stream is None else stream
        rc = self.lib.mg_vocab_reduce_noalloc(ctypes.c_void_p(s), _ptr(logits), ld, rows, V, _dtype_code(logits), K,
                                              _ptr(lse), _ptr(argmax), _ptr(top_idx), _ptr(top_val))
        self._check(rc)

    PROBE_COPY, PROBE_READ, PROBE_WRITE, PROBE_2R2W = 0, 1, 2, 3
    PROBE_COPY_CACHED, PROBE_COPY_4VEC, PROBE_COPY_PERSISTENT = 4, 5, 6

    def probe_stream(self, kind, a=None, b=None, c=None, d=None):
        """HBM stream probe (a measurement aid, no reference counterpart): kind
        PROBE_COPY b = a, PROBE_READ reads a (b: a sink of >= 4 bytes),
        PROBE_WRITE fills b, PROBE_2R2W a = a + c and d = (a + c) ^ c over
        32-bit words; PROBE_COPY_CACHED, PROBE_COPY_4VEC and
        PROBE_COPY_PERSISTENT copy a to b in other forms. The moved size is the first operand's byte count; the
        others must hold as many bytes (contiguous, 16-byte aligned)."""
        ts = [t for t in (a, b, c, d) if t is not None]
        self._dev(*ts)
        self._contig("probe_stream", *ts)
        first = a if kind != self.PROBE_WRITE else b
        if first is None:
            raise MgError("probe_stream: missing operand")
        nbytes = first.numel() * first.element_size()
        for t in ts:
            if t is not b or kind != self.PROBE_READ:
                if t.numel() * t.element_size() < nbytes:
                    raise MgError("probe_stream: operands smaller than the moved size")
        self._check(self.lib.mg_probe_stream(self.h, kind, _ptr(a), _ptr(b), _ptr(c), _ptr(d), nbytes))

    def sample_dist(self, top_idx, top_val, argmax, temperature, top_p, min_p, ids=None, probs=None, n=None,
                    raw_argmax=None):
        """serve/sampler.py's candidate distribution (ids, probs, count per row) from a vocab pass
        over the edited logits; raw_argmax (the raw logits' argmax, for the fully masked fallback)
        defaults to argmax. Row r's first n[r] slots hold its candidates; the slots after them are
        not written."""
        import torch
        self._dev(top_idx, top_val, argmax, raw_argmax)
        self._contig("sample_dist", top_idx, top_val, argmax, raw_argmax)
        rows, K = top_idx.shape
        dev = top_idx.device
        ids = torch.empty((rows, K), dtype=torch.int64, device=dev) if ids is None else ids
        probs = torch.empty((rows, K), dtype=torch.float32, device=dev) if probs is None else probs
        n = torch.empty(rows, dtype=torch.int64, device=dev) if n is None else n
        self._dev(ids, probs, n)
        self._contig("sample_dist", ids, probs, n)
        for t in (top_val, ids, probs):
            self._numel("sample_dist", t, rows * K)
        for t in (argmax, n, raw_argmax):
            if t is not None:
                self._numel("sample_dist", t, rows)
        self._check(self.lib.mg_sample_dist(self.h, _ptr(top_idx), _ptr(top_val), _ptr(argmax), _ptr(raw_argmax),
                                            rows, K, temperature, top_p, min_p, _ptr(ids), _ptr(probs), _ptr(n)))
        return ids, probs, n

    # ------------------------------------------------------------- .npy
    def load_npy(self, path, dtype=None):
        """load_npy (src/tensor.cpp:91-224) into a new device tensor of the file's shape:
        values widened to f64 as there, stored at dtype (torch.float64 by default, or
        float32 / bfloat16 / float16 with the twin's rounding)"""
        import torch
        dtype = torch.float64 if dtype is None else dtype
        _, shape = npy_info(path)
        t = torch.empty(shape, dtype=dtype, device=f"cuda:{self.device}")
        self._check(self.lib.mg_npy_load(self.h, os.fsencode(path), _ptr(t), t.numel(), _dtype_code(t)))
        return t

    def save_npy(self, path, t):
        """save_npy (src/tensor.cpp:62-76): a device tensor written as '<f8' of its shape"""
        self._dev(t)
        self._contig("save_npy", t)
        shape = (ctypes.c_int64 * max(1, t.dim()))(*t.shape)
        self._check(self.lib.mg_npy_save(self.h, os.fsencode(path), _ptr(t), _dtype_code(t),
                                         ctypes.cast(shape, _P), t.dim()))

    def save_npy_i64(self, path, t):
        """save_npy_i64 (src/tensor.cpp:78-89): an int64 device vector as a 1-d '<i8' file"""
        import torch
        self._dev(t)
        self._contig("save_npy_i64", t)
        if t.dtype != torch.int64:
            raise MgError("save_npy_i64: an int64 tensor is needed")
        self._check(self.lib.mg_npy_save_i64(self.h, os.fsencode(path), _ptr(t), t.numel()))

    def sample_rows(self, logits, top_k, temperature, top_p, min_p, raw_argmax=None):
        """Sampler._transformed (serve/sampler.py:43-112) on full rows of edited f32 logits, any
        top_k: (ids [rows, V], probs [rows, V], n [rows]); row r's first n[r] slots hold its
        candidates (value order when top_k > 0 or top_p < 1, else index order); n[r] = -1 marks
        a row left to the host (more than 4096 sorted candidates, or +inf logits)."""
        import torch
        self._dev(logits, raw_argmax)
        ld = self._rows("sample_rows", logits)
        if logits.dtype != torch.float32:
            raise MgError("sample_rows: logits must be float32")
        rows, V = logits.shape
        self._contig("sample_rows", raw_argmax)
        if raw_argmax is not None:
            self._numel("sample_rows", raw_argmax, rows)
        dev = logits.device
        ids = torch.empty((rows, V), dtype=torch.int64, device=dev)
        probs = torch.empty((rows, V), dtype=torch.float32, device=dev)
        n = torch.empty(rows, dtype=torch.int64, device=dev)
        self._check(self.lib.mg_sample_rows(self.h, _ptr(logits), ld, rows, V, _ptr(raw_argmax), top_k, temperature,
                                            top_p, min_p, _ptr(ids), _ptr(probs), _ptr(n)))
        return ids, probs, n

    def vocab_reduce_tail(self, logits, mult, cap, K, logits_out=None):
        """apply_output_tail (src/muse_glimmer.hpp:920-943) fused into the vocab pass:
        lse / first argmax / top-K over the transformed logits; logits_out, when given,
        receives them (the input is left as it is)."""
        import torch
        self._dev(logits, logits_out)
        ld = self._rows("vocab_reduce_tail", logits)
        self._contig("vocab_reduce_tail", logits_out)
        self._same("vocab_reduce_tail", logits, logits_out)
        rows, V = logits.shape
        self._numel("vocab_reduce_tail logits_out", logits_out, rows * V)
        dev = logits.device
        lse = torch.empty(rows, dtype=torch.float64, device=dev)
        argmax = torch.empty(rows, dtype=torch.int64, device=dev)
        top_idx = torch.empty((rows, K), dtype=torch.int64, device=dev)
        top_val = torch.empty((rows, K), dtype=torch.float32, device=dev)
        self._check(self.lib.mg_vocab_reduce_tail(self.h, _ptr(logits), ld, rows, V, _dtype_code(logits), mult, cap, K,
                                                  _ptr(lse), _ptr(argmax), _ptr(top_idx), _ptr(top_val),
                                                  _ptr(logits_out)))
        return lse, argmax, top_idx, top_val
