#!/usr/bin/env python3
"""Benchmark of the MI355X non-GEMM primitives at BASELINE.json's 30B-class shapes.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--reps R] [--no-cpu] [--only OP]

A step is one pass of the three headline primitives over their BASELINE
configs, inputs resident in HBM:
  residual-add + RMSNorm   bf16 [4096, 5120] (+ w [5120]), eps 1e-6      configs[1]
  SwiGLU                   bf16 gate/up [4096, 25600]                     configs[2]
  causal row softmax       f32 scores [40, 2048, 2048] -> bf16, 1/sqrt(128) configs[3]
`value` is the whole step's algorithmic HBM bytes (each tensor read or written
once) divided by the measured step time, in GB/s. Every other primitive
(RoPE, decode softmax, Q8_0 dequant, quantizer and GEMV, vocab lse/argmax/
top-64 with and without the output tail and the sampler distribution, the
fused QK op, decode and prefill attention, decode-shape RMSNorm) is timed on
its own under "ops". Inputs are seeded synthetic data
drawn with torch's generator on the device (N(0,1) activations, N(1,0.05)
weights, N(0,3) scores, U{-127..127} quants, U[1e-3,2e-2] f16 scales, N(0,4)
logits). Per-op times are the median of R launches bracketed by HIP events on
the launch stream, with a 512 MiB buffer rewritten before each launch so no op
is served from the 256 MiB Infinity Cache. Each single launch so timed carries
the protocol's own floor (`launch_floor`, a few us), so every op also reports
`us_in_stream`: R (rewrite, op) pairs against R rewrites alone, both as one
bracketed sequence, the difference divided by R, i.e. the op's kernels and the
gaps between launches inside a stream of work, with the same HBM-resident inputs.

`cpu_baseline` times the CPU restatement of the reference's own tensor path
(oracle/liboracle.so: f64 twin arithmetic with OpenMP over rows, as
src/muse_glimmer.hpp runs it) on a bounded sample (1/8 of the rows) of every
BASELINE op, and reports the step's three in the same unit as `value`.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "muse-glimmer-intel-serve_amd")
sys.path.insert(0, PKG)

METRIC = "achieved HBM GB/s (% of 8 TB/s) + us/op for RMSNorm/SwiGLU/softmax, 30B shapes"
PEAK_GBPS = 8000.0

T, D = 4096, 5120
FFN = 25600
SM_H, SM_Q, SM_K = 40, 2048, 2048
DEC_K = 131072
Q_H, K_H, HD = 40, 8, 128
Q8_R, Q8_C = 25600, 5120
V_ROWS, VOCAB, TOPK = 64, 201088, 64

# algorithmic bytes: every input read once, every output written once
BYTES = {
    "residual_rmsnorm": 4 * 2 * T * D + 2 * D,
    "swiglu": 3 * 2 * T * FFN,
    "softmax_causal": SM_H * (SM_Q * (SM_Q + 1) // 2) * 4 + SM_H * SM_Q * SM_K * 2,
    "rope": 2 * 2 * (T * Q_H * HD + T * K_H * HD) + 2 * 2 * T * (HD // 2),
    "softmax_decode": SM_H * DEC_K * (4 + 2),
    "dequant_q8_0": Q8_R * Q8_C + Q8_R * (Q8_C // 32) * 2 + Q8_R * Q8_C * 2,
    "vocab_lse_argmax_top64": V_ROWS * VOCAB * 4 + V_ROWS * (8 + 8) + V_ROWS * TOPK * (8 + 4),
    "vocab_tail_top64_dist": V_ROWS * VOCAB * 4 + V_ROWS * (8 + 8) + V_ROWS * TOPK * (8 + 4) * 2,
    "quantize_q8_0": Q8_R * Q8_C * 2 + Q8_R * Q8_C + Q8_R * (Q8_C // 32) * 2,
    "gemv_q8_0_decode": Q8_R * Q8_C + Q8_R * (Q8_C // 32) * 2 + Q8_C * 2 + Q8_R * 4,
    "attn_decode_131072": 2 * DEC_K * K_H * HD * 2 + Q_H * HD * 2 + Q_H * HD * 4,
    # q, k read + written, v read, k/v cache rows written, cos/sin read
    "qk_norm_rope_kv": 2 * (2 * T * Q_H * HD + 2 * T * K_H * HD) + 2 * T * K_H * HD + 2 * 2 * T * K_H * HD
                       + 2 * 2 * T * (HD // 2),
    # q and the K/V ring read, f32 out written (the op is bound by the matrix cores: FLOPS)
    "attn_prefill_4096": 2 * T * Q_H * HD + 2 * 2 * T * K_H * HD + 4 * T * Q_H * HD,
    # the embedding norm in place: f32 rows [4096, 5120] read, bf16-valued f32 written back
    "norm_rows_f32_embed": 2 * 4 * T * D,
    # the sampler's whole chain on full rows (top_k <= 0, top_p 0.95): the logits read once
    # (the selections re-read them from the caches) + the candidate lists (at most 4096 per row)
    "sample_rows_topk0": V_ROWS * VOCAB * 4,
    # a plain device copy (torch's copy kernel): the access-pattern ceiling the others are read against
    "copy_256MiB": 2 * (256 << 20),
    # one 4-byte fill (torch's fill kernel): what the timing protocol itself costs for any single launch
    "launch_floor": 4,
    # the library's stream probes (mg_probe_stream): the primitives' access pattern with no arithmetic
    "probe_copy_256MiB": 2 * (256 << 20),
    "probe_read_256MiB": 256 << 20,
    "probe_write_256MiB": 256 << 20,
    "probe_2r2w_norm_shape": 4 * 2 * T * D,
    # other forms of the same copy, to compare the primitives' pattern against
    "probe_copy_cached_256MiB": 2 * (256 << 20),
    "probe_copy_4vec_256MiB": 2 * (256 << 20),
    "probe_copy_persistent_256MiB": 2 * (256 << 20),
}
BYTES["softmax_causal_softcap30"] = BYTES["softmax_causal"]
# size-matched probes: an op's own byte count moved by the probe's pattern (a copy moves half
# the bytes each way), so small ops are read against a ceiling with the same fixed costs
SIZED_PROBES = {"probe_copy_rope_size": ("rope", "copy"), "probe_copy_qk_size": ("qk_norm_rope_kv", "copy"),
                "probe_read_vocab_size": ("vocab_lse_argmax_top64", "read"),
                "probe_read_gemv_size": ("gemv_q8_0_decode", "read")}
for _p, (_op, _kind) in SIZED_PROBES.items():
    BYTES[_p] = BYTES[_op] // 32 * 32 if _kind == "copy" else BYTES[_op] // 16 * 16
# matrix-core ops: q.k and p.v over the causal pairs, 2 * 2 * head_dim flops per (query, key)
FLOPS = {"attn_prefill_4096": Q_H * (T * (T + 1) // 2) * 4 * HD}
PEAK_TFLOPS = 2500.0  # dense bf16 MFMA
STEP_OPS = ("residual_rmsnorm", "swiglu", "softmax_causal")
KERNEL_OF = {
    # the step ops name their kernel as the traffic summary does (template arguments included)
    "residual_rmsnorm": "k_norm_row<mg::SBf16,2,true,true,true>",
    "swiglu": "k_gate_lut<mg::SBf16>",
    "softmax_causal": "k_softmax_fast<mg::SBf16,4,false,true>",
    "rope": "k_rope",
    "softmax_decode": "k_softmax_partial_buf + k_softmax_finish_buf",
    "dequant_q8_0": "k_dequant_q8_0_wide<mg::SBf16>",
    "vocab_lse_argmax_top64": "k_vocab_chunk + k_vocab_merge",
    "qk_norm_rope_kv": "k_qk_pairs",
    "quantize_q8_0": "k_quantize_q8_0",
    "attn_decode_131072": "k_attn_split<5,4> + k_attn_combine",
    "gemv_q8_0_decode": "k_gemv_q8_0<1>",
    "vocab_tail_top64_dist": "k_vocab_chunk<tail> + k_vocab_merge<tail> + k_sample_dist",
    "attn_prefill_4096": "k_attn_prefill<5,4,4,8,2>",
    "softmax_causal_softcap30": "k_softmax_fast<cap>",
    "norm_rows_f32_embed": "k_norm_f32rows",
    "sample_rows_topk0": "k_sample_split_stats + decide + gather + finish",
    "copy_256MiB": "torch copy (memory-only probe)",
    "launch_floor": "torch fill of one float (timing-protocol probe)",
    "probe_copy_256MiB": "k_probe<0> (copy)",
    "probe_read_256MiB": "k_probe<1> (read)",
    "probe_write_256MiB": "k_probe<2> (write)",
    "probe_2r2w_norm_shape": "k_probe<3> (2 reads + 2 writes, the residual_rmsnorm traffic)",
    "probe_copy_cached_256MiB": "k_probe<4> (copy, ordinary cached accesses)",
    "probe_copy_4vec_256MiB": "k_probe_4vec (copy, four 16-byte words a thread)",
    "probe_copy_persistent_256MiB": "k_probe_persist (copy, persistent grid of 2048 work-groups)",
}
for _p, (_op, _kind) in SIZED_PROBES.items():
    KERNEL_OF[_p] = f"k_probe<{0 if _kind == 'copy' else 1}> ({_kind}, {_op}'s bytes)"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--reps", type=int, default=20, help="launches per op for the per-op medians")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", default=None,
                    help="comma-separated ops to run --steps times each, with the cache flush before every "
                         "launch (for profilers); 'copy' is the plain 256 MiB device copy (counter calibration)")
    ap.add_argument("--cpu-seconds", type=float, default=3.0, help="CPU time per op in the CPU baseline")
    ap.add_argument("--traffic", default=os.path.join(ROOT, "profiles", "pmc_traffic.txt"),
                    help="measured HBM bytes per launch (kernel  fetch_bytes  write_bytes)")
    return ap.parse_args()


def make_inputs(torch, P):
    import mgprims as M
    dev = "cuda:0"
    g = torch.Generator(device=dev)
    g.manual_seed(20261201)
    bf = torch.bfloat16

    def randn(shape, mean=0.0, std=1.0, dtype=bf):
        return (torch.randn(shape, generator=g, device=dev, dtype=torch.float32) * std + mean).to(dtype)

    I = {}
    I["h"] = randn((T, D))
    I["x"] = randn((T, D))
    I["w"] = randn((D,), 1.0, 0.05)
    I["y"] = torch.empty((T, D), dtype=bf, device=dev)
    I["gate"] = randn((T, FFN))
    I["up"] = randn((T, FFN))
    I["act"] = torch.empty((T, FFN), dtype=bf, device=dev)
    I["scores"] = randn((SM_H, SM_Q, SM_K), 0.0, 3.0, torch.float32)
    I["probs"] = torch.empty((SM_H, SM_Q, SM_K), dtype=bf, device=dev)
    I["q"] = randn((T, Q_H, HD))
    I["k"] = randn((T, K_H, HD))
    I["cos"], I["sin"] = P.build_rope_table(1e6, HD, T, bf)
    I["dscores"] = randn((SM_H, 1, DEC_K), 0.0, 3.0, torch.float32)
    I["dprobs"] = torch.empty((SM_H, 1, DEC_K), dtype=bf, device=dev)
    I["qs"] = torch.randint(-127, 128, (Q8_R, Q8_C), generator=g, device=dev, dtype=torch.int8)
    I["qd"] = (torch.rand((Q8_R, Q8_C // 32), generator=g, device=dev) * (2e-2 - 1e-3) + 1e-3).to(torch.float16)
    I["deq"] = torch.empty((Q8_R, Q8_C), dtype=bf, device=dev)
    I["logits"] = randn((V_ROWS, VOCAB), 0.0, 4.0, torch.float32)
    I["lse"] = torch.empty(V_ROWS, dtype=torch.float64, device=dev)
    I["amax"] = torch.empty(V_ROWS, dtype=torch.int64, device=dev)
    I["tidx"] = torch.empty((V_ROWS, TOPK), dtype=torch.int64, device=dev)
    I["tval"] = torch.empty((V_ROWS, TOPK), dtype=torch.float32, device=dev)
    I["wq"] = randn((Q8_R, Q8_C), 0.0, 0.05)
    I["qs2"] = torch.empty((Q8_R, Q8_C), dtype=torch.int8, device=dev)
    I["qd2"] = torch.empty((Q8_R, Q8_C // 32), dtype=torch.int16, device=dev)
    I["xg"] = randn((1, Q8_C))
    I["yg"] = torch.empty((1, Q8_R), dtype=torch.float32, device=dev)
    I["qd1"] = randn((Q_H, HD))
    I["kring"] = randn((DEC_K, K_H, HD))
    I["vring"] = randn((DEC_K, K_H, HD))
    I["attn_out"] = torch.empty((Q_H, HD), dtype=torch.float32, device=dev)
    I["v"] = randn((T, K_H, HD))
    I["kcache"] = torch.empty((T, K_H, HD), dtype=bf, device=dev)
    I["vcache"] = torch.empty((T, K_H, HD), dtype=bf, device=dev)
    I["hdec"] = randn((64, D))
    I["xdec"] = randn((64, D))
    I["ydec"] = torch.empty((64, D), dtype=bf, device=dev)
    I["pk"] = randn((T, K_H, HD))
    I["pv"] = randn((T, K_H, HD))
    I["pout"] = torch.empty((T, Q_H, HD), dtype=torch.float32, device=dev)
    I["hf32"] = randn((T, D), 0.0, 1.0, torch.float32)
    I["copy_src"] = torch.ones(256 << 20, dtype=torch.uint8, device=dev)
    I["copy_dst"] = torch.empty_like(I["copy_src"])
    I["one"] = torch.empty(1, dtype=torch.float32, device=dev)
    for name in ("pa", "pc", "pd"):  # the norm-shaped probe's own [T, D] bf16 buffers
        I[name] = torch.zeros((T, D), dtype=bf, device=dev)
    torch.cuda.synchronize()

    scale = 1.0 / math.sqrt(HD)

    def tail_dist():
        # output tail (cap 30) fused into the vocab pass, then the sampler's distribution
        _, am, ti, tv = P.vocab_reduce_tail(I["logits"], 1.0, 30.0, TOPK)
        return P.sample_dist(ti, tv, am, 0.7, 0.95, 0.0)

    ops = {
        "residual_rmsnorm": lambda: P.residual_rmsnorm(M.PLAIN, I["h"], I["x"], I["w"], 1e-6, I["y"]),
        "swiglu": lambda: P.swiglu(I["gate"], I["up"], I["act"]),
        "softmax_causal": lambda: P.softmax_rows(I["scores"], I["probs"], scale, M.MASK_CAUSAL),
        "softmax_causal_softcap30": lambda: P.softmax_rows(I["scores"], I["probs"], scale, M.MASK_CAUSAL, 0, 0,
                                                           30.0),
        "rope": lambda: P.apply_rope(I["q"], I["k"], I["cos"], I["sin"]),
        "softmax_decode": lambda: P.softmax_rows(I["dscores"], I["dprobs"], scale, M.MASK_CAUSAL, 0, DEC_K - 1),
        "dequant_q8_0": lambda: P.dequant_q8_0(I["qs"], I["qd"], I["deq"]),
        "vocab_lse_argmax_top64": lambda: P.vocab_reduce(I["logits"], TOPK, I["lse"], I["amax"], I["tidx"], I["tval"]),
        "vocab_tail_top64_dist": lambda: tail_dist(),
        "quantize_q8_0": lambda: P.quantize_q8_0(I["wq"], I["qs2"], I["qd2"]),
        "attn_decode_131072": lambda: P.attn_decode(I["qd1"], I["kring"], I["vring"], DEC_K - 1, scale, 0, I["attn_out"]),
        "gemv_q8_0_decode": lambda: P.gemv_q8_0(I["qs"], I["qd"], I["xg"], I["yg"]),
        "attn_prefill_4096": lambda: P.attn_prefill(I["q"], I["pk"], I["pv"], 0, scale, 0, I["pout"]),
        "qk_norm_rope_kv": lambda: P.qk_norm_rope(I["q"], I["k"], 1e-6, 3.87, I["cos"], I["sin"], None, 0, I["v"],
                                                  I["kcache"], I["vcache"]),
        "norm_rows_f32_embed": lambda: P.norm_rows_mixed(M.WEIGHTLESS, I["hf32"], None, 1e-6, I["hf32"],
                                                         bf16_as_f32=True),
        "sample_rows_topk0": lambda: P.sample_rows(I["logits"], 0, 1.0, 0.95, 0.0),
        "copy_256MiB": lambda: I["copy_dst"].copy_(I["copy_src"]),
        "launch_floor": lambda: I["one"].zero_(),
        "probe_copy_256MiB": lambda: P.probe_stream(P.PROBE_COPY, I["copy_src"], I["copy_dst"]),
        "probe_read_256MiB": lambda: P.probe_stream(P.PROBE_READ, I["copy_src"], I["one"]),
        "probe_write_256MiB": lambda: P.probe_stream(P.PROBE_WRITE, None, I["copy_dst"]),
        "probe_2r2w_norm_shape": lambda: P.probe_stream(P.PROBE_2R2W, I["pa"], None, I["pc"], I["pd"]),
        "probe_copy_cached_256MiB": lambda: P.probe_stream(P.PROBE_COPY_CACHED, I["copy_src"], I["copy_dst"]),
        "probe_copy_4vec_256MiB": lambda: P.probe_stream(P.PROBE_COPY_4VEC, I["copy_src"], I["copy_dst"]),
        "probe_copy_persistent_256MiB": lambda: P.probe_stream(P.PROBE_COPY_PERSISTENT, I["copy_src"], I["copy_dst"]),
    }
    for name, (_op, kind) in SIZED_PROBES.items():
        if kind == "copy":
            n = BYTES[name] // 2
            ops[name] = (lambda n: lambda: P.probe_stream(P.PROBE_COPY, I["copy_src"][:n], I["copy_dst"][:n]))(n)
        else:
            n = BYTES[name]
            ops[name] = (lambda n: lambda: P.probe_stream(P.PROBE_READ, I["copy_src"][:n], I["one"]))(n)
    for t in (1, 4, 16, 64):
        ops[f"residual_rmsnorm_T{t}"] = (lambda t=t: P.residual_rmsnorm(
            M.PLAIN, I["hdec"][:t], I["xdec"][:t], I["w"], 1e-6, I["ydec"][:t]))
        BYTES[f"residual_rmsnorm_T{t}"] = 4 * 2 * t * D + 2 * D
        KERNEL_OF[f"residual_rmsnorm_T{t}"] = "k_norm_row"
    return ops


def time_op(torch, fn, reps, flush):
    stream = torch.cuda.current_stream()
    for _ in range(3):
        fn()
    times = []
    for _ in range(reps):
        flush.zero_()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        fn()
        b.record(stream)
        b.synchronize()
        times.append(a.elapsed_time(b) * 1e3)  # us
    return statistics.median(times), min(times)


def time_in_stream(torch, fn, reps, flush, rounds=11):
    """An op's cost inside a stream of work, free of the per-launch event floor:
    `reps` (flush, op) pairs and `reps` flushes alone, each sequence bracketed by
    one pair of HIP events; the difference over `reps` is the op's kernels plus
    the gaps between launches, with inputs in HBM as for the per-launch median.
    The median over `rounds` such differences, the two sequences' order
    alternating from round to round."""
    stream = torch.cuda.current_stream()
    diffs = []
    for k in range(rounds):
        spans = {}
        for with_op in ((False, True) if k % 2 == 0 else (True, False)):
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            a.record(stream)
            for _ in range(reps):
                flush.zero_()
                if with_op:
                    fn()
            b.record(stream)
            b.synchronize()
            spans[with_op] = a.elapsed_time(b) * 1e3
        diffs.append((spans[True] - spans[False]) / reps)
    return statistics.median(diffs)


def lib_digest():
    """sha256 of the libmgprims.so this process loads"""
    import hashlib
    import mgprims
    with open(mgprims.LIB_PATH, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()


def read_traffic(path, kernel):
    """Measured HBM bytes per launch for `kernel` from the rocprofv3 PMC summary:
    the line naming it exactly (template arguments included), else the one line
    whose name starts with it; None when absent or ambiguous, and None when the
    summary was measured on another build of the library than the one loaded
    (its '# library sha256:' line), so a kernel change never pairs new times
    with old counters."""
    rows = {}
    digest = None
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("# library sha256:"):
                    digest = line.split(":", 1)[1].strip()
                parts = line.split()
                if len(parts) >= 3 and not line.startswith("#"):
                    rows[parts[0]] = int(float(parts[1]) + float(parts[2]))
    except OSError:
        return None
    if digest != lib_digest():
        return None
    if kernel in rows:
        return rows[kernel]
    hits = [v for k, v in rows.items() if k.startswith(kernel + "<")]
    return hits[0] if len(hits) == 1 else None


def host_isa():
    """CPU model and the vector ISA the oracle was built for (oracle/Makefile)."""
    model = flags = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name") and not model:
                    model = line.split(":", 1)[1].strip()
                if line.startswith("flags") and not flags:
                    flags = line.split(":", 1)[1]
    except OSError:
        pass
    have = [x for x in ("avx2", "fma", "avx512f", "avx512_bf16") if f" {x}" in flags]
    return model, have


def cpu_baseline(seconds):
    """The reference's CPU tensor path (the oracle restatement, f64 twin arithmetic
    with OpenMP over rows / (token, head) pairs as src/muse_glimmer.hpp runs it, the
    k_dequant_q8 formula as a CPU loop, the host argmax / partial_sort / lse) on a
    bounded sample of every BASELINE op: 1/8 of the rows (heads, tokens) of each
    config, each run repeatedly for about `seconds`, timed without the Python
    wrappers' copies (the oracle's C entry points on preallocated arrays)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import oracle as O
    L = O.lib()
    p = O._p
    rn, rs, smh, rt, q8r, vr = T // 8, T // 8, SM_H // 8, T // 8, Q8_R // 8, V_ROWS // 8
    h = O.to_f64(O.normal(1, (rn, D), 0, 1, O.BF16), O.BF16)
    x = O.to_f64(O.normal(2, (rn, D), 0, 1, O.BF16), O.BF16)
    w = O.to_f64(O.normal(3, (D,), 1, 0.05, O.BF16), O.BF16)
    y = np.empty_like(h)
    gt = O.to_f64(O.normal(4, (rs, FFN), 0, 1, O.BF16), O.BF16)
    up = O.to_f64(O.normal(5, (rs, FFN), 0, 1, O.BF16), O.BF16)
    act = np.empty_like(gt)
    sc = O.to_f64(O.normal(8, (smh, SM_Q, SM_K), 0, 3, O.F32), O.F32)
    pr = np.empty_like(sc)
    qk = O.to_f64(O.normal(6, (rt, Q_H + K_H, HD), 0, 1, O.BF16), O.BF16)  # q and k heads of rt tokens
    co, si = O.rope_table(1e6, HD, rt, O.BF16)
    pos = np.arange(rt, dtype=np.int64)
    dsc = O.to_f64(O.normal(9, (smh, 1, DEC_K), 0, 3, O.F32), O.F32)
    dpr = np.empty_like(dsc)
    qs = O.int8_uniform(10, (q8r, Q8_C))
    qd = O.from_f64(O.uniform(11, (q8r, Q8_C // 32), 1e-3, 2e-2), O.F16)
    deq = np.empty((q8r, Q8_C))
    lg = O.to_f64(O.normal(12, (vr, VOCAB), 0, 4, O.F32), O.F32)
    lse, am = np.empty(vr), np.empty(vr, np.int64)
    ti, tv = np.empty((vr, TOPK), np.int64), np.empty((vr, TOPK))
    scale = 1 / math.sqrt(HD)
    hw = h.copy()
    fns = {
        "residual_rmsnorm": (lambda: L.or_residual_rmsnorm(O.PLAIN, p(hw), p(x), p(w), 1e-6, p(y), rn, D, O.BF16),
                             4 * 2 * rn * D + 2 * D, f"bf16-twin [{rn},{D}]"),
        "swiglu": (lambda: L.or_swiglu(p(gt), p(up), p(act), gt.size, O.BF16), 3 * 2 * rs * FFN,
                   f"bf16-twin [{rs},{FFN}]"),
        "softmax_causal": (lambda: L.or_softmax_rows(p(sc), p(pr), smh, SM_Q, SM_K, scale, O.MASK_CAUSAL, 0, 0, 0.0,
                                                     O.F32, O.BF16),
                           smh * (SM_Q * (SM_Q + 1) // 2) * 4 + smh * SM_Q * SM_K * 2, f"f32->bf16 [{smh},{SM_Q},{SM_K}]"),
        "rope": (lambda: L.or_apply_rope(p(qk), rt, Q_H + K_H, HD, (Q_H + K_H) * HD, p(co), p(si), p(pos), O.BF16),
                 2 * 2 * rt * (Q_H + K_H) * HD + 2 * 2 * rt * (HD // 2), f"bf16-twin q+k [{rt},{Q_H}+{K_H},{HD}]"),
        "softmax_decode": (lambda: L.or_softmax_rows(p(dsc), p(dpr), smh, 1, DEC_K, scale, O.MASK_CAUSAL, 0,
                                                     DEC_K - 1, 0.0, O.F32, O.BF16),
                           smh * DEC_K * (4 + 2), f"f32->bf16 [{smh},1,{DEC_K}]"),
        "dequant_q8_0": (lambda: L.or_dequant_q8_0(p(qs), p(qd), p(deq), q8r, Q8_C, O.BF16),
                         q8r * Q8_C * 3 + q8r * (Q8_C // 32) * 2, f"[{q8r},{Q8_C}] -> bf16"),
        "vocab_lse_argmax_top64": (lambda: L.or_vocab_reduce(p(lg), vr, VOCAB, TOPK, p(lse), p(am), p(ti), p(tv)),
                                   vr * VOCAB * 4 + vr * (8 + 8) + vr * TOPK * 12, f"f32 [{vr},{VOCAB}], K={TOPK}"),
    }
    per = {}
    step_b = step_s = 0.0
    for name, (fn, b, what) in fns.items():
        fn()
        reps = 0
        t0 = time.perf_counter()
        while reps < 3 or time.perf_counter() - t0 < seconds:
            fn()
            reps += 1
        dt = (time.perf_counter() - t0) / reps
        per[name] = {"us": round(dt * 1e6, 1), "GBps": round(b / dt / 1e9, 3), "reps": reps, "sample": what,
                     "bytes": b}
        if name in STEP_OPS:
            step_b += b
            step_s += dt
    model, isa = host_isa()
    del np
    return {
        "value": round(step_b / step_s / 1e9, 3),
        "unit": "GB/s",
        "cores": O.num_threads(),
        "kind": "port",
        "sample": (f"1/8 of each BASELINE config's rows (heads, tokens): {per['residual_rmsnorm']['sample']} "
                   f"residual+RMSNorm, {per['swiglu']['sample']} SwiGLU, causal softmax "
                   f"{per['softmax_causal']['sample']} (value = these three, the step); every op in `ops`; "
                   f"each repeated ~{seconds:g} s; f64 arrays as src/muse_glimmer.hpp holds them"),
        "threads": O.num_threads(),
        "nproc": os.cpu_count(),
        "cpu_model": model,
        "build": "g++ -O3 -ffp-contract=off -fno-math-errno -fopenmp -march=x86-64-v3 (oracle/Makefile)",
        "host_isa": isa,
        "ops": per,
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the primitives split across GPUs by rows, the vocab pass by shards with one small exchange)",
              file=sys.stderr)
        sys.exit(2)
    import torch
    import mgprims
    torch.cuda.set_device(0)
    P = mgprims.Prims(0)
    ops = make_inputs(torch, P)

    if args.only:
        flush = torch.empty(512 << 20, dtype=torch.uint8, device="cuda:0")
        ops["copy"] = ops["copy_256MiB"]
        for name in args.only.split(","):
            fn = ops[name]
            for _ in range(args.warmup):
                fn()
            times = []
            for _ in range(args.steps):
                flush.zero_()
                a = torch.cuda.Event(enable_timing=True)
                b = torch.cuda.Event(enable_timing=True)
                a.record()
                fn()
                b.record()
                b.synchronize()
                times.append(a.elapsed_time(b) * 1e3)
            print(json.dumps({"op": name, "us_median": round(statistics.median(times), 2)}), flush=True)
        return

    def step():
        for n in STEP_OPS:
            ops[n]()

    stream = torch.cuda.current_stream()
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(args.steps):
        step()
    b.record(stream)
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / args.steps
    step_bytes = sum(BYTES[n] for n in STEP_OPS)
    value = step_bytes / (ms * 1e-3) / 1e9
    print(f"# step: {ms * 1e3:.1f} us, {value:.1f} GB/s", file=sys.stderr, flush=True)

    flush = torch.empty(512 << 20, dtype=torch.uint8, device="cuda:0")
    per = {}
    for name, fn in ops.items():
        med, best = time_op(torch, fn, args.reps, flush)
        ins = time_in_stream(torch, fn, args.reps, flush)
        gbps = BYTES[name] / (med * 1e-6) / 1e9
        per[name] = {"us": round(med, 2), "us_min": round(best, 2), "bytes": BYTES[name],
                     "GBps": round(gbps, 1), "pct_peak": round(100 * gbps / PEAK_GBPS, 1),
                     "us_in_stream": round(ins, 2), "kernel": KERNEL_OF[name]}
        if name not in FLOPS and ins > 0:
            per[name]["GBps_in_stream"] = round(BYTES[name] / (ins * 1e-6) / 1e9, 1)
        if name in FLOPS:
            tf = FLOPS[name] / (med * 1e-6) / 1e12
            per[name].update({"flops": FLOPS[name], "TFLOPs": round(tf, 1), "bound": "mfma",
                              "pct_peak": round(100 * tf / PEAK_TFLOPS, 1)})
            print(f"# {name:28s} {med:9.2f} us  {tf:8.1f} TFLOP/s {100 * tf / PEAK_TFLOPS:5.1f} % of bf16 MFMA"
                  f"  (in stream {ins:8.2f} us)", file=sys.stderr, flush=True)
            continue
        print(f"# {name:28s} {med:9.2f} us  {gbps:8.1f} GB/s  {100 * gbps / PEAK_GBPS:5.1f} %"
              f"  (in stream {ins:8.2f} us)", file=sys.stderr, flush=True)

    dom = max(STEP_OPS, key=lambda n: per[n]["us"])
    kern = KERNEL_OF[dom]
    achieved = BYTES[dom] / (per[dom]["us"] * 1e-6) / 1e9
    roofline = {"bound": "hbm", "kernel": kern, "op": dom, "achieved": round(achieved, 1),
                "peak": PEAK_GBPS, "unit": "GB/s", "frac": round(achieved / PEAK_GBPS, 4),
                "traffic": read_traffic(args.traffic, kern), "algorithmic_bytes": BYTES[dom]}

    cpu = None if args.no_cpu else cpu_baseline(args.cpu_seconds)
    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded torch generator on device; BASELINE.json distributions)",
        "config": {"workload": "30B-class non-GEMM step: residual-add+RMSNorm bf16 [4096,5120] + "
                               "SwiGLU bf16 [4096,25600] + causal softmax f32->bf16 [40,2048,2048]",
                   "step_bytes": step_bytes, "pct_peak": round(100 * value / PEAK_GBPS, 1)},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "ops": per,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
