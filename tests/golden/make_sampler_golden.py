"""Write tests/golden/sampler.npz from the reference's own sampler.

    python tests/golden/make_sampler_golden.py

The filter chain's closed forms (tests/test_oracle_sampler.py) pin the
candidate set and probabilities everywhere except where a cut falls: the
reference decides top_p and min_p with numpy float32 arithmetic (its
cumulative sum and comparisons), which no closed form reproduces. So this
script runs the reference's Sampler._transformed (serve/sampler.py:43-112,
loaded from /root/reference by file path, in this container only) on seeded
rows and records, per row, the raw logits, the edited logits it returns (after
logit_bias, penalties and the mask), the raw logits' argmax, the parameters,
and its candidates, probabilities and kind. Rows whose top_p equals one of
their own float32 cumulative sums, or its neighbour, are marked `boundary`:
there the cut depends on the precision of the sum. The tests read only the
fixture; the reference never travels with it.
"""
import importlib.util
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REF = "/root/reference/serve/sampler.py"
V = 1536


def load_reference():
    spec = importlib.util.spec_from_file_location("ref_sampler", REF)
    mod = importlib.util.module_from_spec(spec)
    sys.modules["ref_sampler"] = mod  # its dataclasses look their module up here
    spec.loader.exec_module(mod)
    return mod


def main():
    S = load_reference()
    rng = np.random.default_rng(20261202)
    cases = []  # (raw logits, params dict, recent_ids, mask, boundary)

    def row(sigma):
        return (rng.normal(0.0, sigma, V)).astype(np.float32)

    base = dict(temperature=0.7, top_k=64, top_p=0.95, min_p=0.0)
    # the configuration the bench runs, and the K <= 256 device path
    for sigma in (4.0, 1.0):
        cases.append((row(sigma), dict(base), [], None, False))
    # top_k <= 0: every token; a nucleus longer than 256 at sigma 1
    for sigma in (1.0, 3.0):
        cases.append((row(sigma), dict(base, top_k=0, top_p=0.95, temperature=1.0), [], None, False))
    cases.append((row(2.0), dict(base, top_k=-1, top_p=0.5, temperature=1.3), [], None, False))
    # top_k <= 0 and top_p >= 1: index order, with and without min_p
    cases.append((row(2.0), dict(base, top_k=0, top_p=1.0, min_p=0.05, temperature=0.8), [], None, False))
    cases.append((row(1.0), dict(base, top_k=0, top_p=1.0, min_p=0.0, temperature=1.0), [], None, False))
    # top_k beyond 256, and beyond V
    cases.append((row(1.0), dict(base, top_k=1000, top_p=0.9, temperature=1.0), [], None, False))
    cases.append((row(2.0), dict(base, top_k=300, top_p=1.0, min_p=0.0, temperature=0.9), [], None, False))
    cases.append((row(1.0), dict(base, top_k=5000, top_p=1.0, min_p=0.01, temperature=1.0), [], None, False))
    # logit edits that move the argmax: a bias, penalties over recent ids, a mask
    r = row(3.0)
    top = int(np.argmax(r))
    cases.append((r, dict(base, logit_bias={top: -50.0, 7: 20.0}), [], None, False))
    r = row(3.0)
    recent = [int(i) for i in np.argsort(-r)[:5]] * 2
    cases.append((r, dict(base, repeat_penalty=1.3, frequency_penalty=0.5, presence_penalty=0.2), recent, None,
                  False))
    r = row(3.0)
    m = np.ones(V, bool)
    m[np.argsort(-r)[:3]] = False
    cases.append((r, dict(base, top_k=0, top_p=0.9), [], m, False))
    # fully masked: the fallback on the raw logits' argmax, also under a bias
    r = row(2.0)
    cases.append((r, dict(base), [], np.zeros(V, bool), False))
    cases.append((row(2.0), dict(base, logit_bias={3: 100.0}), [], np.zeros(V, bool), False))
    # greedy on the edited logits
    r = row(2.0)
    cases.append((r, dict(base, temperature=0.0, logit_bias={int(np.argmin(r)): 1000.0}), [], None, False))
    # -inf entries in a kept-everything row
    r = row(2.0)
    r[::5] = -np.inf
    cases.append((r, dict(base, top_k=0, top_p=0.8, temperature=1.0), [], None, False))
    # top_p exactly at one of the row's own float32 cumulative sums, and the
    # next float above it: the cut's `>=` and the precision of the sum decide
    for j in (3, 40, 200):
        for nudge in (False, True):
            r = row(1.0)
            srt = np.sort(r)[::-1]
            e = np.exp(srt - srt.max())
            cs = np.cumsum(e / e.sum())
            tp = float(cs[j])
            if nudge:
                tp = float(np.nextafter(np.float32(tp), np.float32(2.0)))
            cases.append((r, dict(base, top_k=0, top_p=tp, temperature=1.0), [], None, True))
    # min_p exactly at a probability ratio
    r = row(1.0)
    srt = np.sort(r)[::-1]
    e = np.exp(srt - srt.max())
    p = e / e.sum()
    cases.append((r, dict(base, top_k=0, top_p=1.0, min_p=float(p[10] / p.max())), [], None, True))

    n = len(cases)
    raw = np.zeros((n, V), np.float32)
    edited = np.zeros((n, V), np.float32)
    raw_argmax = np.zeros(n, np.int64)
    params = np.zeros((n, 4), np.float64)  # temperature, top_k, top_p, min_p
    cand = np.full((n, V), -1, np.int64)
    probs = np.zeros((n, V), np.float32)
    count = np.zeros(n, np.int64)
    kind = np.zeros(n, np.int64)  # 0 dist, 1 greedy, 2 masked
    boundary = np.zeros(n, bool)
    for i, (lg, prm, recent, mask, bnd) in enumerate(cases):
        sp = S.SampleParams(**prm)
        lg_out, c, pr, k = S.Sampler(sp)._transformed(lg.copy(), recent, mask)
        raw[i] = lg
        edited[i] = lg_out
        raw_argmax[i] = int(np.argmax(lg))
        params[i] = (sp.temperature, sp.top_k, sp.top_p, sp.min_p)
        cand[i, :len(c)] = c
        probs[i, :len(pr)] = pr
        count[i] = len(c)
        kind[i] = {"dist": 0, "greedy": 1, "masked": 2}[k]
        boundary[i] = bnd
    np.savez_compressed(os.path.join(HERE, "sampler.npz"), raw=raw, edited=edited, raw_argmax=raw_argmax,
                        params=params, cand=cand, probs=probs, count=count, kind=kind, boundary=boundary)
    print("wrote sampler.npz:", n, "rows, counts", count.tolist())


if __name__ == "__main__":
    main()
