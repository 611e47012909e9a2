"""Brute-force sampler for tiny inputs, written independently of the C oracle: Python lists,
a full sort with Python's sort, math.exp and math.fsum. Used to pin the oracle.

The contract it implements: z = fl32(x * fl32(1/T)); penalties per distinct history id
(repetition: z * fl32(1/rp) if z > 0 else z * rp; then minus count * fp + pp, fp32);
allow-mask bit (t & 31) of word t >> 5; rank by z descending, id ascending; top-k, top-p
(shortest prefix with cumulative >= top_p), min-p (exp(z - zmax) >= min_p); draw: the
first kept id in ascending id order whose cumulative probability exceeds u.
"""
from __future__ import annotations

import math
from collections import Counter

import numpy as np

F = np.float32


def bf16_to_f32(h: int) -> float:
    return float(np.array([h << 16], dtype=np.uint32).view(np.float32)[0])


def tempered(params, x_row, hist_row, mask_row):
    V = params.vocab
    inv_t = F(1.0) / F(params.temperature)
    xs = [bf16_to_f32(int(v)) for v in x_row[:V]] if params.dtype == 1 else [float(v) for v in x_row[:V]]
    z = [F(F(v) * inv_t) + F(0.0) for v in xs]
    if hist_row is not None and params.hist_len > 0:
        ids = [int(t) for t in hist_row[: params.hist_len] if int(t) >= 0]
        if any(t >= V for t in ids):
            return -3, None
        rp = F(params.repetition_penalty)
        inv_rp = F(1.0) / rp
        for t, c in Counter(ids).items():
            v = z[t]
            v = F(v * inv_rp) if v > 0 else F(v * rp)
            pen = F(F(F(c) * F(params.frequency_penalty)) + F(params.presence_penalty))
            z[t] = F(v - pen) + F(0.0)
    if mask_row is not None:
        for t in range(V):
            if not (int(mask_row[t >> 5]) >> (t & 31)) & 1:
                z[t] = F(-np.inf)
    if any(math.isnan(v) or v == math.inf for v in z):
        return -2, None
    return 0, z


def sample_row(params, x_row, hist_row, mask_row, u: float, tol: float = 1e-6):
    """(id, kept ids, probability of each kept id, ambiguous) for one row. `ambiguous` is
    True when the outcome is within `tol` of a decision (CDF step, top-p or min-p cut)."""
    st, z = tempered(params, x_row, hist_row, mask_row)
    if st != 0:
        return st, [], {}, False
    finite = [(float(v), i) for i, v in enumerate(z) if v != -math.inf]
    if not finite:
        return -1, [], {}, False
    order = sorted(finite, key=lambda p: (-p[0], p[1]))
    k = params.top_k
    n = k if 0 < k < len(order) else len(order)
    top = order[:n]
    zmax = top[0][0]
    e = [math.exp(v - zmax) for v, _ in top]
    ek = math.fsum(e)
    ambiguous = False
    lp = n
    if params.top_p < 1.0:
        tp = float(F(params.top_p))
        for j in range(n):
            frac = math.fsum(e[: j + 1]) / ek
            if abs(frac - tp) < tol:
                ambiguous = True
            if frac >= tp:
                lp = j + 1
                break
    kept_n = lp
    if params.min_p > 0.0:
        mp = float(F(params.min_p))
        kept_n = sum(1 for j in range(lp) if e[j] >= mp)
        if any(abs(e[j] / mp - 1.0) < tol for j in range(lp)):
            ambiguous = True
    kept = sorted((top[j][1], e[j]) for j in range(kept_n))
    E = math.fsum(w for _, w in kept)
    probs = {i: w / E for i, w in kept}
    cum = 0.0
    pick = kept[-1][0]
    found = False
    acc = []
    for i, w in kept:
        acc.append(w)
        c = math.fsum(acc) / E
        if abs(c - u) < tol:
            ambiguous = True
        if not found and c > u:
            pick, found = i, True
    return pick, [i for i, _ in kept], probs, ambiguous
