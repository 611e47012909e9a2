"""Checks that pin the CPU oracle to the sampling contract without trusting its code:
closed forms and known answers, a brute-force sampler written separately (brute.py),
invariants, and a stratified frequency test. Each check takes an oracle.Oracle and
returns a list of failure messages, so the same checks can also be run against planted
mistakes (test_oracle_pins.py) to show that each of them is caught."""
from __future__ import annotations

import math

import numpy as np

import brute
from arbornet_amd.sampling import SamplingParams

F = np.float32


def _one(orc, V, logits, u, hist=None, mask=None, **kw):
    B = logits.shape[0]
    p = SamplingParams.make(B, V, ld_logits=logits.shape[1], **kw)
    if hist is not None:
        p.hist_len = hist.shape[1]
    ids, info, probs = orc.sample(p, logits, hist, mask, np.asarray(u, np.float32), probs=True)
    return ids, info, probs


def check_temperature_reciprocal(orc):
    """z = x * fl32(1/T): the reference's scalar Divide is Multiply(1f / scalar)
    (ArborNet.Core/Backends/CpuBackend.cs:265). 3 * fl32(1/7) = 0.42857146 while
    fl32(3/7) = 0.42857143; 1 * fl32(1/3) = 0.33333334 as in the reference's
    TensorComprehensiveTests.cs:76 known answer."""
    p = SamplingParams.make(1, 4, temperature=7.0)
    st, z = orc.tempered_row(p, np.array([3.0, 1.0, -2.0, 0.0], np.float32), None, None)
    out = []
    if st != 0 or z[0] != np.float32(0.42857146) or z[0] == np.float32(3.0) / np.float32(7.0):
        out.append(f"temperature: 3 * (1/7) gave {z[0]!r}")
    p = SamplingParams.make(1, 1, temperature=3.0)
    st, z = orc.tempered_row(p, np.array([1.0], np.float32), None, None)
    if z[0] != np.float32(0.33333334):
        out.append(f"temperature: 1 * (1/3) gave {z[0]!r}")
    return out


def check_penalties_hand_computed(orc):
    """z = [2, -1, 0.5, 0], history [0, 0, 1, 3, -1], rp 2, fp 0.5, pp 0.25, T 1:
    id 0 (count 2): 2 / 2 - (2 * 0.5 + 0.25) = -0.25; id 1 (count 1): -1 * 2 - 0.75 = -2.75;
    id 2 untouched 0.5; id 3 (count 1): 0 * 2 - 0.75 = -0.75; the -1 is padding."""
    p = SamplingParams.make(1, 4, repetition_penalty=2.0, frequency_penalty=0.5, presence_penalty=0.25, hist_len=5)
    st, z = orc.tempered_row(p, np.array([2.0, -1.0, 0.5, 0.0], np.float32), np.array([0, 0, 1, 3, -1], np.int32),
                             None)
    want = np.array([-0.25, -2.75, 0.5, -0.75], np.float32)
    return [] if st == 0 and np.array_equal(z, want) else [f"penalties: got {z}, want {want}"]


def check_mask_bit_order(orc):
    """Only bit 3 of word 0 set: id 3 is the only allowed token whatever the logits."""
    x = np.array([[9.0, 8.0, 7.0, -5.0] + [3.0] * 36], np.float32)
    mask = np.array([[1 << 3, 0]], np.uint32)
    ids, _, _ = _one(orc, 40, x, [0.7], mask=mask)
    return [] if ids[0] == 3 else [f"mask: allowed id 3 only, drew {ids[0]}"]


def check_uniform_cdf_strict(orc):
    """Four equal logits: C = [0.25, 0.5, 0.75, 1] exactly; the draw is the first id whose
    C exceeds u (KMeans.cs:149 intent), so u = 0.25 draws id 1 and u = 0 draws id 0."""
    x = np.zeros((4, 4), np.float32)
    ids, _, _ = _one(orc, 4, x, [0.0, 0.25, 0.5, 0.9999])
    want = [0, 1, 2, 3]
    return [] if list(ids) == want else [f"cdf: u=(0, .25, .5, .9999) drew {list(ids)}, want {want}"]


def check_top_p_inclusive(orc):
    """Four equal logits, top_p = 0.5: the shortest prefix with mass >= 0.5 is 2 tokens
    (ids 0, 1), so u = 0.8 draws id 1 (a strict > would keep 3 tokens and draw id 2)."""
    x = np.zeros((1, 4), np.float32)
    ids, info, _ = _one(orc, 4, x, [0.8], top_p=0.5)
    return [] if ids[0] == 1 and info["n_kept"][0] == 2 else [f"top-p: drew {ids[0]} kept {info['n_kept'][0]}"]


def check_min_p_relative_to_max(orc):
    """p = [0.5, 0.3, 0.2] (logits ln p), min_p = 0.5: keep p >= 0.25 -> {0, 1},
    renormalised [0.625, 0.375]; u = 0.9 draws id 1."""
    x = np.log(np.array([[0.5, 0.3, 0.2]], np.float64)).astype(np.float32)
    ids, info, probs = _one(orc, 3, x, [0.9], min_p=0.5)
    out = []
    if ids[0] != 1 or info["n_kept"][0] != 2:
        out.append(f"min-p: drew {ids[0]} kept {info['n_kept'][0]}")
    elif abs(probs[0, 0] - 0.625) > 1e-6:
        out.append(f"min-p: q0 = {probs[0, 0]}")
    return out


def check_ties_lowest_id(orc):
    """Equal logits rank by ascending id: top-k 2 keeps ids 0 and 1; top-k 1 equals the
    first maximum, the rule of ArgMax (CpuBackend.cs:1044-1055) and numpy.argmax."""
    out = []
    x = np.zeros((1, 10), np.float32)
    _, info, probs = _one(orc, 10, x, [0.99], top_k=2)
    if not (probs[0, 0] > 0 and probs[0, 1] > 0 and probs[0, 2:].max() == 0):
        out.append(f"ties: top-k 2 kept {np.nonzero(probs[0])[0].tolist()}")
    rng = np.random.default_rng(3)
    xr = np.round(rng.standard_normal((16, 50)) * 2).astype(np.float32)  # many ties
    ids, _, _ = _one(orc, 50, xr, rng.random(16), top_k=1)
    want = np.argmax(xr, axis=1)
    if not np.array_equal(ids, want):
        out.append(f"ties: top-k 1 {ids.tolist()} != argmax {want.tolist()}")
    return out


def check_sentinels(orc):
    out = []
    x = np.zeros((3, 40), np.float32)
    x[1, 7] = np.nan
    mask = np.full((3, 2), 0xFFFFFFFF, np.uint32)
    mask[0, :] = 0
    hist = np.array([[1, 2], [3, 4], [5, 40]], np.int32)
    ids, _, _ = _one(orc, 40, x, [0.5, 0.5, 0.5], hist=hist, mask=mask, repetition_penalty=1.3)
    if list(ids) != [-1, -2, -3]:
        out.append(f"sentinels: {list(ids)}")
    return out


def check_brute_force(orc, cases: int = 40, seed: int = 11):
    """Random small rows against brute.py: ids equal unless either side calls the row
    ambiguous; kept sets and probabilities equal where neither does."""
    rng = np.random.default_rng(seed)
    out = []
    for c in range(cases):
        V = int(rng.choice([8, 37, 257, 1000]))
        B = 4
        H = int(rng.choice([0, 6, 40]))
        kw = dict(temperature=float(rng.choice([0.5, 0.7, 1.0, 1.9])),
                  top_k=int(rng.choice([0, 0, 1, 3, 17, 50])),
                  top_p=float(rng.choice([1.0, 1.0, 0.9, 0.5])),
                  min_p=float(rng.choice([0.0, 0.0, 0.05, 0.3])))
        if H:
            kw.update(repetition_penalty=float(rng.choice([1.0, 1.3, 0.8])),
                      frequency_penalty=float(rng.choice([0.0, 0.4, -0.2])),
                      presence_penalty=float(rng.choice([0.0, 0.3])))
        x = (rng.standard_normal((B, V)) * rng.choice([0.5, 2.0, 4.0])).astype(np.float32)
        if rng.random() < 0.3:
            x = np.round(x)
        hist = rng.integers(-1, V, size=(B, H), dtype=np.int32) if H else None
        mask = None
        if rng.random() < 0.3:
            bits = rng.random((B, V)) < 0.4
            mask = np.zeros((B, (V + 31) // 32), np.uint32)
            for b, t in zip(*np.nonzero(bits)):
                mask[b, t >> 5] |= np.uint32(1 << (t & 31))
        u = rng.random(B).astype(np.float32)
        ids, info, probs = _one(orc, V, x, u, hist=hist, mask=mask, **kw)
        p = SamplingParams.make(B, V, **kw)
        p.hist_len = H
        for b in range(B):
            bid, kept, bprob, amb = brute.sample_row(p, x[b], None if hist is None else hist[b],
                                                     None if mask is None else mask[b], float(u[b]))
            if amb:
                continue
            if bid != ids[b]:
                out.append(f"brute case {c} row {b}: oracle {ids[b]} brute {bid} ({kw}, V={V}, H={H})")
                continue
            if bid < 0:
                continue
            got = np.nonzero(probs[b])[0].tolist()
            if got != kept:
                out.append(f"brute case {c} row {b}: kept sets differ")
                continue
            for i in kept:
                if abs(probs[b, i] - bprob[i]) > 1e-6 * max(1.0, bprob[i]) + 1e-12:
                    out.append(f"brute case {c} row {b}: q[{i}] {probs[b, i]} vs {bprob[i]}")
                    break
    return out


def check_stratified_frequencies(orc):
    """N = 20000 uniforms (i + 0.5) / N on one distribution: each id is drawn N * q +- 1
    times, q from the closed-form softmax of the kept set."""
    V, N = 12, 20000
    rng = np.random.default_rng(5)
    row = (rng.standard_normal(V) * 1.5).astype(np.float32)
    x = np.repeat(row[None, :], N, axis=0)
    u = ((np.arange(N) + 0.5) / N).astype(np.float32)
    ids, _, _ = _one(orc, V, x, u, top_k=8, temperature=0.8)
    z = row.astype(np.float32) * (np.float32(1) / np.float32(0.8))
    keep = np.argsort(-z, kind="stable")[:8]
    e = np.exp(z[keep].astype(np.float64) - z[keep].max())
    q = np.zeros(V)
    q[keep] = e / e.sum()
    counts = np.bincount(ids, minlength=V)
    bad = np.abs(counts - N * q) > 1.0 + 1e-9
    return [] if not bad.any() else [f"frequencies: counts {counts.tolist()} vs {np.round(N * q, 1).tolist()}"]


def check_invariants(orc):
    """Adding an integer to every logit (T = 1) changes no probability; top-k keeps
    min(k, finite) tokens and every kept z >= every dropped z; top-p's kept mass reaches
    top_p and falls short of it without its last token."""
    out = []
    rng = np.random.default_rng(9)
    x = np.round(rng.standard_normal((8, 300)) * 64).astype(np.float32) / 16  # exact in fp32
    u = rng.random(8).astype(np.float32)
    a_ids, _, a_p = _one(orc, 300, x, u, top_k=40, top_p=0.9)
    b_ids, _, b_p = _one(orc, 300, x + 5, u, top_k=40, top_p=0.9)
    if not np.array_equal(a_ids, b_ids) or np.abs(a_p - b_p).max() > 1e-6:
        out.append("invariant: shifting logits changed the result")
    _, info, probs = _one(orc, 300, x, u, top_k=40)
    for b in range(8):
        kept = probs[b] > 0
        if kept.sum() != 40 or x[b][kept].min() < x[b][~kept].max():
            out.append(f"invariant: top-k row {b}")
    _, info, probs = _one(orc, 300, x, u, top_p=0.7)
    for b in range(8):
        z = x[b].astype(np.float64)
        kept = probs[b] > 0
        e = np.exp(z - z.max())
        mass = e[kept].sum() / e.sum()
        last = e[kept].min() / e.sum()
        if not (mass >= 0.7 - 1e-6 and mass - last < 0.7 + 1e-6):
            out.append(f"invariant: top-p row {b} mass {mass}")
    return out


ALL = [check_temperature_reciprocal, check_penalties_hand_computed, check_mask_bit_order, check_uniform_cdf_strict,
       check_top_p_inclusive, check_min_p_relative_to_max, check_ties_lowest_id, check_sentinels,
       check_brute_force, check_stratified_frequencies, check_invariants]


def run_all(orc) -> list[str]:
    out = []
    for chk in ALL:
        try:
            out += chk(orc)
        except Exception as e:  # a crash in a planted-mistake build counts as caught
            out.append(f"{chk.__name__} raised {e!r}")
    return out
