#!/usr/bin/env python3
"""Writes the golden fixtures of the sampling step (run from the repository root:
`python tests/golden/make_golden.py`). The reference holds no golden vectors for this
path, so these fixtures, made by the CPU oracle (itself pinned by closed forms, a
brute-force sampler and planted-mistake checks), are the committed pin.

small.npz / small.json   small cases, B <= 8, V in {8, 257, 4096, 32000}, every stage
                         toggled: inputs (numpy-seeded, stored whole) and expected ids,
                         kept counts, boundary flags, kept mass and probabilities
c1.npz                   configuration c1 whole (one 32000-token row) with its outputs
configs.npz / .json      c1..c5: generator seed and shape, sha256 of each generated input
                         array, and per row the expected id, kept count, boundary flags
                         and distance of u to the nearest CDF step
"""
from __future__ import annotations

import hashlib
import json
import sys
from dataclasses import asdict
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

from arbornet_amd import sampling as S  # noqa: E402
from arbornet_amd import synthetic as syn  # noqa: E402
from oracle import oracle  # noqa: E402

# (name, B, V, ld, dtype, H, mask_frac, ties, scale, params)
SMALL = [
    ("v8_plain", 4, 8, 0, "f32", 0, 0.0, False, 2.0, dict()),
    ("v8_penalties", 4, 8, 0, "f32", 16, 0.0, False, 2.0,
     dict(repetition_penalty=1.3, frequency_penalty=0.5, presence_penalty=0.25)),
    ("v8_topk_ties", 8, 8, 0, "f32", 0, 0.0, True, 1.0, dict(top_k=3)),
    ("v257_topk", 8, 257, 0, "f32", 0, 0.0, False, 2.0, dict(top_k=5, temperature=0.7)),
    ("v257_topp", 8, 257, 0, "f32", 0, 0.0, False, 2.0, dict(top_p=0.8)),
    ("v257_minp", 8, 257, 0, "f32", 0, 0.0, False, 2.0, dict(min_p=0.1)),
    ("v257_mask", 8, 257, 0, "f32", 0, 0.25, False, 2.0, dict(top_k=10)),
    ("v257_all_ld", 8, 257, 272, "f32", 24, 0.5, False, 3.0,
     dict(temperature=1.3, repetition_penalty=1.2, frequency_penalty=0.2, presence_penalty=0.1, top_k=20,
          top_p=0.9, min_p=0.05)),
    ("v257_bf16", 8, 257, 0, "bf16", 12, 0.0, False, 2.0, dict(top_k=8, top_p=0.95, repetition_penalty=1.1)),
    ("v4096_topk1", 4, 4096, 0, "f32", 64, 0.0, True, 2.0, dict(top_k=1, repetition_penalty=1.5)),
    ("v4096_topk_topp_pen", 4, 4096, 0, "f32", 128, 0.0, False, 2.0,
     dict(top_k=50, top_p=0.95, repetition_penalty=1.15)),
    ("v4096_minp_mask", 4, 4096, 0, "f32", 64, 0.3, False, 2.0,
     dict(min_p=0.05, frequency_penalty=0.5, presence_penalty=0.3)),
    ("v4096_bf16_all", 4, 4096, 0, "bf16", 64, 0.1, False, 2.0,
     dict(temperature=0.6, top_k=40, top_p=0.9, min_p=0.02, repetition_penalty=1.1, frequency_penalty=0.1)),
    ("v4096_topk_large", 4, 4096, 0, "f32", 0, 0.0, False, 1.0, dict(top_k=700, top_p=0.7)),
    ("v32000_topp", 2, 32000, 0, "f32", 32, 0.0, False, 1.5, dict(top_p=0.9, repetition_penalty=1.1)),
]


def sha256(a: np.ndarray | None) -> str | None:
    return None if a is None else hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def small_inputs(case, seed):
    name, B, V, ld, dtype, H, mask_frac, ties, scale, _ = case
    rng = np.random.default_rng(seed)
    ld = ld or V
    x = (rng.standard_normal((B, ld)) * scale).astype(np.float32)
    if ties:
        x = np.round(x).astype(np.float32)
    if dtype == "bf16":
        b = x.view(np.uint32)
        logits = ((b + np.uint32(0x7FFF) + ((b >> 16) & np.uint32(1))) >> 16).astype(np.uint16)
    else:
        logits = x
    hist = None
    if H:
        hist = rng.integers(-1, V, size=(B, H), dtype=np.int32)
        hist[:, H // 2:] = hist[:, : H - H // 2][:, : H - H // 2]  # repeats
    mask = None
    if mask_frac > 0:
        allowed = rng.random((B, V)) < (1.0 - mask_frac)
        mask = np.zeros((B, (V + 31) // 32), np.uint32)
        bb, tt = np.nonzero(allowed)
        np.bitwise_or.at(mask, (bb, tt >> 5), np.uint32(1) << (tt & 31).astype(np.uint32))
    u = rng.random(B).astype(np.float32)
    return logits, hist, mask, u


def small_params(case, logits, hist):
    name, B, V, ld, dtype, H, mask_frac, ties, scale, kw = case
    p = S.SamplingParams.make(B, V, ld_logits=logits.shape[1],
                              dtype=S.ARBOR_DTYPE_BF16 if dtype == "bf16" else S.ARBOR_DTYPE_F32, **kw)
    p.hist_len = H
    return p


def main():
    arrays, manifest = {}, {"cases": []}
    for i, case in enumerate(SMALL):
        name = case[0]
        seed = 1000 + i
        logits, hist, mask, u = small_inputs(case, seed)
        p = small_params(case, logits, hist)
        ids, info, probs = oracle.sample(p, logits, hist, mask, u, probs=True)
        arrays[f"{name}/logits"] = logits
        if hist is not None:
            arrays[f"{name}/history"] = hist
        if mask is not None:
            arrays[f"{name}/mask"] = mask
        arrays[f"{name}/uniforms"] = u
        arrays[f"{name}/ids"] = ids
        arrays[f"{name}/n_kept"] = info["n_kept"]
        arrays[f"{name}/boundary"] = info["boundary"]
        arrays[f"{name}/kept_mass"] = info["kept_mass"]
        arrays[f"{name}/probs"] = probs
        manifest["cases"].append({"name": name, "seed": seed, "params": p.as_dict()})
    np.savez_compressed(HERE / "small.npz", **arrays)
    (HERE / "small.json").write_text(json.dumps(manifest, indent=1) + "\n")

    w = syn.CONFIGS["c1"]
    inp = syn.generate(w)
    ids, info, probs = oracle.sample(S.params_for(w), inp.logits, inp.history, inp.mask, inp.uniforms, probs=True)
    np.savez_compressed(HERE / "c1.npz", logits=inp.logits, uniforms=inp.uniforms, ids=ids,
                        n_kept=info["n_kept"], boundary=info["boundary"], probs=probs)

    carr, cman = {}, {}
    for name, w in syn.CONFIGS.items():
        inp = syn.generate(w)
        p = S.params_for(w)
        ids, info, _ = oracle.sample(p, inp.logits, inp.history, inp.mask, inp.uniforms, threads=8)
        carr[f"{name}/ids"] = ids
        carr[f"{name}/n_kept"] = info["n_kept"]
        carr[f"{name}/boundary"] = info["boundary"]
        carr[f"{name}/cdf_gap"] = info["cdf_gap"]
        wd = asdict(w)
        wd.pop("extra")
        cman[name] = {"workload": wd, "params": p.as_dict(),
                      "sha256": {"logits": sha256(inp.logits), "history": sha256(inp.history),
                                 "mask": sha256(inp.mask), "uniforms": sha256(inp.uniforms)}}
        print(f"{name}: {len(ids)} rows, {int(((info['boundary'] & oracle.BOUNDARY_CDF) != 0).sum())} boundary")
    np.savez_compressed(HERE / "configs.npz", **carr)
    (HERE / "configs.json").write_text(json.dumps(cman, indent=1) + "\n")


if __name__ == "__main__":
    main()
