"""GPU parity on the product paths that only large shapes reach: full-vocabulary rows on
the one-workgroup-per-row solver (a batch that fills the chip), rows longer than 262,144
ids (the solvers' unfused passes), and rows at the header's vocabulary limit (the streaming
kernel's forced split into chunks). Each case names the path make_plan takes for it; ids
must equal the oracle's on every non-boundary row, and boundary rows must pass
check_boundary_row."""
from __future__ import annotations

import sys

import numpy as np
import pytest

from arbornet_amd import sampling as S
from arbornet_amd import synthetic as syn

from gpu_helpers import compare, run_gpu

pytestmark = pytest.mark.gpu

# c2's input distribution (N(0, 1.5^2) plus 16 spikes at +6..+12) at other shapes
BASE = syn.CONFIGS["c2"]

CASES = [
    # (label, batch, vocab, dtype, sampling overrides, rows whose probabilities are checked)
    # a batch that fills the chip: one workgroup per row on full-vocabulary rows
    ("top-p 0.9, B=256 (c2 parameters at c3's batch)", 256, 128256, "f32", {}, 8),
    ("no filter, B=256", 256, 128256, "f32", dict(top_p=1.0, repetition_penalty=1.0, hist_len=0), 8),
    ("top-k 300, B=256", 256, 128256, "f32", dict(top_k=300, top_p=1.0), 8),
    # rows longer than 262,144 ids
    ("top-k 50 stream, V=300007", 2, 300007, "f32", dict(top_k=50, top_p=1.0), 2),
    ("top-k 50 stream, V=300007 bf16", 2, 300007, "bf16", dict(top_k=50, top_p=1.0), 2),
    ("min-p band, V=300007", 2, 300007, "f32", dict(top_p=1.0, min_p=0.05), 2),
    ("min-p band, V=300007 bf16", 2, 300007, "bf16", dict(top_p=1.0, min_p=0.05), 2),
    ("top-p split rows, V=300007", 2, 300007, "f32", dict(top_p=0.9), 2),
    ("top-p split rows, V=300007 bf16", 2, 300007, "bf16", dict(top_p=0.9), 2),
    ("top-p one row per workgroup, V=300007, B=256", 256, 300007, "f32", dict(top_p=0.9), 4),
    ("top-p one row per workgroup, V=300007, B=256 bf16", 256, 300007, "bf16", dict(top_p=0.9), 4),
    ("top-p two chunks of 300,000 ids, B=100", 100, 600000, "f32", dict(top_p=0.9, hist_len=128), 2),
    # the vocabulary limit: a batch that fills the chip forces the streaming kernel to split
    # each row into chunks (the chunk's history bitmap holds at most 262,144 ids)
    ("top-k 50 stream at ARBOR_VOCAB_MAX, B=256 bf16", 256, 1048575, "bf16", dict(top_k=50, top_p=0.95), 2),
    ("top-k 50 stream at ARBOR_VOCAB_MAX, B=2", 2, 1048575, "f32", dict(top_k=50), 2),
    # the two-pass top-p kernel with min-p beside top-p, on c4's inputs (min-p's edge far
    # above top-p's cut, so min-p decides), rows split over workgroups and whole
    ("c4 inputs, top-p 0.9 + min-p 0.05, B=64", -64, 152064, "bf16", dict(top_p=0.9), 4),
    ("c4 inputs, top-p 0.9 + min-p 0.05, B=256", -256, 152064, "bf16", dict(top_p=0.9), 4),
    ("c4 inputs, top-p 0.3 + min-p 0.01, B=64", -64, 152064, "bf16", dict(top_p=0.3, min_p=0.01), 4),
    # masked fp32 rows streamed whole: after their first batches they visit only the units
    # that hold an allowed id, from an LDS list of up to 8192 units; denser masks walk every
    # unit
    ("masked stream, sparse mask (unit list), B=256", 256, 128256, "f32",
     dict(top_k=20, top_p=0.9, repetition_penalty=1.0, hist_len=0, mask_block_frac=0.02, mask_scatter=300), 2),
    ("masked stream, dense mask (list overflows), B=256", 256, 152064, "f32",
     dict(top_k=50, top_p=0.95, mask_block_frac=0.9, mask_scatter=64), 2),
    ("masked stream, min-p band, sparse mask, B=256", 256, 100000, "f32",
     dict(top_p=1.0, min_p=0.05, mask_block_frac=0.05, mask_scatter=32), 2),
    ("masked split rows, sparse mask, B=8", 8, 128256, "f32",
     dict(top_k=20, top_p=0.9, mask_block_frac=0.05, mask_scatter=32), 2),
]


@pytest.fixture(scope="module", autouse=True)
def _device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    S.library()
    yield


@pytest.mark.parametrize("case", range(len(CASES)), ids=lambda i: CASES[i][0])
def test_large_shape_paths(case):
    label, B, V, dtype, kw, nprob = CASES[case]
    base = BASE
    if B < 0:  # c4's inputs and parameters
        base, B = syn.CONFIGS["c4"], -B
    w = base.scaled(batch=B, vocab=V, dtype=dtype, seed=40 + case, **kw)
    print(f"[paths {case}] {label}: B={B} V={V} {dtype} {kw}", flush=True)
    sys.stdout.flush()
    inp = syn.generate(w)
    ids, _ = run_gpu(S.params_for(w), inp, repeat=2)
    # top-p rows that keep tens of thousands of ids have CDF steps of ~1e-5, so a tenth to
    # a half of them fall within 1e-6 (plus the ambiguous mass at the cut) of a step
    n, nb, nbm = compare(S.params_for(w), inp, ids, label=label, max_boundary=max(2, (6 * B) // 10))
    print(f"[paths {case}] rows {n}, boundary {nb}, boundary rows differing {nbm}", flush=True)
    if B * V <= 80_000_000:  # probabilities of the whole batch, on the same path
        ids_p, probs = run_gpu(S.params_for(w), inp, write_probs=True)
        compare(S.params_for(w), inp, ids_p, probs, label=f"{label} (probs)")
        assert np.all(ids >= 0)
        return
    # probabilities on the first rows only (host copies of a whole batch would be large)
    ws = w.scaled(batch=nprob)
    sub = syn.Inputs(inp.logits[:nprob], None if inp.history is None else inp.history[:nprob],
                     None if inp.mask is None else inp.mask[:nprob], inp.uniforms[:nprob])
    ids_p, probs = run_gpu(S.params_for(ws), sub, write_probs=True)
    compare(S.params_for(ws), sub, ids_p, probs, label=f"{label} (probs)")
    assert np.all(ids >= 0)


def _flat_top(inp: syn.Inputs, rows, dtype: str, width, seed: int) -> syn.Inputs:
    """The given rows get a plateau: `width` random ids (an int, or a list cycled over the
    rows) lifted to 4 above the row's maximum (within +-0.05 of each other), so min-p's
    band holds far more ids than the streaming kernel's 64-entry list: up to 1024 of them
    are drawn from the list and the entries it spilled, more go to the band solver."""
    rng = np.random.default_rng(seed)
    widths = width if isinstance(width, (list, tuple)) else [width]
    x = inp.logits.copy()
    for i, r in enumerate(rows):
        wr = widths[i % len(widths)]
        if dtype == "bf16":
            row = (x[r].astype(np.uint32) << 16).view(np.float32)
        else:
            row = x[r].copy()
        top = float(np.max(row[np.isfinite(row)]))
        ids = rng.choice(row.size, size=wr, replace=False)
        row[ids] = top + 4.0 + rng.uniform(-0.05, 0.05, size=wr).astype(np.float32)
        x[r] = (row.view(np.uint32) >> 16).astype(np.uint16) if dtype == "bf16" else row
    return syn.Inputs(x, inp.history, inp.mask, inp.uniforms)


BAND_CASES = [
    # (label, batch, vocab, dtype, plateau width(s), mask, other parameters) on c4's
    # parameters (min-p 0.05 alone, frequency and presence penalties, history of up to 2048
    # ids). Rows of a batch of 256 or more are finished by their streaming workgroup: bands
    # of up to 1024 ids from the list and its spill, wider ones by the band solver.
    ("c4 shape, every other row flat, B=512", 512, 152064, "bf16", 400, False, {}),
    ("spill and spill overflow, fp32, B=256", 256, 50000, "f32", [100, 900, 1500, 65], False, {}),
    ("spill, masked bf16, B=256", 256, 65536, "bf16", [300, 2000, 700], True, {}),
    ("spill, repetition penalty below 1, B=256", 256, 40000, "f32", [500, 1200], False,
     {"repetition_penalty": 0.9, "frequency_penalty": 0.0, "presence_penalty": -0.2}),
    ("spill, whole rows of a small vocabulary, B=8", 8, 8000, "f32", [500, 64, 1000, 3000], False, {}),
    ("split rows (finished by the finishing kernel), B=4", 4, 152064, "bf16", 2000, False, {}),
    ("split rows, fp32, masked, B=3", 3, 50000, "f32", 300, True, {}),
    ("one row, B=1", 1, 32000, "f32", 100, False, {}),
]


@pytest.mark.parametrize("case", range(len(BAND_CASES)), ids=lambda i: BAND_CASES[i][0])
def test_band_overflow(case):
    # flat-topped min-p rows go to the band solver, mixed with rows the 64-entry list
    # finishes; both kinds must match the oracle
    label, B, V, dtype, width, masked, extra = BAND_CASES[case]
    w = syn.CONFIGS["c4"].scaled(batch=B, vocab=V, dtype=dtype, seed=90 + case,
                                 hist_len=min(2048, V // 8), **extra)
    if masked:
        w = w.scaled(mask_block_frac=0.5, mask_scatter=8)
    print(f"[band {case}] {label}: B={B} V={V} {dtype} plateau {width}", flush=True)
    inp = _flat_top(syn.generate(w), range(0, B, 2), dtype, width, seed=case)
    p = S.params_for(w)
    ids, _ = run_gpu(p, inp, repeat=2)
    compare(S.params_for(w), inp, ids, label=label, max_boundary=max(1, B // 10))
    assert np.all(ids >= 0)
    if B * V <= 20_000_000:
        ids_p, probs = run_gpu(S.params_for(w), inp, write_probs=True)
        compare(S.params_for(w), inp, ids_p, probs, label=f"{label} (probs)")
