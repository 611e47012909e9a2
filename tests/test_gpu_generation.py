"""GPU: the generation step (arbor_sample_append) in a multi-step loop. At every step the
sampled ids must equal the oracle's on the history the device holds before the step
(ids bit-exact on non-boundary rows), and the history ring after the step must be that
history with each valid sampled id written at slot positions % H."""
from __future__ import annotations

import sys

import numpy as np
import pytest

from arbornet_amd import sampling as S
from arbornet_amd import synthetic as syn

from gpu_helpers import compare, pack_mask

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    S.library()
    yield


def _ring_after(hist, pos, ids):
    """The ring update the step must make (host restatement of the documented contract)."""
    hist, pos = hist.copy(), pos.copy()
    for b, i in enumerate(ids):
        if i >= 0:
            hist[b, pos[b] % hist.shape[1]] = i
            pos[b] += 1
    return hist, pos


LOOPS = [
    # (B, V, seq, H, steps, dtype, sampling params)
    (8, 32000, 3, 16, 40, "f32", dict(temperature=0.8, repetition_penalty=1.3, frequency_penalty=0.3,
                                       presence_penalty=0.2, top_k=20, top_p=0.9)),
    (6, 20000, 1, 64, 30, "bf16", dict(temperature=1.2, repetition_penalty=1.5, min_p=0.05)),
    (4, 40000, 2, 8, 25, "f32", dict(repetition_penalty=0.8, top_p=0.7)),  # split row solver, raising penalty
    # a batch that fills the chip: one workgroup per row, the id appended by the kernel that draws it
    (256, 32000, 1, 32, 4, "f32", dict(temperature=0.7, repetition_penalty=1.15, top_k=50, top_p=0.95)),
    # near-flat rows: the min-p band overflows the 64-entry list and the band solver draws
    # (one workgroup per row), appending the id itself
    (256, 4096, 1, 16, 3, "bf16", dict(min_p=0.05, repetition_penalty=1.1, _scale=0.01)),
    # the same with rows split over workgroups: the finishing kernel's band solver appends
    (4, 40000, 1, 16, 3, "f32", dict(min_p=0.05, repetition_penalty=1.1, _scale=0.01)),
    (300, 6000, 1, 16, 3, "f32", dict(top_k=100, _scale=0.5)),  # k > 64: the histogram solver, then an append launch
]


@pytest.mark.parametrize("case", range(len(LOOPS)))
def test_generation_loop_matches_oracle(case):
    import torch

    B, V, seq, H, steps, dtype, kw = LOOPS[case]
    kw = dict(kw)
    scale = kw.pop("_scale", 2.0)
    print(f"[generation {case}] B={B} V={V} seq={seq} H={H} steps={steps} {dtype} {kw}", flush=True)
    rng = np.random.default_rng(50 + case)
    base = (rng.standard_normal((B, V)) * scale).astype(np.float32)
    state = S.GenerationState(B, H, "cuda:0", prompt=rng.integers(0, V, size=(B, 5), dtype=np.int32))
    tdt = torch.float32 if dtype == "f32" else torch.bfloat16
    for step in range(steps):
        # the model's [B, seq, V] output; its last position changes a little every step
        x = np.repeat(base[:, None, :], seq, axis=1)
        x[:, -1, :] += (rng.standard_normal((B, V)) * (scale / 4)).astype(np.float32)
        logits = torch.from_numpy(x).to("cuda:0", dtype=tdt)
        u = rng.random(B).astype(np.float32)
        hist_before = state.history.cpu().numpy()
        pos_before = state.positions.cpu().numpy()
        ids = state.step(logits, torch.from_numpy(u), **kw).cpu().numpy()
        # ids against the oracle on the same (rounded) last-position logits and history
        last = logits[:, -1, :].contiguous()
        if dtype == "bf16":
            last_np = last.view(torch.int16).cpu().numpy().view(np.uint16)
        else:
            last_np = last.cpu().numpy()
        p = S.SamplingParams.make(B, V, dtype=S.ARBOR_DTYPE_BF16 if dtype == "bf16" else S.ARBOR_DTYPE_F32,
                                  hist_len=H, **kw)
        compare(p, syn.Inputs(last_np, hist_before, None, u), ids, label=f"gen{case}-step{step}")
        want_h, want_p = _ring_after(hist_before, pos_before, ids)
        np.testing.assert_array_equal(state.history.cpu().numpy(), want_h, err_msg=f"step {step} ring")
        np.testing.assert_array_equal(state.positions.cpu().numpy(), want_p, err_msg=f"step {step} positions")
    assert (state.positions.cpu().numpy() >= steps).all()  # every row appended every step (wrapped the ring)


def test_generation_sentinel_rows_append_nothing():
    import torch

    B, V, H = 4, 5000, 8
    rng = np.random.default_rng(3)
    state = S.GenerationState(B, H, "cuda:0")
    x = torch.from_numpy((rng.standard_normal((B, V)) * 2.0).astype(np.float32)).to("cuda:0")
    allowed = np.ones((B, V), bool)
    allowed[1] = False  # row 1: everything masked -> ARBOR_ID_EMPTY
    mask = torch.from_numpy(pack_mask(allowed).view(np.int32)).to("cuda:0")
    for _ in range(3):
        ids = state.step(x, torch.from_numpy(rng.random(B).astype(np.float32)), top_k=10,
                         repetition_penalty=1.2, allow_mask=mask).cpu().numpy()
        assert ids[1] == S.ARBOR_ID_EMPTY and (np.delete(ids, 1) >= 0).all()
    pos = state.positions.cpu().numpy()
    assert pos[1] == 0 and (np.delete(pos, 1) == 3).all()
    assert (state.history.cpu().numpy()[1] == -1).all()
