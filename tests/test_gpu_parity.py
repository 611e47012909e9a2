"""GPU parity: libarbor_hip against the CPU oracle on identical seeded inputs.

Token ids must be bit-exact on every row the oracle does not flag as a boundary row
(|C_j - u| < 1e-6 plus the mass of tokens whose top-p / min-p membership is ambiguous);
filtered probabilities must match to 1e-5 relative wherever the kept sets agree. Every
test goes through the C ABI (arbor_sample) with device buffers.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

from arbornet_amd import sampling as S
from arbornet_amd import synthetic as syn

from gpu_helpers import compare, pack_mask, run_gpu

pytestmark = pytest.mark.gpu


def _announce(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    S.library()
    yield


# ----------------------------------------------------------------------------------------
# The five benchmark configurations at full size (ids), and with probabilities on a slice
# ----------------------------------------------------------------------------------------
# boundary rows each configuration may hold (the oracle flags c2: 5 of 64, the others 0)
MAX_BOUNDARY = {"c1": 0, "c2": 8, "c3": 2, "c4": 2, "c5": 2}


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c4", "c5"])
def test_config_ids_full(name):
    w = syn.CONFIGS[name]
    _announce(f"[parity] {name} full B={w.batch} V={w.vocab} {w.dtype}")
    inp = syn.generate(w)
    p = S.params_for(w)
    ids, _ = run_gpu(p, inp, repeat=2)
    n, nb, nbm = compare(S.params_for(w), inp, ids, label=name, max_boundary=MAX_BOUNDARY[name])
    _announce(f"[parity] {name}: rows {n}, boundary {nb}, boundary rows differing {nbm}")


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c4", "c5"])
def test_config_probs(name):
    w = syn.CONFIGS[name]
    nb = min(w.batch, 32)
    w = w.scaled(batch=nb)
    _announce(f"[parity] {name} probs B={nb}")
    inp = syn.generate(w)
    ids, probs = run_gpu(S.params_for(w), inp, write_probs=True)
    compare(S.params_for(w), inp, ids, probs, label=f"{name}-probs")


# ----------------------------------------------------------------------------------------
# Edge cases on small random inputs (numpy RNG, seeded)
# ----------------------------------------------------------------------------------------
def _random_inputs(B, V, *, ld=None, dtype="f32", H=0, mask_frac=0.0, seed=0, scale=2.0, ties=False):
    rng = np.random.default_rng(seed)
    ld = ld or V
    x = (rng.standard_normal((B, ld)) * scale).astype(np.float32)
    if ties:
        x = np.round(x)  # many equal values
    if dtype == "bf16":
        b = x.view(np.uint32)
        logits = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    else:
        logits = x
    hist = rng.integers(-1, V, size=(B, H), dtype=np.int32) if H else None
    if hist is not None and H > 4:  # repeats
        hist[:, H // 2:] = hist[:, : H - H // 2][:, : H // 2]
    mask = None
    if mask_frac > 0:
        mask = pack_mask(rng.random((B, V)) < mask_frac)
    u = rng.random(B).astype(np.float32)
    return syn.Inputs(logits, hist, mask, u)


def _params(B, V, inp, **kw):
    dtype = S.ARBOR_DTYPE_BF16 if inp.logits.dtype == np.uint16 else S.ARBOR_DTYPE_F32
    p = S.SamplingParams.make(B, V, ld_logits=inp.logits.shape[1], dtype=dtype, **kw)
    if inp.history is not None:
        p.hist_len = inp.history.shape[1]
    return p


EDGE = [
    # (B, V, ld, dtype, H, mask_frac, params)
    (4, 8, None, "f32", 0, 0.0, dict(top_k=3)),
    (4, 8, None, "f32", 6, 0.0, dict(top_k=2, top_p=0.7, repetition_penalty=1.3)),
    (5, 257, None, "f32", 0, 0.0, dict(top_k=17, top_p=0.8)),
    (5, 257, 260, "f32", 0, 0.0, dict(top_k=9)),
    (3, 257, None, "bf16", 0, 0.0, dict(top_k=5, min_p=0.1)),
    (8, 4096, None, "f32", 64, 0.0, dict(top_k=1)),
    (8, 4096, None, "f32", 64, 0.3, dict(top_k=20, top_p=0.9, frequency_penalty=0.4, presence_penalty=0.2)),
    (16, 32000, None, "f32", 256, 0.0, dict(top_k=256, temperature=0.5)),
    (16, 32000, None, "bf16", 256, 0.05, dict(top_k=64, top_p=0.5, repetition_penalty=1.2)),
    (8, 32000, None, "f32", 128, 0.0, dict(top_k=1000, top_p=0.9)),  # row solver (k > 256)
    (8, 32000, None, "f32", 128, 0.0, dict(top_p=0.8)),  # row solver (top-p only)
    (8, 32000, None, "f32", 0, 0.0, dict()),  # row solver (no filter)
    (8, 32000, None, "f32", 0, 0.2, dict(min_p=0.02)),  # stream, min-p band
    (8, 32000, None, "bf16", 512, 0.0, dict(top_p=0.95, min_p=0.1, temperature=1.3)),
    (9, 5000, None, "f32", 0, 0.0, dict(top_k=50, top_p=0.95)),  # batch not a multiple of 8
    (3, 100000, None, "f32", 4096, 0.0, dict(top_k=40, repetition_penalty=1.5, frequency_penalty=0.1)),
    # split row solver: strided rows, odd vocabularies, unaligned bf16 rows, masks
    (6, 24577, 24580, "f32", 64, 0.0, dict(top_p=0.85, repetition_penalty=1.2)),
    (5, 30001, 30003, "bf16", 0, 0.0, dict(top_p=0.9, temperature=0.9)),
    (7, 50000, None, "f32", 128, 0.1, dict(top_k=200, top_p=0.95, presence_penalty=0.5)),
    (4, 65537, None, "f32", 0, 0.0, dict(top_p=0.5, min_p=0.01)),
]


@pytest.mark.parametrize("case", range(len(EDGE)))
def test_edge(case):
    B, V, ld, dtype, H, mf, kw = EDGE[case]
    _announce(f"[edge {case}] B={B} V={V} ld={ld} {dtype} H={H} mask={mf} {kw}")
    inp = _random_inputs(B, V, ld=ld, dtype=dtype, H=H, mask_frac=mf, seed=100 + case)
    ids, probs = run_gpu(_params(B, V, inp, **kw), inp, write_probs=True)
    compare(_params(B, V, inp, **kw), inp, ids, probs, label=f"edge{case}")


@pytest.mark.parametrize("kw", [dict(top_k=4), dict(top_p=0.5), dict(min_p=0.5), dict()])
def test_ties_lowest_id_wins(kw):
    # all-equal logits: the ranking is by id, so top-k keeps the lowest ids
    B, V = 4, 1000
    inp = syn.Inputs(np.zeros((B, V), np.float32), None, None, np.array([0.0, 0.3, 0.7, 0.999], np.float32))
    ids, probs = run_gpu(_params(B, V, inp, **kw), inp, write_probs=True)
    compare(_params(B, V, inp, **kw), inp, ids, probs, label=f"ties{kw}")
    if "top_k" in kw:
        assert np.all(ids < kw["top_k"])


@pytest.mark.parametrize("kw", [dict(top_p=0.5), dict(top_k=300), dict(top_k=3000, top_p=0.9)])
@pytest.mark.parametrize("rounded", [False, True])
@pytest.mark.parametrize("V", [5000, 40000])
def test_solver_many_ties(kw, rounded, V):
    # More tied entries at the cut than the row solver ranks directly (1024): all-equal
    # rows, and integer-valued logits (thousands of exact ties per value). V = 40000 puts
    # each row on several workgroups (the split solver).
    B = 4
    if rounded:
        inp = _random_inputs(B, V, seed=23, ties=True)
    else:
        inp = syn.Inputs(np.zeros((B, V), np.float32), None, None, np.array([0.0, 0.3, 0.7, 0.999], np.float32))
    _announce(f"[solver ties] V={V} rounded={rounded} {kw}")
    ids, probs = run_gpu(_params(B, V, inp, **kw), inp, write_probs=True)
    compare(_params(B, V, inp, **kw), inp, ids, probs, label=f"solver-ties{kw}{rounded}")


@pytest.mark.parametrize("kw", [dict(top_p=0.5), dict(top_k=3000), dict(top_k=3000, top_p=0.7)])
@pytest.mark.parametrize("V", [5000, 40000])
def test_solver_dense_bin(kw, V):
    # One level-0 bin (a 4096th of the z span) holds nearly the whole row: distinct values
    # spread over [0, 1e-3) and one outlier at -30, so the cut lies inside a bin with more
    # entries than are collected directly and is found by the level-1 histogram.
    # V = 40000 puts each row on several workgroups (the split solver).
    B = 4
    rng = np.random.default_rng(31)
    x = (rng.random((B, V)) * 1e-3).astype(np.float32)
    x[:, 7] = -30.0
    inp = syn.Inputs(x, None, None, np.array([0.05, 0.3, 0.7, 0.95], np.float32))
    _announce(f"[solver dense bin] V={V} {kw}")
    ids, probs = run_gpu(_params(B, V, inp, **kw), inp, write_probs=True)
    compare(_params(B, V, inp, **kw), inp, ids, probs, label=f"solver-dense{kw}")


def test_sentinels():
    B, V = 6, 3000
    inp = _random_inputs(B, V, H=8, mask_frac=0.5, seed=7)
    inp.mask[0, :] = 0  # row 0: everything masked -> EMPTY
    inp.logits[1, 17] = np.nan  # row 1: NaN logit -> INVALID (unless masked)
    inp.mask[1, 0] |= np.uint32(1 << 17)
    inp.logits[2, 5] = np.inf  # row 2: +inf -> INVALID
    inp.mask[2, 0] |= np.uint32(1 << 5)
    inp.history[3, 3] = V  # row 3: history id >= V -> BAD_HISTORY
    inp.logits[4, 9] = np.nan  # row 4: NaN but masked -> fine
    inp.mask[4, 0] &= np.uint32(~(1 << 9) & 0xFFFFFFFF)
    inp.history[5, :] = -1  # row 5: all padding
    for kw in (dict(top_k=10), dict(top_p=0.9), dict(min_p=0.1)):
        ids, probs = run_gpu(_params(B, V, inp, **kw), inp, write_probs=True)
        assert ids[0] == S.ARBOR_ID_EMPTY, (kw, ids)
        assert ids[1] == S.ARBOR_ID_INVALID, (kw, ids)
        assert ids[2] == S.ARBOR_ID_INVALID, (kw, ids)
        assert ids[3] == S.ARBOR_ID_BAD_HISTORY, (kw, ids)
        assert ids[4] >= 0 and ids[5] >= 0, (kw, ids)
        assert np.all(probs[:4] == 0.0)
        compare(_params(B, V, inp, **kw), inp, ids, probs, label=f"sentinels{kw}")


def test_uniform_extremes():
    # u = 0 draws the first kept id; u just below 1 the last kept id (ascending id order)
    B, V = 4, 2000
    inp = _random_inputs(B, V, seed=11)
    inp.uniforms[:] = np.array([0.0, 0.0, np.float32(1) - np.float32(2 ** -24), 0.5], np.float32)
    for kw in (dict(top_k=30), dict(top_p=0.6)):
        ids, _ = run_gpu(_params(B, V, inp, **kw), inp)
        compare(_params(B, V, inp, **kw), inp, ids, label=f"uext{kw}")


@pytest.mark.parametrize("kw", [dict(top_k=8, repetition_penalty=3.0), dict(top_k=30, top_p=0.8, presence_penalty=2.0),
                                dict(min_p=0.3, frequency_penalty=1.5), dict(top_k=8, repetition_penalty=0.5)])
def test_masked_block_with_penalised_leaders(kw):
    # Only a contiguous block of each row is allowed, so the first batches over the block
    # overflow the stage and raise thresholds from raw values; the block's largest logits
    # are history ids, which the penalties lower (or, repetition < 1, raise). The kept set
    # must still be exact (thresholds that overshot send the row to the exact solver).
    B, V = 8, 40000
    rng = np.random.default_rng(31)
    x = (rng.standard_normal((B, V)) * 1.5).astype(np.float32)
    allowed = np.zeros((B, V), bool)
    hist = np.full((B, 64), -1, np.int32)
    for r in range(B):
        lo = int(rng.integers(0, V - 4096))
        allowed[r, lo:lo + 4096] = True
        lead = lo + np.argsort(x[r, lo:lo + 4096])[::-1][:40]
        x[r, lead[:20]] += 6.0
        hist[r, :40] = lead
        hist[r, 40:48] = lead[:8]  # repeats
    inp = syn.Inputs(x, hist, pack_mask(allowed), rng.random(B).astype(np.float32))
    _announce(f"[masked leaders] {kw}")
    ids, probs = run_gpu(_params(B, V, inp, **kw), inp, write_probs=True)
    compare(_params(B, V, inp, **kw), inp, ids, probs, label=f"masked-leaders{kw}")


def test_minp_overflow_falls_back_to_row_solver():
    # flat logits: every token is inside the min-p band, so the stream path's candidate
    # lists overflow and the finishing workgroup solves the row exactly instead
    B, V = 8, 50000
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((B, V)) * 0.01).astype(np.float32)
    inp = syn.Inputs(x, None, None, rng.random(B).astype(np.float32))
    ids, probs = run_gpu(_params(B, V, inp, min_p=0.5), inp, write_probs=True)
    compare(_params(B, V, inp, min_p=0.5), inp, ids, probs, label="minp-overflow")


def test_sample_op_on_torch_tensors():
    import torch

    w = syn.CONFIGS["c3"].scaled(batch=16)
    inp = syn.generate(w)
    x = torch.from_numpy(inp.logits).cuda()
    ids = S.Sampling.sample(x, torch.from_numpy(inp.uniforms), temperature=w.temperature,
                            repetition_penalty=w.repetition_penalty, top_k=w.top_k, top_p=w.top_p,
                            history=torch.from_numpy(inp.history))
    torch.cuda.synchronize()
    compare(S.params_for(w), inp, ids.cpu().numpy(), label="Sampling.sample")
    with pytest.raises(S.ArborSamplingError) as ei:
        S.Sampling.sample(x, torch.from_numpy(inp.uniforms), temperature=0.0)
    assert ei.value.status == -5


def _random_case(i):
    """A seeded random parameter set (sizes small enough for the oracle)."""
    rng = np.random.default_rng(1000 + i)
    B = int(rng.integers(1, 10))
    V = int(rng.choice([257, 1000, 4099, 12000, 32000, 50001]))
    ld = V + int(rng.choice([0, 0, 3, 16]))
    dtype = "bf16" if rng.random() < 0.3 else "f32"
    H = int(rng.choice([0, 0, 8, 64, 512]))
    mf = float(rng.choice([0.0, 0.0, 0.05, 0.5]))
    kw = dict(temperature=float(rng.choice([0.5, 0.8, 1.0, 1.7])))
    r = rng.random()
    if r < 0.45:
        kw["top_k"] = int(rng.choice([1, 5, 40, 64, 100, 2000]))
    if rng.random() < 0.5:
        kw["top_p"] = float(rng.choice([0.3, 0.9, 0.99]))
    if rng.random() < 0.35:
        kw["min_p"] = float(rng.choice([0.01, 0.1, 0.5]))
    if H:
        kw["repetition_penalty"] = float(rng.choice([0.7, 1.0, 1.3]))
        kw["frequency_penalty"] = float(rng.choice([0.0, 0.0, 0.4, -0.2]))
        kw["presence_penalty"] = float(rng.choice([0.0, 0.3]))
    return B, V, ld, dtype, H, mf, kw


@pytest.mark.parametrize("i", range(300))
def test_random_parameter_sets(i):
    B, V, ld, dtype, H, mf, kw = _random_case(i)
    _announce(f"[random {i}] B={B} V={V} ld={ld} {dtype} H={H} mask={mf} {kw}")
    inp = _random_inputs(B, V, ld=ld, dtype=dtype, H=H, mask_frac=mf, seed=2000 + i)
    ids, probs = run_gpu(_params(B, V, inp, **kw), inp, write_probs=True)
    compare(_params(B, V, inp, **kw), inp, ids, probs, label=f"random{i}")


def test_split_barrier_give_up_reports_stalled(monkeypatch):
    # The split row solver's barriers wait at most a spin limit, then give up: the row's
    # failure word makes every workgroup of the row stop waiting and the row reads
    # ARBOR_ID_STALLED. A spin limit of one sleep (set from the host) makes waits give up
    # whenever a row's workgroups are not perfectly in step; every kernel still ends. Each
    # row is then either STALLED or exact, and a normal call afterwards is exact again.
    B, V = 6, 40000
    inp = _random_inputs(B, V, H=16, seed=77)
    kw = dict(top_p=0.8, repetition_penalty=1.2)
    monkeypatch.setenv("ARBOR_SPLIT_SPIN_LIMIT", "1")
    _announce("[split give-up] spin limit 1")
    ids, _ = run_gpu(_params(B, V, inp, **kw), inp)
    stalled = ids == S.ARBOR_ID_STALLED
    _announce(f"[split give-up] {int(stalled.sum())} of {B} rows stalled")
    if (~stalled).any():
        keep = np.nonzero(~stalled)[0]
        from oracle import oracle
        want, info, _ = oracle.sample(_params(B, V, inp, **kw), inp.logits, inp.history, None, inp.uniforms)
        ok = (ids[keep] == want[keep]) | ((info["boundary"][keep] & oracle.BOUNDARY_CDF) != 0)
        assert ok.all(), (ids, want)
    monkeypatch.delenv("ARBOR_SPLIT_SPIN_LIMIT")
    ids, _ = run_gpu(_params(B, V, inp, **kw), inp)
    compare(_params(B, V, inp, **kw), inp, ids, label="split after give-up")
