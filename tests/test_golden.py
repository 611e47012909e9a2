"""The committed golden fixtures on the CPU: the oracle reproduces every expected output,
the brute-force sampler agrees on every row it does not call ambiguous, and the seeded
generators reproduce the configurations' inputs bit for bit (sha256)."""
from __future__ import annotations

import numpy as np
import pytest

import brute
import golden_data as G
from arbornet_amd import sampling as S
from arbornet_amd import synthetic as syn
from oracle import oracle


@pytest.mark.parametrize("case", G.small_cases(), ids=lambda c: c.name)
def test_small_fixture_oracle(case):
    p = case.sampling_params()
    ids, info, probs = oracle.sample(p, case.logits, case.history, case.mask, case.uniforms, probs=True)
    np.testing.assert_array_equal(ids, case.ids)
    np.testing.assert_array_equal(info["n_kept"], case.n_kept)
    np.testing.assert_array_equal(info["boundary"], case.boundary)
    np.testing.assert_allclose(info["kept_mass"], case.kept_mass, rtol=1e-12)
    np.testing.assert_allclose(probs, case.probs, rtol=1e-6, atol=0)


@pytest.mark.parametrize("case", G.small_cases(), ids=lambda c: c.name)
def test_small_fixture_brute(case):
    p = case.sampling_params()
    checked = 0
    for b in range(p.batch):
        h = None if case.history is None else case.history[b]
        m = None if case.mask is None else case.mask[b]
        bid, kept, bprob, amb = brute.sample_row(p, case.logits[b], h, m, float(case.uniforms[b]))
        if amb:
            continue
        checked += 1
        assert bid == case.ids[b], f"row {b}: fixture {case.ids[b]} brute {bid}"
        if bid >= 0:
            assert np.nonzero(case.probs[b])[0].tolist() == kept
            got = np.array([case.probs[b, i] for i in kept])
            np.testing.assert_allclose(got, [bprob[i] for i in kept], rtol=2e-6)
    assert checked > 0


def test_small_fixture_sizes():
    vocabs = {c.params["vocab"] for c in G.small_cases()}
    assert vocabs == {8, 257, 4096, 32000}
    assert all(c.params["batch"] <= 8 for c in G.small_cases())


def test_c1_whole():
    z = np.load(G.GOLDEN / "c1.npz")
    w = syn.CONFIGS["c1"]
    inp = syn.generate(w)
    np.testing.assert_array_equal(inp.logits, z["logits"])
    np.testing.assert_array_equal(inp.uniforms, z["uniforms"])
    ids, info, probs = oracle.sample(S.params_for(w), z["logits"], None, None, z["uniforms"], probs=True)
    np.testing.assert_array_equal(ids, z["ids"])
    np.testing.assert_array_equal(info["n_kept"], z["n_kept"])
    np.testing.assert_allclose(probs, z["probs"], rtol=1e-6, atol=0)
    assert info["n_kept"][0] == 40


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c4", "c5"])
def test_config_fixture(name):
    man = G.config_manifest()[name]
    out = G.config_outputs()
    w = syn.CONFIGS[name]
    assert S.params_for(w).as_dict() == man["params"]
    inp = syn.generate(w)
    for k in ("logits", "history", "mask", "uniforms"):
        assert G.sha256(getattr(inp, k)) == man["sha256"][k], f"{name}: generated {k} changed"
    ids, info, _ = oracle.sample(S.params_for(w), inp.logits, inp.history, inp.mask, inp.uniforms, threads=8)
    np.testing.assert_array_equal(ids, out[f"{name}/ids"])
    np.testing.assert_array_equal(info["n_kept"], out[f"{name}/n_kept"])
    np.testing.assert_array_equal(info["boundary"], out[f"{name}/boundary"])
