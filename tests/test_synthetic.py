"""The seeded workload generators (csrc/synth.c): their own log/cos/sin against libm, row
subsets regenerate bit-identically, and the distributions are the ones the benchmark
configurations name."""
from __future__ import annotations

import math

import numpy as np
import pytest

from arbornet_amd import synthetic as syn


def test_det_log_matches_libm():
    rng = np.random.default_rng(0)
    for x in np.concatenate([rng.random(2000), [1e-300, 2.0 ** -53, 0.5, 1.0 - 2.0 ** -53, 0.75]]):
        got, want = syn.det_log(float(x)), math.log(float(x))
        assert abs(got - want) <= 4e-16 * max(1.0, abs(want)), (x, got, want)


def test_det_cossin_matches_libm():
    for u in np.linspace(0.0, 1.0, 1001, endpoint=False):
        c, s = syn.det_cossin(float(u))
        assert abs(c - math.cos(2 * math.pi * u)) < 1e-14 and abs(s - math.sin(2 * math.pi * u)) < 1e-14, u


@pytest.mark.parametrize("name", ["c2", "c4", "c5"])
def test_row_subsets_regenerate(name):
    w = syn.CONFIGS[name].scaled(batch=12)
    full = syn.generate(w)
    part = syn.generate(w, row0=5, nrows=4)
    np.testing.assert_array_equal(part.logits, full.logits[5:9])
    np.testing.assert_array_equal(part.uniforms, full.uniforms[5:9])
    if full.history is not None:
        np.testing.assert_array_equal(part.history, full.history[5:9])
    if full.mask is not None:
        np.testing.assert_array_equal(part.mask, full.mask[5:9])


def test_spiked_normal_logits():
    w = syn.CONFIGS["c3"].scaled(batch=8)
    x = syn.generate(w).logits
    assert x.dtype == np.float32 and x.shape == (8, 128256)
    for row in x:
        spikes = np.sort(row)[-16:]
        rest = np.sort(row)[:-16]
        assert abs(rest.mean()) < 0.03 and abs(rest.std() - 1.5) < 0.03
        assert spikes.min() > 6.0 - 1.0  # N(0, 1.5^2) + U(6, 12) rarely drops below ~5
    # a different seed gives different bits
    y = syn.generate(w.scaled(seed=99)).logits
    assert not np.array_equal(x, y)


def test_bf16_zipf_logits():
    w = syn.CONFIGS["c4"].scaled(batch=4)
    x = syn.generate(w).logits
    assert x.dtype == np.uint16 and x.shape == (4, 152064)
    f = (x.astype(np.uint32) << 16).view(np.float32)
    assert np.isfinite(f).all()
    # the Zipf rank bias -1.1 ln(rank) makes the row mean about -1.1 (ln V - 1)
    assert abs(f.mean() - (-1.1 * (math.log(152064) - 1))) < 0.1
    # ranks follow one permutation shared by all rows, so rows correlate through the bias:
    # Var(1.1 ln rank) = 1.21 Var(ln U) = 1.21 against noise variance 4 -> 1.21 / 5.21 = 0.232
    assert abs(np.corrcoef(f[0], f[1])[0, 1] - 1.21 / 5.21) < 0.02


def test_history_repeats():
    w = syn.CONFIGS["c3"].scaled(batch=16)
    h = syn.generate(w).history
    assert h.shape == (16, 1024) and h.min() >= 0 and h.max() < w.vocab
    # with probability 0.2 a position copies an earlier id; fresh draws rarely collide
    dup = np.mean([1.0 - len(np.unique(r)) / len(r) for r in h])
    assert 0.17 < dup < 0.23


def test_mask_block_and_scatter():
    w = syn.CONFIGS["c5"].scaled(batch=8)
    m = syn.generate(w).mask
    assert m.shape == (8, (128256 + 31) // 32)
    bits = np.unpackbits(m.view(np.uint8), bitorder="little").reshape(8, -1)[:, :128256]
    block = math.ceil(0.05 * 128256)
    for row in bits:
        on = np.nonzero(row)[0]
        assert block <= len(on) <= block + 32
        # the longest run of allowed ids is the block
        runs = np.split(on, np.nonzero(np.diff(on) != 1)[0] + 1)
        assert max(len(r) for r in runs) >= block


def test_uniforms_grid():
    w = syn.CONFIGS["c3"]
    u = syn.generate(w.scaled(batch=256)).uniforms
    assert u.dtype == np.float32 and (u >= 0).all() and (u < 1).all()
    assert np.all((u * 2.0 ** 24) == np.round(u * 2.0 ** 24))  # 24 random bits
