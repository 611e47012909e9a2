"""GPU parity against the committed golden fixtures, through the C ABI: ids equal the
fixture's on every row whose u is not within 1e-6 of a CDF step (boundary flag), and
probabilities within 1e-5 relative on rows with no ambiguity at all (boundary == 0)."""
from __future__ import annotations

import sys

import numpy as np
import pytest

import golden_data as G
from arbornet_amd import sampling as S
from arbornet_amd import synthetic as syn
from gpu_helpers import check_boundary_row, run_gpu
from oracle import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    S.library()
    yield


# boundary rows each fixture may hold (the fixtures' own counts: c2 5 of 64, the others 0)
MAX_BOUNDARY = {"c1": 0, "c2": 8, "c3": 2, "c4": 2, "c5": 2}


def _check_ids(ids, want, boundary, label, params=None, inp=None, max_boundary=None):
    """ids equal the fixture's on every non-boundary row; a boundary row whose id differs
    must be a legitimate draw (check_boundary_row against the oracle)."""
    bnd = (boundary & oracle.BOUNDARY_CDF) != 0
    ok = bnd | (ids == want)
    assert ok.all(), f"{label}: rows {np.nonzero(~ok)[0].tolist()} gpu {ids[~ok].tolist()} want {want[~ok].tolist()}"
    if max_boundary is not None:
        assert int(bnd.sum()) <= max_boundary, f"{label}: {int(bnd.sum())} boundary rows, more than {max_boundary}"
    for r in np.nonzero(bnd & (ids != want))[0]:
        _, info, _ = oracle.sample(params, inp.logits, inp.history, inp.mask, inp.uniforms, row0=int(r), nrows=1)
        check_boundary_row(params, inp, int(r), int(ids[r]), int(want[r]), float(info["flip_mass"][0]), label)


@pytest.mark.parametrize("case", G.small_cases(), ids=lambda c: c.name)
def test_small_fixture_gpu(case):
    print(f"[golden] {case.name}", flush=True)
    sys.stdout.flush()
    inp = syn.Inputs(case.logits, case.history, case.mask, case.uniforms)
    ids, probs = run_gpu(case.sampling_params(), inp, write_probs=True, repeat=2)
    _check_ids(ids, case.ids, case.boundary, case.name, case.sampling_params(), inp)
    for r in np.nonzero(case.boundary == 0)[0]:
        if case.ids[r] < 0:
            continue
        np.testing.assert_allclose(probs[r], case.probs[r], rtol=1e-5, atol=1e-12, err_msg=f"{case.name} row {r}")


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c4", "c5"])
def test_config_fixture_gpu(name):
    print(f"[golden] {name}", flush=True)
    man = G.config_manifest()[name]
    out = G.config_outputs()
    w = syn.CONFIGS[name]
    inp = syn.generate(w)
    assert G.sha256(inp.logits) == man["sha256"]["logits"]
    ids, _ = run_gpu(S.params_for(w), inp)
    _check_ids(ids, out[f"{name}/ids"], out[f"{name}/boundary"], name, S.params_for(w), inp, MAX_BOUNDARY[name])
