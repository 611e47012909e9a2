"""The GPU tests' rule for boundary rows, checked on the CPU against a row whose CDF is known
in closed form: eight equal logits give steps C_j = (j + 1) / 8 in id order, so
u = 0.25 + 5e-7 lies within 1e-6 of the step between ids 1 and 2. The oracle draws id 2;
id 1 is also a legitimate draw there (its step ends within the tolerance of u); ids 0, 3
and 4 are not, and neither is an id that top-k removed."""
from __future__ import annotations

import numpy as np
import pytest

from arbornet_amd import sampling as S
from arbornet_amd import synthetic as syn
from gpu_helpers import check_boundary_row
from oracle import oracle


def _row(u, **kw):
    inp = syn.Inputs(np.zeros((1, 8), np.float32), None, None, np.array([u], np.float32))
    return S.SamplingParams.make(1, 8, **kw), inp


def test_oracle_flags_the_row_and_draws_id_2():
    p, inp = _row(0.25 + 5e-7)
    ids, info, _ = oracle.sample(p, inp.logits, None, None, inp.uniforms)
    assert ids[0] == 2 and (info["boundary"][0] & oracle.BOUNDARY_CDF)
    assert info["flip_mass"][0] == 0.0


@pytest.mark.parametrize("gid", [1, 2])
def test_neighbour_across_the_step_is_accepted(gid):
    p, inp = _row(0.25 + 5e-7)
    check_boundary_row(p, inp, 0, gid, 2, 0.0, "closed form")


@pytest.mark.parametrize("gid", [0, 3, 4, -2])
def test_other_ids_are_rejected(gid):
    p, inp = _row(0.25 + 5e-7)
    with pytest.raises(AssertionError):
        check_boundary_row(p, inp, 0, gid, 2, 0.0, "closed form")


def test_removed_id_is_rejected():
    # top-k 2 keeps ids 0 and 1 (ties rank by id): C = [0.5, 1.0]; u = 0.5 + 5e-7 is a
    # boundary row between them, and id 2 (removed) is never a legitimate draw
    p, inp = _row(0.5 + 5e-7, top_k=2)
    ids, info, _ = oracle.sample(p, inp.logits, None, None, inp.uniforms)
    assert ids[0] == 1 and (info["boundary"][0] & oracle.BOUNDARY_CDF)
    check_boundary_row(p, inp, 0, 0, 1, 0.0, "top-k")
    with pytest.raises(AssertionError):
        check_boundary_row(p, inp, 0, 2, 1, 0.0, "top-k")
