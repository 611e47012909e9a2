"""The CPU oracle against closed forms, known answers, a separately written brute-force
sampler and invariants (see oracle_pins.py), and the same checks against planted mistakes:
each of the oracle's mutation hooks (ORACLE_MUTATION in sampling_oracle.c) must be caught."""
from __future__ import annotations

import pytest

import oracle_pins
from oracle import oracle

MUTATIONS = {
    1: "frequency/presence penalty added instead of subtracted",
    2: "repetition penalty multiplies positive logits",
    3: "ties ranked by descending id",
    4: "draw takes the first C_j >= u",
    5: "top-p keeps the prefix with mass > top_p",
    6: "CDF accumulated in rank order instead of id order",
    7: "temperature as a true division",
    8: "allow-mask read MSB-first",
    9: "min-p relative to the total instead of the best token",
    10: "frequency penalty ignores the count",
}


@pytest.mark.parametrize("check", oracle_pins.ALL, ids=lambda c: c.__name__)
def test_oracle_pinned(check):
    assert check(oracle.default()) == []


@pytest.fixture(scope="module")
def mutant_dir(tmp_path_factory):
    return tmp_path_factory.mktemp("oracle_mutants")


@pytest.mark.parametrize("mutation", sorted(MUTATIONS), ids=lambda m: MUTATIONS[m].replace(" ", "_"))
def test_planted_mistake_is_caught(mutation, mutant_dir):
    lib = oracle.build_variant(mutant_dir / f"liboracle_m{mutation}.so", {"ORACLE_MUTATION": mutation})
    failures = oracle_pins.run_all(oracle.Oracle(lib))
    assert failures, f"mutation {mutation} ({MUTATIONS[mutation]}) passed every pin"
