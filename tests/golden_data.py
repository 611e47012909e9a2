"""Loaders of the committed golden fixtures (tests/golden/, written by make_golden.py)."""
from __future__ import annotations

import hashlib
import json
from dataclasses import dataclass
from functools import lru_cache
from pathlib import Path

import numpy as np

from arbornet_amd import sampling as S

GOLDEN = Path(__file__).resolve().parent / "golden"


@dataclass
class SmallCase:
    name: str
    params: dict
    logits: np.ndarray
    history: np.ndarray | None
    mask: np.ndarray | None
    uniforms: np.ndarray
    ids: np.ndarray
    n_kept: np.ndarray
    boundary: np.ndarray
    kept_mass: np.ndarray
    probs: np.ndarray

    def sampling_params(self) -> S.SamplingParams:
        d = dict(self.params)
        B, V = d.pop("batch"), d.pop("vocab")
        d.pop("struct_size")
        return S.SamplingParams.make(B, V, **d)


@lru_cache(maxsize=1)
def small_cases() -> list[SmallCase]:
    man = json.loads((GOLDEN / "small.json").read_text())
    z = np.load(GOLDEN / "small.npz")
    out = []
    for c in man["cases"]:
        n = c["name"]
        get = lambda k: z[f"{n}/{k}"] if f"{n}/{k}" in z.files else None  # noqa: E731
        out.append(SmallCase(n, c["params"], get("logits"), get("history"), get("mask"), get("uniforms"),
                             get("ids"), get("n_kept"), get("boundary"), get("kept_mass"), get("probs")))
    return out


@lru_cache(maxsize=1)
def config_manifest() -> dict:
    return json.loads((GOLDEN / "configs.json").read_text())


@lru_cache(maxsize=1)
def config_outputs():
    return np.load(GOLDEN / "configs.npz")


def sha256(a) -> str | None:
    return None if a is None else hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()
