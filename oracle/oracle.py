"""ctypes wrapper of the CPU oracle (oracle/sampling_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker, never as the thing measured or
shipped.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

_DIR = Path(__file__).resolve().parent
LIB_PATH = _DIR / "_build" / "liboracle_sampling.so"
SOURCE = _DIR / "sampling_oracle.c"

BOUNDARY_CDF = 1
BOUNDARY_TOP_P = 2
BOUNDARY_MIN_P = 4

ROW_INFO_DTYPE = np.dtype([
    ("id", np.int32), ("n_finite", np.int32), ("n_topk", np.int32), ("n_topp", np.int32),
    ("n_kept", np.int32), ("cut_id", np.int32), ("cut_z", np.float32), ("max_z", np.float32),
    ("boundary", np.uint32), ("reserved", np.uint32), ("kept_mass", np.float64), ("cdf_gap", np.float64),
    ("flip_mass", np.float64),
])


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(_DIR)], check=True)
    return LIB_PATH


def build_variant(out: Path, defines: dict[str, int]) -> Path:
    """Compile the oracle with extra -D definitions (planted-mistake variants in tests)."""
    cmd = ["gcc", "-O2", "-fPIC", "-shared", "-std=c11", "-fopenmp", "-ffp-contract=off", "-fno-fast-math",
           *[f"-D{k}={v}" for k, v in defines.items()], str(SOURCE), "-o", str(out), "-lm"]
    subprocess.run(cmd, check=True)
    return out


def _ptr(a):
    return None if a is None else a.ctypes.data


class Oracle:
    """One loaded oracle library."""

    def __init__(self, path: Path = LIB_PATH):
        if not Path(path).exists():
            raise RuntimeError(f"{path} is not built; run `make -C oracle`")
        L = ctypes.CDLL(str(path))
        vp, i32 = ctypes.c_void_p, ctypes.c_int
        L.oracle_sample.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32]
        L.oracle_sample.restype = i32
        L.oracle_tempered_row.argtypes = [vp, vp, vp, vp, vp]
        L.oracle_tempered_row.restype = i32
        L.oracle_info_size.restype = i32
        assert L.oracle_info_size() == ROW_INFO_DTYPE.itemsize, "oracle_row_info layout mismatch"
        self.lib = L

    def sample(self, params, logits: np.ndarray, history, mask, uniforms: np.ndarray, *, row0: int = 0,
               nrows: int | None = None, probs: bool = False, threads: int = 1):
        """Rows [row0, row0+nrows) of the batch `params` describes (arrays hold the whole
        batch). Returns (ids, info, probs or None)."""
        n = params.batch - row0 if nrows is None else nrows
        ids = np.empty(n, dtype=np.int32)
        info = np.zeros(n, dtype=ROW_INFO_DTYPE)
        pr = np.empty((n, params.vocab), dtype=np.float32) if probs else None
        logits = np.ascontiguousarray(logits)
        history = None if history is None else np.ascontiguousarray(history, dtype=np.int32)
        mask = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint32)
        uniforms = np.ascontiguousarray(uniforms, dtype=np.float32)
        st = self.lib.oracle_sample(ctypes.byref(params), _ptr(logits), _ptr(history), _ptr(mask), _ptr(uniforms),
                                    _ptr(ids), _ptr(pr), _ptr(info), row0, n, threads)
        if st != 0:
            raise ValueError(f"oracle_sample status {st}")
        return ids, info, pr

    def tempered_row(self, params, logits_row: np.ndarray, history_row, mask_row) -> tuple[int, np.ndarray]:
        """Contract steps 1-3 for one row: (status, z[vocab])."""
        z = np.empty(params.vocab, dtype=np.float32)
        logits_row = np.ascontiguousarray(logits_row)
        h = None if history_row is None else np.ascontiguousarray(history_row, dtype=np.int32)
        m = None if mask_row is None else np.ascontiguousarray(mask_row, dtype=np.uint32)
        st = self.lib.oracle_tempered_row(ctypes.byref(params), _ptr(logits_row), _ptr(h), _ptr(m), _ptr(z))
        return st, z


_default: Oracle | None = None


def default() -> Oracle:
    global _default
    if _default is None:
        _default = Oracle(LIB_PATH)
    return _default


def sample(params, logits, history, mask, uniforms, **kw):
    return default().sample(params, logits, history, mask, uniforms, **kw)


def tempered_row(params, logits_row, history_row, mask_row):
    return default().tempered_row(params, logits_row, history_row, mask_row)
