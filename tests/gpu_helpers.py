"""Shared helpers for the GPU parity tests: run a workload through the C ABI and compare
with the oracle."""
from __future__ import annotations

import numpy as np

from arbornet_amd import sampling as S
from arbornet_amd import synthetic as syn
from oracle import oracle

ORACLE_THREADS = 16


def pack_mask(allowed: np.ndarray) -> np.ndarray:
    """[B, V] bool -> [B, ceil(V/32)] uint32, bit (t & 31) of word t >> 5 (LSB first)."""
    B, V = allowed.shape
    words = (V + 31) // 32
    mask = np.zeros((B, words), dtype=np.uint32)
    b, t = np.nonzero(allowed)
    np.bitwise_or.at(mask, (b, t >> 5), (np.uint32(1) << (t & 31).astype(np.uint32)))
    return mask


def to_device(a, torch):
    if a is None:
        return None
    if a.dtype == np.uint16:  # bf16 bits
        return torch.from_numpy(a.view(np.int16)).cuda().view(torch.bfloat16)
    if a.dtype == np.uint32:
        return torch.from_numpy(a.view(np.int32)).cuda()
    return torch.from_numpy(a).cuda()


def run_gpu(params: S.SamplingParams, inp: syn.Inputs, write_probs: bool = False, repeat: int = 1):
    """ids (and probs) from libarbor_hip for host inputs; params.batch must match."""
    import torch

    x = to_device(inp.logits, torch)
    h = to_device(inp.history, torch)
    m = to_device(inp.mask, torch)
    u = to_device(inp.uniforms, torch)
    B, V = params.batch, params.vocab
    ids = torch.full((B,), -100, dtype=torch.int32, device="cuda")
    probs = torch.full((B, V), -1.0, dtype=torch.float32, device="cuda") if write_probs else None
    if write_probs:
        params.flags |= S.ARBOR_FLAG_WRITE_PROBS
    need = S.workspace_bytes(params)
    assert need > 0, S.library().arbor_last_error()
    ws = torch.full((need,), 0xA5, dtype=torch.uint8, device="cuda")  # no initialisation needed
    stream = torch.cuda.current_stream().cuda_stream
    outs = []
    for _ in range(repeat):
        st = S.sample_raw(params, x.data_ptr(), None if h is None else h.data_ptr(),
                          None if m is None else m.data_ptr(), u.data_ptr(), ids.data_ptr(),
                          None if probs is None else probs.data_ptr(), ws.data_ptr(), need, stream)
        S.check(st)
        torch.cuda.synchronize()
        outs.append(ids.cpu().numpy().copy())
    for o in outs[1:]:
        np.testing.assert_array_equal(o, outs[0], err_msg="GPU result not deterministic across calls")
    return outs[0], (probs.cpu().numpy() if write_probs else None)


BOUNDARY_TOL = 1e-6  # the oracle's BOUNDARY_TOL: |C_j - u| below this flags a boundary row


def check_boundary_row(params, inp: syn.Inputs, r: int, gid: int, oid: int, flip_mass: float, label=""):
    """A boundary row's GPU id must still be a legitimate draw: a kept id (or, when the
    top-p / min-p membership of some ids is ambiguous, an id at the edge of the kept set)
    whose CDF step in ascending id order brackets u to within BOUNDARY_TOL plus the
    ambiguous mass, and, when no membership is ambiguous, the oracle's id or its immediate
    neighbour in ascending kept-id order."""
    _, _, pr = oracle.sample(params, inp.logits, inp.history, inp.mask, inp.uniforms, row0=r, nrows=1, probs=True)
    q = pr[0].astype(np.float64)
    kept = np.nonzero(q > 0)[0]
    u = float(inp.uniforms[r])
    tol = BOUNDARY_TOL + flip_mass + 1e-7  # + fp32 rounding of the oracle's q
    assert gid >= 0, f"{label}: boundary row {r}: gpu gave sentinel {gid}, oracle {oid}"
    before = float(q[kept[kept < gid]].sum())
    step = float(q[gid]) if gid < q.size else 0.0
    ok_cdf = before - tol <= u <= before + step + tol
    assert ok_cdf, (f"{label}: boundary row {r}: gpu id {gid} spans CDF [{before:.9f}, {before + step:.9f}] "
                    f"which misses u = {u:.9f} by more than {tol:.2e} (oracle id {oid})")
    if flip_mass == 0.0:
        pg, po = np.searchsorted(kept, gid), np.searchsorted(kept, oid)
        assert pg < kept.size and kept[pg] == gid, f"{label}: boundary row {r}: gpu id {gid} is not kept"
        assert abs(int(pg) - int(po)) <= 1, (f"{label}: boundary row {r}: gpu id {gid} is {int(pg) - int(po)} "
                                              f"kept places from the oracle's {oid}")


def compare(params, inp: syn.Inputs, ids_gpu, probs_gpu=None, label="", fp_rtol=1e-5, max_boundary=None):
    """Assert GPU ids equal the oracle's on every non-boundary row, and that every boundary
    row's id passes check_boundary_row; probs within fp_rtol where the kept sets agree.
    max_boundary, when given, bounds the number of boundary rows (the benchmark
    configurations state theirs; rows built to tie, such as all-equal logits, are boundary
    rows by construction). Returns (n_rows, n_boundary, n_boundary_mismatch)."""
    want_probs = probs_gpu is not None
    ids_o, info, probs_o = oracle.sample(params, inp.logits, inp.history, inp.mask, inp.uniforms,
                                         probs=want_probs, threads=ORACLE_THREADS)
    boundary = (info["boundary"] & oracle.BOUNDARY_CDF) != 0
    bad = (ids_gpu != ids_o) & ~boundary
    if bad.any():
        rows = np.nonzero(bad)[0][:10]
        detail = [(int(r), int(ids_gpu[r]), int(ids_o[r]), int(info["n_kept"][r]), float(info["cdf_gap"][r]))
                  for r in rows]
        raise AssertionError(f"{label}: {int(bad.sum())} non-boundary rows differ "
                             f"(row, gpu, oracle, kept, gap): {detail}")
    n_rows = len(ids_o)
    limit = n_rows if max_boundary is None else max_boundary
    assert int(boundary.sum()) <= limit, f"{label}: {int(boundary.sum())} boundary rows, more than {limit}"
    for r in np.nonzero(boundary & (ids_gpu != ids_o))[0]:
        check_boundary_row(params, inp, int(r), int(ids_gpu[r]), int(ids_o[r]), float(info["flip_mass"][r]), label)
    if want_probs:
        clean = info["flip_mass"] == 0.0
        for r in np.nonzero(clean)[0]:
            g, o = probs_gpu[r], probs_o[r]
            nz_g, nz_o = g != 0, o != 0
            if not np.array_equal(nz_g, nz_o):
                diff = np.nonzero(nz_g != nz_o)[0][:8]
                raise AssertionError(f"{label}: row {r} kept sets differ at ids {diff.tolist()}")
            np.testing.assert_allclose(g[nz_o], o[nz_o], rtol=fp_rtol, atol=0,
                                       err_msg=f"{label}: row {r} probabilities")
    n_bnd = int(boundary.sum())
    n_bnd_mis = int(((ids_gpu != ids_o) & boundary).sum())
    return len(ids_o), n_bnd, n_bnd_mis
