"""arbor_sample_noalloc (the library's static device scratch as the workspace) against
arbor_sample with a caller-owned workspace, through the C ABI: the same ids, bit for bit, on
two calls in a row, the second with a smaller input (the scratch keeps the first call's
contents). Cases: streamed rows split into chunks (the chunk lists live in the scratch),
the split histogram solver (z rows, chunk records and barrier counters in the scratch,
counters cleared by a fill kernel each call), and params that need more than the scratch
holds (rejected before any launch)."""
from __future__ import annotations

import sys

import numpy as np
import pytest

from arbornet_amd import sampling as S
from arbornet_amd import synthetic as syn

from gpu_helpers import to_device

pytestmark = pytest.mark.gpu

SCRATCH = 16 << 20


@pytest.fixture(scope="module", autouse=True)
def _device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    S.library()
    yield


def _both(w: syn.Workload, write_probs=False):
    """ids (and probs) from arbor_sample_noalloc and from arbor_sample on the same inputs."""
    import torch

    inp = syn.generate(w)
    p = S.params_for(w, write_probs=write_probs)
    need = S.workspace_bytes(p)
    assert 0 < need <= SCRATCH, need
    x, h, m, u = (to_device(a, torch) for a in (inp.logits, inp.history, inp.mask, inp.uniforms))
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    stream = torch.cuda.current_stream().cuda_stream
    out = []
    for noalloc in (True, False):
        ids = torch.full((w.batch,), -100, dtype=torch.int32, device="cuda")
        probs = torch.full((w.batch, w.vocab), -1.0, dtype=torch.float32, device="cuda") if write_probs else None
        if noalloc:
            st = S.sample_noalloc_raw(p, x.data_ptr(), ptr(h), ptr(m), u.data_ptr(), ids.data_ptr(), ptr(probs), stream)
        else:
            ws = torch.full((need,), 0x5A, dtype=torch.uint8, device="cuda")
            st = S.sample_raw(p, x.data_ptr(), ptr(h), ptr(m), u.data_ptr(), ids.data_ptr(), ptr(probs),
                              ws.data_ptr(), need, stream)
        S.check(st)
        torch.cuda.synchronize()
        out.append((ids.cpu().numpy(), None if probs is None else probs.cpu().numpy()))
    return out


CASES = [
    # (label, first workload, second (smaller) workload)
    ("streamed rows in chunks (c5 shape)", syn.CONFIGS["c5"], syn.CONFIGS["c5"].scaled(batch=32, vocab=64000)),
    ("split histogram solver (top-k 200, top-p)", syn.CONFIGS["c2"].scaled(batch=8, vocab=32000, hist_len=64, top_k=200),
     syn.CONFIGS["c2"].scaled(batch=4, vocab=20000, hist_len=16, seed=9, top_k=200)),
    ("two-pass top-p kernel", syn.CONFIGS["c2"], syn.CONFIGS["c2"].scaled(batch=16, vocab=50000, seed=10)),
    ("streamed top-k, one chunk per row", syn.CONFIGS["c3"].scaled(batch=256),
     syn.CONFIGS["c3"].scaled(batch=64, vocab=50000, seed=8)),
]


@pytest.mark.parametrize("case", range(len(CASES)), ids=lambda i: CASES[i][0])
def test_noalloc_matches_workspace_call(case):
    label, first, second = CASES[case]
    for k, w in enumerate((first, second)):
        print(f"[noalloc {case}] {label}, call {k + 1}: B={w.batch} V={w.vocab}", flush=True)
        sys.stdout.flush()
        (ids_n, pr_n), (ids_w, pr_w) = _both(w, write_probs=(k == 1))
        np.testing.assert_array_equal(ids_n, ids_w, err_msg=f"{label} call {k + 1}")
        assert np.all(ids_n >= 0)
        if pr_n is not None:
            np.testing.assert_array_equal(pr_n, pr_w, err_msg=f"{label} call {k + 1} probs")


def test_noalloc_rejects_params_beyond_the_scratch():
    # top-k 300 at B=64, V=128256 takes the histogram solver, which needs a z row per row
    # (32.8 MB) and its split records: more than the 16 MB of scratch
    p = S.params_for(syn.CONFIGS["c2"].scaled(top_k=300))
    assert S.workspace_bytes(p) > SCRATCH
    st = S.sample_noalloc_raw(p, 16, 16, None, 16, 16, None, None)
    assert st == -12
    assert b"static scratch" in S.library().arbor_last_error()
