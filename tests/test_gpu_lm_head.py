"""GPU: the LM head (arbor_lm_head, through the C ABI) against a float64 product of the same
bf16-rounded operands on the CPU. The kernel multiplies bf16 operands exactly and sums in
fp32, so the only differences are fp32 summation orders: every logit must be within
2e-6 * sum_h |x_h w_h| + 1e-6 of the float64 value (H <= 4096 terms: a worst-case fp32
order error is ~H * 6e-8 of that sum, a typical one ~sqrt(H) * 6e-8). bf16 outputs must
equal the float64 value rounded to bf16, or be one bf16 step from it when the value lies
within the fp32 tolerance of a rounding boundary. row_max must equal the maximum of the
stored row."""
from __future__ import annotations

import sys

import numpy as np
import pytest

from arbornet_amd import sampling as S

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    S.library()
    yield


def _bf16_round(a: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 (round to nearest even) -> fp32, as numpy float32."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def _announce(msg):
    print(msg, flush=True)
    sys.stdout.flush()


CASES = [
    # (B, H, V, x dtype, weight dtype, layout, logits dtype, bias, scale, column sample)
    (1, 128, 1000, "f32", "f32", "hv", "f32", True, 1.0, None),
    (7, 512, 32000, "bf16", "bf16", "hv", "f32", True, 1.0 / 0.7, None),
    (32, 256, 5003, "f32", "bf16", "vh", "f32", False, 1.0, None),
    (100, 1024, 32000, "bf16", "f32", "vh", "bf16", True, 1.0, None),
    (256, 4096, 128256, "bf16", "bf16", "hv", "f32", True, 1.0, 3000),  # the LM-head shape of c3
    (300, 128, 4096, "f32", "f32", "hv", "f32", True, 2.0, None),  # two launches (256 + 44 rows)
    (65, 384, 777, "f32", "f32", "vh", "bf16", False, 0.5, None),
]


@pytest.mark.parametrize("case", range(len(CASES)), ids=lambda i: "B{}-H{}-V{}-x{}-w{}-{}-o{}".format(*CASES[i][:7]))
def test_lm_head_matches_float64(case):
    import torch

    B, H, V, xdt, wdt, layout, odt, with_bias, scale, sample = CASES[case]
    _announce(f"[lm_head {case}] B={B} H={H} V={V} x {xdt} w {wdt} {layout} out {odt} scale {scale}")
    rng = np.random.default_rng(100 + case)
    x = (rng.standard_normal((B, H)) * 0.5).astype(np.float32)
    w_hv = (rng.standard_normal((H, V)) / np.sqrt(H)).astype(np.float32)  # [hidden, vocab]
    bias = (rng.standard_normal(V) * 0.1).astype(np.float32) if with_bias else None
    tdt = {"f32": torch.float32, "bf16": torch.bfloat16}
    w_host = w_hv if layout == "hv" else np.ascontiguousarray(w_hv.T)
    w_dev = torch.from_numpy(w_host).to("cuda", dtype=tdt[wdt]).contiguous()
    head = S.LMHead(w_dev, None if bias is None else torch.from_numpy(bias).cuda(), layout=layout)
    # x with a row stride beyond H (aligned), as a model's hidden-state buffer may have
    x_pad = np.zeros((B, H + 64), dtype=np.float32)
    x_pad[:, :H] = x
    x_dev = torch.from_numpy(x_pad).to("cuda", dtype=tdt[xdt])[:, :H]
    out = torch.full((B, V + 3), float("nan"), dtype=tdt[odt], device="cuda")[:, :V] if odt == "f32" else None
    got, rm = head(x_dev, scale=scale, out_dtype=tdt[odt], out=out, row_max=True)
    torch.cuda.synchronize()
    got = got.float().cpu().numpy()
    rm = rm.cpu().numpy()

    xr = _bf16_round(x).astype(np.float64)
    wr = _bf16_round(w_hv).astype(np.float64)
    cols = np.arange(V) if sample is None else np.sort(rng.choice(V, size=sample, replace=False))
    want = xr @ wr[:, cols]
    mag = np.abs(xr) @ np.abs(wr[:, cols])
    if bias is not None:
        want = want + bias[cols].astype(np.float64)
        mag = mag + np.abs(bias[cols]).astype(np.float64)
    want *= scale
    mag *= abs(scale)
    tol = 2e-6 * mag + 1e-6
    g = got[:, cols].astype(np.float64)
    if odt == "f32":
        err = np.abs(g - want)
        assert np.all(err <= tol), f"max err {err.max():.3e} at {np.unravel_index(np.argmax(err - tol), err.shape)}"
    else:
        lo = _bf16_round((want - tol).astype(np.float32)).astype(np.float64)
        hi = _bf16_round((want + tol).astype(np.float32)).astype(np.float64)
        ok = (g >= np.minimum(lo, hi)) & (g <= np.maximum(lo, hi))
        assert ok.all(), f"{(~ok).sum()} bf16 logits outside the rounding of the float64 value"
    np.testing.assert_array_equal(rm, got.max(axis=1))


def test_lm_head_then_sample():
    # the two steps back to back on the device: the LM head's logits feed arbor_sample,
    # whose ids must equal sampling the same logits handed over as a plain tensor
    import torch

    B, H, V = 64, 512, 32000
    rng = np.random.default_rng(5)
    w = torch.from_numpy((rng.standard_normal((H, V)) / np.sqrt(H) * 4).astype(np.float32)).cuda()
    head = S.LMHead(w)
    x = torch.from_numpy(rng.standard_normal((B, H)).astype(np.float32)).cuda()
    logits = head(x)
    u = torch.from_numpy(rng.random(B).astype(np.float32)).cuda()
    ids = S.Sampling.sample(logits, u, temperature=0.8, top_k=40, top_p=0.9)
    ids2 = S.Sampling.sample(logits.clone(), u, temperature=0.8, top_k=40, top_p=0.9)
    torch.cuda.synchronize()
    assert np.all(ids.cpu().numpy() >= 0)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids2.cpu().numpy())
