"""Host-side logic of the Python mirror (no device): integer fields that would wrap in the
int32 ABI fields are rejected, and the workspace cache keeps calls on different streams
apart."""
from __future__ import annotations

import pytest

from arbornet_amd import sampling as S


def test_row_stride_beyond_int32_is_rejected():
    # [B, seq, V] logits sliced at the last position: ld = seq * V overflows int32 at
    # seq * V >= 2^31 and must not wrap to a smaller (valid-looking) stride
    with pytest.raises(S.ArborSamplingError) as ei:
        S.SamplingParams.make(2, 131072, ld_logits=32769 * 131072)
    assert ei.value.status == -3
    p = S.SamplingParams.make(2, 131072, ld_logits=16383 * 131072)  # < 2^31: accepted unchanged
    assert p.ld_logits == 16383 * 131072
    for field in ("hist_len", "mask_words", "top_k"):
        with pytest.raises(S.ArborSamplingError):
            S.SamplingParams.make(1, 8, **{field: 2**31})
    with pytest.raises(S.ArborSamplingError):
        S.SamplingParams.make(2**31, 8)
    with pytest.raises(S.ArborSamplingError):
        S.SamplingParams.make(1, 2**32 + 8)


def test_workspace_cache_is_per_stream():
    import torch

    S._workspaces.clear()
    dev = torch.device("cpu")
    a = S._workspace(dev, 0x1000, 1024)
    b = S._workspace(dev, 0x2000, 1024)
    assert a.data_ptr() != b.data_ptr()                      # different streams: different buffers
    assert S._workspace(dev, 0x1000, 512).data_ptr() == a.data_ptr()   # same stream, fits: reused
    c = S._workspace(dev, 0x1000, 4096)                      # grows: a new buffer for that stream only
    assert c.numel() >= 4096 and c.data_ptr() != a.data_ptr()
    assert S._workspace(dev, 0x2000, 1024).data_ptr() == b.data_ptr()
    assert S._workspace(dev, None, 64).data_ptr() == S._workspace(dev, 0, 64).data_ptr()  # NULL = default
    S._workspaces.clear()
