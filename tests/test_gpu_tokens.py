"""GPU: token decoding (arbor_decode) and the embedding gather (arbor_embed) against the CPU
restatement in oracle/tokens.py, through the C ABI. Decoded bytes and gathered rows must be
identical (byte moves, nothing rounded)."""
from __future__ import annotations

import sys

import numpy as np
import pytest

from arbornet_amd import sampling as S
from arbornet_amd import synthetic as syn
from oracle import tokens as T

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    S.library()
    yield


def _announce(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _random_vocab(n, seed):
    """A vocabulary of n ids with multi-byte pieces, some ids missing, one id shared by two keys."""
    rng = np.random.default_rng(seed)
    alphabet = list("abcdefghijklmnopqrstuvwxyz ") + ["é", "ß", "→", "日", "本", "🙂"]
    vocab = {"<unk>": 0}
    for i in range(1, n):
        if rng.random() < 0.02:
            continue  # a missing id decodes as <unk>
        piece = "".join(rng.choice(alphabet, size=int(rng.integers(1, 8))))
        while piece in vocab:
            piece += "x"
        vocab[piece] = i
    vocab["shared-second"] = 1  # FirstOrDefault keeps the first key of id 1
    return vocab


@pytest.mark.parametrize("n_ids", [1, 256, 5000])
def test_decode_matches_oracle(n_ids):
    import torch

    vocab = _random_vocab(32000, seed=n_ids)
    table = S.TokenTable(vocab, "<unk>")
    rng = np.random.default_rng(7 + n_ids)
    ids = rng.integers(0, 32000, size=n_ids).astype(np.int32)
    ids[: min(4, n_ids)] = [-1, -4, 32000, 1][: min(4, n_ids)]  # sentinels and out-of-range: <unk>
    _announce(f"[decode] {n_ids} ids")
    got = table.decode(torch.from_numpy(ids).cuda())
    assert got == T.decode(vocab, "<unk>", ids)


def test_decode_reports_size_when_capacity_is_short():
    import torch

    vocab = _random_vocab(1000, seed=3)
    table = S.TokenTable(vocab, "<unk>")
    ids = torch.arange(1, 300, dtype=torch.int32).cuda()
    want = T.decode(vocab, "<unk>", ids.cpu().numpy()).encode("utf-8")
    offs, out = table.decode_raw(ids, capacity=100)
    torch.cuda.synchronize()
    assert int(offs[-1].item()) == len(want)  # the full size, though only 100 bytes were written
    assert bytes(out[:100].cpu().numpy()) == want[:100]
    starts = offs[:-1].cpu().numpy()
    assert np.all(np.diff(starts) >= 0) and starts[0] == 0


@pytest.mark.parametrize("dtype,width", [("f32", 4096), ("f32", 1001), ("bf16", 4096), ("bf16", 333)])
def test_embed_matches_gather(dtype, width):
    import torch

    vocab = 5000
    rng = np.random.default_rng(width)
    table = torch.from_numpy(rng.standard_normal((vocab, width)).astype(np.float32)).cuda()
    if dtype == "bf16":
        table = table.to(torch.bfloat16)
    ids = rng.integers(0, vocab, size=257).astype(np.int32)
    ids[:3] = [-1, vocab, -3]  # no row: zeros
    _announce(f"[embed] {dtype} width {width}")
    out = S.embed(torch.from_numpy(ids).cuda(), table)
    torch.cuda.synchronize()
    if dtype == "bf16":
        got = out.view(torch.int16).cpu().numpy()
        want = T.embed(table.view(torch.int16).cpu().numpy(), ids)
    else:
        got = out.cpu().numpy()
        want = T.embed(table.cpu().numpy(), ids)
    np.testing.assert_array_equal(got, want)


def test_generation_step_then_embed_and_decode():
    # the device half of a generation loop: sample the last position, append the ids to the
    # history ring, gather their embedding rows and decode them, without leaving the device
    import torch

    w = syn.CONFIGS["c3"].scaled(batch=16, vocab=32000)
    inp = syn.generate(w)
    state = S.GenerationState(w.batch, w.hist_len, "cuda:0")
    state.history.copy_(torch.from_numpy(inp.history))
    logits = torch.from_numpy(inp.logits).cuda()
    ids = state.step(logits, torch.from_numpy(inp.uniforms), temperature=w.temperature, top_k=w.top_k,
                     top_p=w.top_p, repetition_penalty=w.repetition_penalty)
    emb_table = torch.randn(w.vocab, 512, device="cuda")
    rows = S.embed(ids, emb_table)
    vocab = _random_vocab(w.vocab, seed=11)
    text = S.TokenTable(vocab, "<unk>").decode(ids)
    torch.cuda.synchronize()
    ids_h = ids.cpu().numpy()
    assert np.all(ids_h >= 0)
    np.testing.assert_array_equal(rows.cpu().numpy(), T.embed(emb_table.cpu().numpy(), ids_h))
    assert text == T.decode(vocab, "<unk>", ids_h)
