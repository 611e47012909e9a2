"""CPU restatement of the two steps around a sampled id: decoding ids to text and gathering
their embedding rows.

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker of arbor_decode and arbor_embed,
never by the product path.

- decode follows the reference's Decode (ArborNet.Data/Tokenizers.cs:191-200 for BPE,
  :304-313 for SentencePiece): for each id, the first key of the vocabulary, in the
  dictionary's enumeration order, whose value is the id (FirstOrDefault), else the unknown
  token; the pieces are joined with "" between them. Ids outside the vocabulary find no
  key, so they decode as the unknown token too.
- embed is what ArborNet.Layers/Embedding.cs:53-57 means to compute (its Forward returns
  the weight table, a stub): row i of the output is row ids[i] of the table. Ids that name
  no row (the sampler's negative sentinels, ids past the table) give zero rows, the
  convention of the device gather.
"""
from __future__ import annotations

import numpy as np


def decode(vocab: dict, unk_token: str, ids) -> str:
    pieces = []
    for t in ids:
        t = int(t)
        piece = next((k for k, v in vocab.items() if v == t), None)  # FirstOrDefault(kvp => kvp.Value == t)
        pieces.append(unk_token if piece is None else piece)
    return "".join(pieces)


def embed(table: np.ndarray, ids) -> np.ndarray:
    ids = np.asarray(ids, dtype=np.int64)
    out = np.zeros((ids.size, table.shape[1]), dtype=table.dtype)
    ok = (ids >= 0) & (ids < table.shape[0])
    out[ok] = table[ids[ok]]
    return out
