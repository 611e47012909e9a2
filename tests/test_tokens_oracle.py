"""Pins of the CPU restatement of token decoding and the embedding gather (oracle/tokens.py)
by closed-form cases, each chosen so that a plausible mistake fails it: the first key wins
when several map to one id (FirstOrDefault), unknown and out-of-range ids give the unknown
token, pieces are joined with nothing between them, and the gather picks row ids[i]."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import tokens as T


def test_decode_joins_pieces_without_separator():
    vocab = {"he": 0, "llo": 1, " ": 2, "world": 3, "<unk>": 4}
    assert T.decode(vocab, "<unk>", [0, 1, 2, 3]) == "hello world"
    assert T.decode(vocab, "<unk>", []) == ""


def test_first_key_wins_for_a_shared_id():
    vocab = {"<unk>": 0, "a": 5, "b": 5}
    assert T.decode(vocab, "<unk>", [5, 5]) == "aa"


@pytest.mark.parametrize("bad", [7, -1, -4, 1 << 20])
def test_unknown_ids_decode_as_the_unknown_token(bad):
    vocab = {"x": 0, "y": 1, "?": 2}
    assert T.decode(vocab, "?", [0, bad, 1]) == "x?y"


def test_unicode_pieces():
    assert T.decode({"é": 0, "→": 1, "日本": 2}, "<u>", [2, 1, 0]) == "日本→é"


def test_embed_picks_rows_and_zeroes_sentinels():
    table = (np.arange(6)[:, None] * 1000 + np.arange(4)[None, :]).astype(np.float32)
    out = T.embed(table, [3, 0, -1, 5, 6])
    np.testing.assert_array_equal(out[0], [3000, 3001, 3002, 3003])
    np.testing.assert_array_equal(out[1], [0, 1, 2, 3])
    np.testing.assert_array_equal(out[2], 0)
    np.testing.assert_array_equal(out[3], [5000, 5001, 5002, 5003])
    np.testing.assert_array_equal(out[4], 0)


def test_planted_mistakes_fail_a_pin():
    # a decode that takes the last key for a shared id, or joins with spaces, or maps
    # unknown ids to "" fails at least one of the cases above
    vocab = {"<unk>": 0, "a": 5, "b": 5}

    def last_key(v, unk, ids):
        return "".join(next((k for k, x in reversed(list(v.items())) if x == t), unk) for t in ids)

    def spaced(v, unk, ids):
        return " ".join(next((k for k, x in v.items() if x == t), unk) for t in ids)

    def empty_unknown(v, unk, ids):
        return "".join(next((k for k, x in v.items() if x == t), "") for t in ids)

    assert last_key(vocab, "<unk>", [5]) != T.decode(vocab, "<unk>", [5])
    assert spaced(vocab, "<unk>", [5, 5]) != T.decode(vocab, "<unk>", [5, 5])
    assert empty_unknown(vocab, "<unk>", [9]) != T.decode(vocab, "<unk>", [9])
