"""CPU: pin the restatement of the session store's span checkpoints
(``oracle.span_checkpoints``, ``tail.rs:173-205``) and the token byte
lengths it walks, before the GPU seed is checked against them."""

from __future__ import annotations

import numpy as np
import pytest

from conftest import kit
from oracle.oracle import span_checkpoints, token_byte_lengths


def test_ascii_checkpoints_are_the_prefix_sums():
    data = b"hello world"
    lens = np.array([0, 5, 1, 5], dtype=np.int64)  # ids 1..3: "hello" " " "world"
    pts = span_checkpoints(data, [1, 2, 3], lens, 1)
    assert pts.tolist() == [[0, 0, 0], [5, 5, 5], [6, 6, 6]]
    assert span_checkpoints(data, [1, 2, 3], lens, 2).tolist() == [[0, 0, 0], [6, 6, 6]]
    assert span_checkpoints(data, [1, 2, 3], lens, 4096).tolist() == [[0, 0, 0]]
    assert span_checkpoints(b"", [], lens, 4).shape == (0, 3)


def test_checkpoints_inside_characters_anchor_to_the_character():
    # "é中a" = c3 a9 | e4 b8 ad | 61; tokens split both characters:
    # bytes [0,1) [1,3) [3,5) [5,6)
    data = "é中a".encode()
    lens = np.array([1, 2, 2, 1], dtype=np.int64)
    pts = span_checkpoints(data, [0, 1, 2, 3], lens, 1)
    # byte 1 lies inside é (anchor 0, char 0); byte 3 inside 中 (anchor 2,
    # char 1); byte 5 is 'a' (char 2)
    assert pts.tolist() == [[0, 0, 0], [1, 0, 0], [3, 2, 1], [5, 5, 2]]


def test_tokens_must_close_over_the_text():
    lens = np.array([3, 0], dtype=np.int64)
    with pytest.raises(ValueError):
        span_checkpoints(b"abcd", [0], lens, 1)       # 3 of 4 bytes
    with pytest.raises(ValueError):
        span_checkpoints(b"abc", [1], lens, 1)        # an id without bytes


@pytest.mark.parametrize("name", ["qwen3_8b", "deepseek_v3"])
def test_token_byte_lengths_close_over_hf_encodings(name):
    """The byte lengths of the certified engine's ids sum to the text's
    byte length, chat literals included, and the checkpoints taken from
    them land on the byte offsets of a direct walk."""
    from toktier_amd import workloads
    k = kit(name)
    lens = token_byte_lengths(k.json)
    for t in k.added:
        lens[t.id] = len(t.content.encode("utf-8"))
    text = workloads.chat(k.json, name, n_chars=20_000)
    data = text.encode("utf-8")
    ids = k.hf_ids(text)
    assert int(lens[np.asarray(ids)].sum()) == len(data)
    pts = span_checkpoints(data, ids, lens, 97)
    offs = np.concatenate([[0], np.cumsum(lens[np.asarray(ids)])[:-1]])
    assert pts[:, 0].tolist() == offs[::97].tolist()
    for byte, a, c in pts.tolist():
        assert a <= byte < a + 4 and len(data[:a].decode("utf-8")) == c
