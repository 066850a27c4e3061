"""GPU parity: the gfx950 engine (through the C-ABI) against the CPU
oracle and the certified engine (HF tokenizers 0.22.2), bit for bit."""

from __future__ import annotations

import numpy as np
import pytest

from conftest import FAMILY_NAMES, kit

pytestmark = pytest.mark.gpu

_TOKS: dict = {}


def tok(name: str):
    if name not in _TOKS:
        import toktier_amd
        _TOKS[name] = toktier_amd.load(name)
    return _TOKS[name]


SAMPLES = [
    "", "a", " ", "  ", "\n", "\r\n", "hello world", "Hello, World!",
    "it's 'S they'RE we'VE I'M you'LL he'D don't", "x'sy  'll",
    "12345 1234567 3.14159 0x1F", "  leading and trailing  ",
    "tabs\tand\tnew\nlines\r\n\r\n  \n", "naïve café résumé Ångström",
    "中文字符测试，这是一个句子。", "😀👍🏽 👨‍👩‍👧 ❤️", "!!!???...---",
    "a  b   c    d", "\t\tword", " !x", "'s", "''s", "!'s", "ſ'ſ", "'ſ",
    "foo\r\n\r\n\tbar", "x \r\n y", "end with spaces   ", " nbsp ",
]


@pytest.mark.parametrize("name", FAMILY_NAMES)
def test_samples_match_hf_and_oracle(name):
    k, t = kit(name), tok(name)
    for s in SAMPLES:
        got = list(t.encode(s).array)
        assert got == k.hf_ids(s), (name, s)


@pytest.mark.parametrize("name", FAMILY_NAMES)
def test_fuzz_alphabet(name):
    k, t = kit(name), tok(name)
    alpha = ["a", "A", "'", "s", "S", "ſ", "1", "2", " ", "\t", "\r",
             "\n", "!", "é", "中", " ", "t", "l", "e", "r",
             "v", "d", "m", "L", "E", "D", "\U0001f600", "-", "."]
    rng = np.random.default_rng(7)
    texts = ["".join(alpha[int(i)] for i in rng.integers(0, len(alpha), int(n)))
             for n in rng.integers(0, 80, size=400)]
    for s in texts:
        assert list(t.encode(s).array) == k.hf_ids(s), (name, s)


@pytest.mark.parametrize("name", FAMILY_NAMES)
def test_long_mixed_text(name):
    from toktier_amd import workloads
    k, t = kit(name), tok(name)
    fn = {"qwen3_8b": workloads.config2, "llama_3_1_8b": workloads.config4,
          "gpt2": workloads.config2}[name]
    text = fn(k.json, n_chars=300_000)
    got = t.encode(text).array
    want = k.oracle.encode_bytes(text.encode())
    assert not isinstance(want, int)
    assert np.array_equal(got, want)
    assert list(got[:2000]) == k.hf_ids(text[:0] + text)[:2000]


def test_batch_rows_equal_single():
    name = "gpt2"
    k, t = kit(name), tok(name)
    rng = np.random.default_rng(3)
    from toktier_amd import workloads
    base = workloads.config2(k.json, n_chars=50_000)
    docs = []
    for _ in range(40):
        a = int(rng.integers(0, len(base) - 1))
        docs.append(base[a:a + int(rng.integers(0, 3000))])
    docs += ["", " ", "a", "'s", "  x"]
    rows = t.encode_batch(docs)
    for d, r in zip(docs, rows):
        assert list(r.array) == k.hf_ids(d)


def _long_texts(name):
    from toktier_amd import workloads
    k = kit(name)
    rng = np.random.default_rng(11)
    base = workloads.config2(k.json, n_chars=40_000)
    letters = "".join(ch for ch in base if ch.isalpha())
    texts = [
        "a" * 300, "ab" * 200, "=" * 500, "-" * 129 + "x", " " * 200 + "x",
        "\n" * 150, "\r\n" * 100 + " y", "1" * 300, "中" * 100, "é" * 90,
        "\U0001f600" * 70, " " + "q" * 65, "'s" + "t" * 80,
        letters[:5000], letters[5000:5130], " " + letters[6000:9000],
    ]
    for _ in range(30):
        n = int(rng.integers(65, 1500))
        a = int(rng.integers(0, len(letters) - n))
        texts.append(letters[a:a + n])
    return texts


@pytest.mark.parametrize("name", FAMILY_NAMES)
def test_long_pieces(name):
    k, t = kit(name), tok(name)
    for s in _long_texts(name):
        got = list(t.encode(s).array)
        assert got == k.hf_ids(s), (name, s[:80], len(s))


def test_cjk_and_pathological_runs():
    from toktier_amd import workloads
    name = "qwen3_8b"
    k, t = kit(name), tok(name)
    text = workloads.config5(k.json, n_chars=400_000, n_runs=4, run_chars=30_000)
    data = text.encode()
    got = t.encode(text).array
    want = k.oracle.encode_bytes(data)
    assert not isinstance(want, int)
    assert np.array_equal(got, want)
