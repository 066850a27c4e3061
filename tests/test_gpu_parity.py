"""GPU parity: the gfx950 engine (through the C-ABI) against the CPU
oracle and the certified engine (HF tokenizers 0.22.2), bit for bit."""

from __future__ import annotations

import numpy as np
import pytest

from conftest import FAMILY_NAMES, kit

pytestmark = pytest.mark.gpu


def _pt_tile() -> int:
    """The pretokenizer's tile in bytes (PT_TILE in the device header)."""
    import re
    from pathlib import Path
    h = Path(__file__).resolve().parent.parent / "toktier_amd" / "csrc" / "tk_device.h"
    return int(re.search(r"constexpr int PT_TILE = (\d+);", h.read_text()).group(1))


TILE = _pt_tile()

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
          "gpt2": workloads.config2, "laguna_s_2_1": workloads.config4,
          "gpt_oss_120b": lambda js, n_chars: workloads.config5(
              js, n_chars=n_chars, n_runs=4, run_chars=20_000),
          "kimi_k3": lambda js, n_chars: workloads.config5(
              js, n_chars=n_chars, n_runs=4, run_chars=20_000),
          "deepseek_v3": lambda js, n_chars: workloads.config5(
              js, n_chars=n_chars, n_runs=4, run_chars=20_000),
          "nemotron_3_nano_4b": lambda js, n_chars: workloads.config5(
              js, n_chars=n_chars, n_runs=4, run_chars=20_000),
          "qwen3_5_08b": _qwen35_mixed}[name]
    text = fn(k.json, n_chars=300_000)
    got = t.encode(text).array
    want = k.expected(text)
    assert not isinstance(want, int)
    assert np.array_equal(got, want)
    assert list(got[:2000]) == k.hf_ids(text[:0] + text)[:2000]


def _qwen35_mixed(js: str, n_chars: int) -> str:
    """Mixed text and lines dense in combining marks (Devanagari, Thai,
    stacked accents), NFC-normal."""
    import unicodedata
    from toktier_amd import standin, workloads
    marks = "\n".join(standin._mark_corpus(5, 2000))
    return unicodedata.normalize(
        "NFC", workloads.config2(js, n_chars=n_chars) + "\n" + marks)


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


def test_golden_vectors_through_the_c_abi():
    import json
    from pathlib import Path
    g = json.loads((Path(__file__).resolve().parent / "golden" /
                    "golden_ids.json").read_text(encoding="utf-8"))
    for name in FAMILY_NAMES:
        t = tok(name)
        for case in g["families"][name]["cases"]:
            assert list(t.encode(case["text"]).array) == case["ids"], (name, case["text"])


@pytest.mark.parametrize("cfg", [1, 2, 4, 5])
def test_full_size_configs_match_oracle(cfg):
    from toktier_amd import workloads
    name, gen = workloads.CONFIGS[cfg]
    k, t = kit(name), tok(name)
    data = gen(k.json).encode()
    got = t.encode_bytes(data)
    want = k.oracle.encode_bytes(data)
    assert not isinstance(want, int)
    assert np.array_equal(got, want)
    if cfg == 1:
        assert list(got) == k.hf_ids(data.decode())


@pytest.mark.family("gpt2")
def test_full_size_batch_config3_rows():
    from toktier_amd import workloads
    k, t = kit("gpt2"), tok("gpt2")
    docs = workloads.config3(k.json)
    rows = t.encode_batch(docs)
    assert len(rows) == len(docs)
    for d, r in zip(docs, rows):
        want = k.oracle.encode_bytes(d.encode())
        assert np.array_equal(r.array, want)


@pytest.mark.family("qwen3_8b")
def test_nfc_fallback_matches_hf():
    k, t = kit("qwen3_8b"), tok("qwen3_8b")
    texts = ["cafe\u0301 au lait", "A\u030a and \u212b", "e\u0301\u0323",
             "plain ascii", "\u1e9b\u0323 \uac00\u11a8",
             "x" * 70 + "e\u0301" * 40]
    for s in texts:
        assert list(t.encode(s).array) == k.hf_ids(s), s
    rows = t.encode_batch(texts)
    for s, r in zip(texts, rows):
        assert list(r.array) == k.hf_ids(s), s


@pytest.mark.family("gpt2")
def test_invalid_utf8_is_an_error():
    from toktier_amd import _ffi
    t = tok("gpt2")
    for bad in (b"\xff", b"ok\xc3", b"\xc0\x80", b"\xed\xa0\x80 x", b"\x80"):
        with pytest.raises(_ffi.EngineError) as err:
            t.engine.encode(bad)
        assert err.value.status == _ffi.TK_E_UTF8


@pytest.mark.family("qwen3_8b")
def test_device_resident_entry_and_determinism():
    import torch
    from toktier_amd import workloads
    k, t = kit("qwen3_8b"), tok("qwen3_8b")
    data = workloads.config5(k.json, n_chars=200_000, n_runs=2,
                             run_chars=10_000).encode()
    d_text = torch.frombuffer(bytearray(data), dtype=torch.uint8).to("cuda:0")
    d_ids = torch.empty(len(data), dtype=torch.int32, device="cuda:0")
    want = k.oracle.encode_bytes(data)
    for _ in range(3):
        n = t.engine.encode_device(d_text.data_ptr(), len(data),
                                   d_ids.data_ptr(), len(data))
        got = d_ids[:n].cpu().numpy().view(np.uint32)
        assert np.array_equal(got, want)


@pytest.mark.parametrize("name", ["deepseek_v3", "laguna_s_2_1"])
def test_batch_rows_equal_single_with_region_cuts(name):
    """Document boundaries at arbitrary offsets of CJK / digit / newline
    runs: every row equals the oracle's encode of that document alone."""
    from toktier_amd import workloads
    k, t = kit(name), tok(name)
    rng = np.random.default_rng(21)
    base = workloads.config5(k.json, n_chars=60_000, n_runs=2, run_chars=3_000)
    base += "12345678901234 中文かな゛・テスト 99\n\n\r\n x " * 50
    docs = []
    at = 0
    while at < len(base) and len(docs) < 300:
        n = int(rng.integers(0, 400))
        docs.append(base[at:at + n])
        at += n
    rows = t.encode_batch(docs)
    for d, r in zip(docs, rows):
        want = k.oracle.encode_bytes(d.encode("utf-8"))
        assert np.array_equal(r.array, want), (name, d[:40])


# DeepSeek's `[ascii punct][A-Za-z]+` alternative meets an accented letter
# after a run of three or more ASCII letters (the word-level branch of the
# fast predicate): every arm of the character before the punctuation, a
# run that crosses a 64-byte word, and document starts at the punctuation
# and inside the run
DEEPSEEK_PUNCT_RUNS = [
    " !abcdé", "!!abcdé", "a!abcdé", "1!abcdé", "!abcdé", "x" * 60 + "!abcdé",
    "\t!abcdé", "x" * 61 + " !abcdé", "é!abcdé", "中!abcdé", "!abcdéfg!hij",
    " !abcdé " * 20, "\n!abcdé", "ab!cdé", "!" + "q" * 70 + "é",
]


@pytest.mark.family("deepseek_v3")
def test_deepseek_punct_letter_runs_match_hf():
    k, t = kit("deepseek_v3"), tok("deepseek_v3")
    for s in DEEPSEEK_PUNCT_RUNS:
        assert list(t.encode(s).array) == k.hf_ids(s), s
        for pre in ("", "z", " ", "x" * 40):
            u = pre + s + "é"
            assert list(t.encode(u).array) == k.hf_ids(u), u


@pytest.mark.family("deepseek_v3")
def test_deepseek_batch_rows_cut_at_the_punctuation_and_inside_the_run():
    k, t = kit("deepseek_v3"), tok("deepseek_v3")
    for s in DEEPSEEK_PUNCT_RUNS:
        p = s.index("!")
        for cut in sorted({p, p + 1, p + 2, min(len(s), p + 4), len(s) - 1}):
            docs = [s[:cut], s[cut:], s]
            rows = t.encode_batch(docs)
            for d, r in zip(docs, rows):
                assert list(r.array) == k.hf_ids(d), (s, cut, d)


@pytest.mark.family("deepseek_v3")
def test_deepseek_marks_after_long_ascii_runs():
    """A letter or mark right after an ASCII-letter run that began words or
    tiles before it: the wave searches the staged bytes and then the text
    in HBM for the run's start (a 70,000-letter run is 17 steps of 4 KiB).
    Against the oracle, alone, joined into one request at shifting
    offsets, and as batch rows cut inside the run."""
    k, t = kit("deepseek_v3"), tok("deepseek_v3")
    cases = []
    for n in (63, 64, 65, 200, TILE - 1, TILE, TILE + 1, 3 * TILE + 17, 70_000):
        for pre in ("", "!", "a!", " !", "!!", "中!", "\n!", "é!", "1!"):
            for tail in ("\u0301", "\ufe0f", "é", "中", "b"):
                cases.append(pre + "Q" * n + tail)
    for s in cases:
        want = k.oracle.encode_bytes(s.encode())
        assert np.array_equal(t.encode(s).array, want), (len(s), s[:4], s[-2:])
    joined = " ".join(cases)
    assert np.array_equal(t.encode(joined).array,
                          k.oracle.encode_bytes(joined.encode()))
    long_runs = [c for c in cases if len(c) > 3 * TILE]
    for s in long_runs[::7]:
        for cut in (3, len(s) // 2, len(s) - 2):
            docs = [s[:cut], s[cut:]]
            for d, r in zip(docs, t.encode_batch(docs)):
                assert np.array_equal(r.array, k.oracle.encode_bytes(d.encode())), \
                    (len(s), cut)


@pytest.mark.parametrize("name", ["llama_3_1_8b", "qwen3_8b"])
def test_whole_piece_block_merges_match_oracle(name):
    """Every piece over 512 bytes merged whole by a workgroup
    (TK_OPT_REPAIR_WIDEN 0: 65,536-letter Latin and CJK runs, thousands of
    guarded rounds on the Llama table), and failed cuts widened from the
    first repair pass (1): each run alone in a fresh small workspace and
    the C5 request whole, against the oracle."""
    from toktier_amd import _ffi, workloads
    k, t = kit(name), tok(name)
    data = workloads.config5(k.json, n_chars=1_200_000, n_runs=4, sample=2).encode()
    starts = k.oracle.pretokenize(data)
    big = [(a, b) for a, b in zip(starts, starts[1:]) if b - a > 512]
    assert len(big) >= 4
    try:
        for opt in (0, 1):
            t.engine.set_option(_ffi.TK_OPT_REPAIR_WIDEN, opt)
            for a, b in big:
                piece = data[a:b]
                assert np.array_equal(t.encode_bytes(piece),
                                      k.oracle.encode_bytes(piece)), (name, opt, b - a)
            assert np.array_equal(t.encode_bytes(data), k.oracle.encode_bytes(data)), \
                (name, opt)
    finally:
        t.engine.set_option(_ffi.TK_OPT_REPAIR_WIDEN, 4)


@pytest.mark.family("deepseek_v3")
def test_deepseek_c5_runs_glued_to_marks_are_linear():
    """C5's text at full size with each of its ten 65,536-letter runs made
    of ASCII letters led by punctuation and glued to a mark: the ten
    run-start searches cost a few HBM steps each, not a walk per letter
    (62 ms per run before), and the ids equal the oracle's."""
    import time
    from toktier_amd import workloads
    k, t = kit("deepseek_v3"), tok("deepseek_v3")
    base = workloads.config5(k.json, n_chars=4_194_304 - 10 * 65_538, n_runs=0,
                             sample=2)
    rng = np.random.default_rng(5)
    cuts = np.sort(rng.integers(0, len(base), 10))
    parts, a = [], 0
    for j, c in enumerate(cuts):
        run = "".join(rng.choice(list("QwertyZ"), size=65_536))
        lead = "!" if j % 2 else " ,"
        parts += [base[a:c], lead + run + ("️" if j % 3 else "́")]
        a = c
    parts.append(base[a:])
    text = "".join(parts)
    data = text.encode()
    t.encode_bytes(data)  # warm the workspace for this size
    t0 = time.perf_counter()
    got = t.encode_bytes(data)
    dt = time.perf_counter() - t0
    want = k.oracle.encode_bytes(data)
    assert np.array_equal(got, want)
    assert dt < 0.05, dt


@pytest.mark.parametrize("name", ["llama_3_1_8b", "qwen3_8b"])
def test_c5_style_long_runs_match_oracle_and_repairs_run(name):
    """C5's text (ten 65,536-char letter runs, five Latin and five CJK) at
    full size: the pieces over 512 bytes are cut and certified (from the
    first / last-token events on the monotone Qwen table, from every merge
    round on the non-monotone Llama table), some cuts fail and are
    repaired, and the ids equal the oracle's."""
    from toktier_amd import workloads
    k, t = kit(name), tok(name)
    for sample in (0, 3):
        data = workloads.config5(k.json, sample=sample).encode()
        got = t.encode_bytes(data)
        st = t.engine.last_stats()
        want = k.oracle.encode_bytes(data)
        assert not isinstance(want, int)
        assert np.array_equal(got, want), (name, sample)
        assert st["big_pieces"] >= 10, st
        assert st["repair_passes"] > 0, st
        assert t.explain()["last_execution"]["repair_passes"] == st["repair_passes"]


@pytest.mark.family("llama_3_1_8b")
def test_non_monotone_long_pieces_match_hf():
    """Pieces over 512 bytes on the non-monotone Llama table (flagged
    ranks), against the certified engine."""
    k, t = kit("llama_3_1_8b"), tok("llama_3_1_8b")
    from toktier_amd import workloads
    base = workloads.config5(k.json, n_chars=200_000, n_runs=4,
                             run_chars=3_000, sample=11)
    letters = "".join(ch for ch in base if ch.isalpha())
    rng = np.random.default_rng(13)
    for _ in range(12):
        n = int(rng.integers(513, 9000))
        a = int(rng.integers(0, len(letters) - n))
        s = " " + letters[a:a + n]
        assert list(t.encode(s).array) == k.hf_ids(s), (n, s[:60])
    for s in ("a" * 3000, "ab" * 1500, "xyz" * 700 + "中" * 400):
        assert list(t.encode(s).array) == k.hf_ids(s), s[:40]


def _digit_texts(rng):
    """Digit runs of every length class around the 64-byte word, the
    64-byte halo and the pretokenizer's tile (TILE bytes; also the former
    3072), at shifted offsets, with ASCII and non-ASCII N characters
    (Arabic-Indic, fullwidth, superscript, Roman numeral), runs broken by
    other characters, and runs at the text ends."""
    out = []
    for n in (1, 2, 3, 4, 5, 63, 64, 65, 127, 128, 129,
              TILE - 1, TILE, TILE + 1, TILE + 63, TILE + 64, TILE + 65,
              2 * TILE - 1, 2 * TILE, 2 * TILE + 1, 3071, 3072, 3073, 9300):
        for pre in ("", "x", "ab ", " " * 61, "y" * (TILE - 2)):
            out.append(pre + "7" * n + " z")
    digits = "0123456789" + "٠١٢٣" + "０１２" + "²³" + "Ⅻ"
    for _ in range(40):
        n = int(rng.integers(1, 9000))
        s = "".join(digits[int(i)] for i in rng.integers(0, len(digits), n))
        a = int(rng.integers(0, 100))
        out.append("q" * a + s + ("" if rng.random() < 0.3 else " end"))
    out.append("12 34\n56a78\t9" * 300)
    return out


@pytest.mark.parametrize("name", ["llama_3_1_8b", "deepseek_v3"])
def test_digit_runs_of_any_length_match_hf(name):
    """\\p{N}{1,3}: the group count carried across 64-byte words, the halo
    and tiles (each tile's run count looked up from the tiles before)."""
    k, t = kit(name), tok(name)
    rng = np.random.default_rng(31)
    for s in _digit_texts(rng):
        got = t.encode(s).array
        want = k.oracle.encode_bytes(s.encode())
        assert np.array_equal(got, want), (name, len(s), s[:30])
    for s in _digit_texts(rng)[::7]:
        assert list(t.encode(s).array) == k.hf_ids(s), (name, len(s), s[:30])
    # document starts inside long runs (batch rows cut anywhere)
    base = "3" * 7000 + " x " + "4" * 5000
    docs, at = [], 0
    while at < len(base):
        n = int(rng.integers(0, 4000))
        docs.append(base[at:at + n])
        at += n
    for d, r in zip(docs, t.encode_batch(docs)):
        assert np.array_equal(r.array, k.oracle.encode_bytes(d.encode())), len(d)


@pytest.mark.parametrize("name", ["llama_3_1_8b", "deepseek_v3"])
def test_million_digit_request_is_linear(name):
    """A request of one 1,000,000-digit run (and one of 4,194,304) encodes
    in linear time: each digit's group is one lookup, each tile reads its
    predecessors' run counts once."""
    import time
    k, t = kit(name), tok(name)
    for n in (1_000_000, 4_194_304):
        s = "1234567890" * (n // 10) + "5" * (n % 10)
        t.encode(s)  # warm the workspace for this size
        t0 = time.perf_counter()
        got = t.encode(s).array
        dt = time.perf_counter() - t0
        want = k.oracle.encode_bytes(s.encode())
        assert np.array_equal(got, want), (name, n)
        assert dt < 0.25, (name, n, dt)


@pytest.mark.parametrize("name", ["qwen3_8b", "llama_3_1_8b", "gpt2"])
def test_boundary_pair_table_matches(name):
    """Every merge path with the compact pair table switched off: lookups
    probe the boundary-format table (splitmix64 open addressing)."""
    from toktier_amd import workloads
    from toktier_amd._ffi import TK_OPT_COMPACT_PAIRS
    k, t = kit(name), tok(name)
    texts = [workloads.config2(k.json, n_chars=60_000, sample=4)]
    texts += _long_texts(name)[:12] + SAMPLES
    try:
        t.engine.set_option(TK_OPT_COMPACT_PAIRS, 0)
        for s in texts:
            got = t.encode(s).array
            want = k.oracle.encode_bytes(s.encode())
            assert np.array_equal(got, want), (name, s[:40])
    finally:
        t.engine.set_option(TK_OPT_COMPACT_PAIRS, 1)
    with pytest.raises(Exception):
        t.engine.set_option(TK_OPT_COMPACT_PAIRS, 2)


@pytest.mark.family("gpt2")
def test_dropped_bytes_match_hf():
    """An artifact without some single-byte tokens ('q', 'Z', TAB, the
    second byte of U+00A9): those bytes are dropped before merging, on the
    short, wide and long (serial) paths and in batches."""
    import toktier_amd
    from conftest import drop_byte_tokens
    from tokenizers import Tokenizer
    from toktier_amd import workloads
    k = kit("gpt2")
    js = drop_byte_tokens(k.json, bytes([ord("q"), ord("Z"), 9, 0xA9]))
    hf = Tokenizer.from_str(js)
    t = toktier_amd.load("gpt2", tokenizer_json=js)
    try:
        assert t.tables.byte_id[ord("q")] == -1
        base = workloads.config2(k.json, n_chars=20_000, sample=5)
        texts = ["quiz Zebra\tq", "aqa", "©q", "qqqq", "q" * 100,
                 " " + "aqZb" * 200, "Q\tq\t" * 50, base,
                 " " + "".join(ch for ch in base if ch.isalpha())[:3000]]
        for s in texts:
            assert list(t.encode(s).array) == hf.encode(
                s, add_special_tokens=False).ids, s[:40]
        rows = t.encode_batch(texts)
        for s, r in zip(texts, rows):
            assert list(r.array) == hf.encode(s, add_special_tokens=False).ids
    finally:
        t.close()


# o200k (gpt-oss): strings through every state of the split automaton
# (letters split by case, contractions, marks in letter runs and between
# punctuation, the [\r\n/]* tail, whitespace after CR/LF, digit groups)
O200K_BRANCHES = [
    "HelloWorld", "HTTPServer", "ABCdef", "iPhone", "camelCaseWord",
    "ÀÉÎ'll", "x'S", "X'RE", "it'sſ", "don'tcha", "'s", "!'s", "a'b",
    "é́", "!́!", "!!́a", " ́a", "a ́!",
    "́x", "中文ABC def", "中ABCd", "a中文Abc", "ʰABC", "ǅungla ǅUNG ǆx",
    "!\n/\n/x", "...\n\n  x", "!\r\n/!", "a!\n/́b", "\n   x",
    "  \n  \n\t", "x \r\n y", "\t\tword", "end   ", "1234567", "12 345",
    "a1234b", "½²³⁴", "SHOUT'S Mc'Donald O'NEIL", "I'M HERE'LL 'VE",
]


def _o200k_long_runs(rng):
    """Runs no word or tile resolves alone: C letters after a lower-case
    letter or not (the state differs until an upper-case letter ends the
    run), P / mark alternations after one P or two, whitespace after a
    CR/LF, upper-case runs after a C letter; at lengths around the 64-byte
    word and the pretokenizer's tile, with and without a lead-in. The long C
    runs are random ideographs (each run is one piece; a periodic piece of
    tens of KB would be merged serially)."""
    def cjk(n):
        return "".join(chr(int(c)) for c in rng.integers(0x4E00, 0x9FA5, n))
    out = []
    for n in (20, 21, 22, 1023, 1024, 1025, TILE - 1, TILE, TILE + 1, 12_000,
              40_000):
        run = cjk(n)
        for lead in ("", "a", "A", " ", "x" * 61, "y" * (TILE - 2)):
            out.append(lead + run + "ABC d")
            out.append(lead + run + "ABCd")
        if n > 3100:
            continue
        out.append("!" + "\u0301!" * n + "x")
        out.append("!!" + "\u0301!" * n + "x")
        out.append("\n" + " " * n + "x")
        out.append("\n" + " " * n + "\n x")
        out.append("\u4e2d" + "A" * n + " b")
        out.append("\u4e2d" + "A" * n + "b")
    for _ in range(20):
        alpha = ["\u4e2d", "\u6587", "a", "A", "\u0301", "!", ".", " ", "\n",
                 "/", "'", "s"]
        w = rng.dirichlet(np.ones(len(alpha)))
        n = int(rng.integers(1, 20_000))
        out.append("".join(alpha[int(i)] for i in rng.choice(len(alpha), size=n, p=w)))
    return out


O200K_ROWS = ["gpt_oss_120b", "nemotron_3_nano_4b"]


@pytest.mark.parametrize("name", O200K_ROWS)
def test_o200k_branches_match_hf(name):
    k, t = kit(name), tok(name)
    for s in O200K_BRANCHES:
        for pre in ("", "z", " ", "中", "x" * 62):
            u = pre + s
            assert list(t.encode(u).array) == k.hf_ids(u), repr(u)


@pytest.mark.parametrize("name", O200K_ROWS)
def test_o200k_long_runs_match_oracle(name):
    """The automaton's state carried across words, the waves' blocks and
    tiles (a tile whose halo word does not fix its entry state composes
    its function and looks back over the tiles before it)."""
    k, t = kit(name), tok(name)
    rng = np.random.default_rng(41)
    texts = _o200k_long_runs(rng)
    for s in texts:
        got = t.encode(s).array
        want = k.oracle.encode_bytes(s.encode())
        assert np.array_equal(got, want), (len(s), s[:20])
    for s in texts[::9]:
        assert list(t.encode(s).array) == k.hf_ids(s), (len(s), s[:20])


@pytest.mark.parametrize("name", O200K_ROWS)
def test_o200k_documents_cut_inside_runs(name):
    """Batch rows cut anywhere in long runs: a document start resets the
    state, and each row equals the oracle's encode of that document."""
    k, t = kit(name), tok(name)
    rng = np.random.default_rng(43)
    run = "".join(chr(int(c)) for c in rng.integers(0x4E00, 0x9FA5, 9000))
    base = ("a" + run + "ABC d " + "!!" + "\u0301!" * 3000 + "\n" +
            " " * 3000 + "x" + "\u4e2d" + "A" * 3000 + "b")
    docs, at = [], 0
    while at < len(base):
        n = int(rng.integers(0, 5000))
        docs.append(base[at:at + n])
        at += n
    for d, r in zip(docs, t.encode_batch(docs)):
        assert np.array_equal(r.array, k.oracle.encode_bytes(d.encode())), len(d)


@pytest.mark.family("gpt_oss_120b")
def test_o200k_long_cjk_request_is_linear():
    """900 KB of C letters (random ideographs) after a lower-case letter,
    then an upper-case run: no halo word fixes a tile's entry state, so
    every tile composes its function and looks back (a decoupled
    look-back: each tile reads the tiles before it only until one has
    published the state after it). The request is one letter match, a
    single 900 KB piece."""
    import time
    k, t = kit("gpt_oss_120b"), tok("gpt_oss_120b")
    rng = np.random.default_rng(47)
    s = ("a" + "".join(chr(int(c)) for c in rng.integers(0x4E00, 0x9FA5, 300_000))
         + "ABC d")
    t.encode(s)
    t0 = time.perf_counter()
    got = t.encode(s).array
    dt = time.perf_counter() - t0
    assert np.array_equal(got, k.oracle.encode_bytes(s.encode()))
    assert dt < 0.5, dt


@pytest.mark.family("qwen3_5_08b")
def test_qwen35_marks_continue_letter_runs():
    """The m2l class table (Qwen3.5: combining marks continue a letter run,
    [\\p{L}\\p{M}]+): syllables with vowel signs and viramas, and stacked
    accents, in runs that cross the 64-byte word and the pretokenizer's
    tile and make pieces over 512 bytes (cut and certified), after letters,
    digits, punctuation and spaces; against the oracle, and a selection
    against HF."""
    name = "qwen3_5_08b"
    k, t = kit(name), tok(name)
    texts = []
    for unit in ("\u0915\u094d\u0937", "\u0928\u094d", "\u093f",
                 "\u0e19\u0e49\u0e33", "q\u0301\u0331"):
        for n in (1, 21, 22, 64, 65, TILE // 3, TILE // 3 + 1, 200, 700):
            for lead in ("", " ", "a", "1", "!", "x" * 61):
                texts.append(lead + unit * n + " z")
    rng = np.random.default_rng(53)
    from toktier_amd import standin
    lines = standin._mark_corpus(7, 600)
    for _ in range(10):
        a = int(rng.integers(0, len(lines) - 60))
        texts.append("".join(lines[a:a + 60]))  # runs joined without spaces
    for s in texts:
        got = t.encode(s).array
        want = k.expected(s)
        assert not isinstance(want, int), (len(s), s[:20])
        assert np.array_equal(got, want), (len(s), s[:20])
    for s in texts[::7]:
        assert list(t.encode(s).array) == k.hf_ids(s), (len(s), s[:20])


@pytest.mark.family("nemotron_3_nano_4b")
def test_nemotron_single_digits_and_no_contractions():
    """The o200k row without the contraction suffix and with single digits
    (Nemotron-3): digit runs at the word and tile edges (each digit a piece
    of its own), apostrophes after letters of either case (the letter run
    ends before the apostrophe); against the oracle, and a selection
    against HF."""
    name = "nemotron_3_nano_4b"
    k, t = kit(name), tok(name)
    texts = []
    for n in (1, 2, 3, 4, 63, 64, 65, TILE - 1, TILE, TILE + 1, 5000):
        for lead in ("", "a", " ", "x" * 61, "\u4e2d"):
            texts.append(lead + "7" * n + "x")
            texts.append(lead + "12" * n + "'s")
            texts.append(lead + "\u0663" * n + " ")
    for w in ("it's", "DON'T", "they'RE", "Mc'Donald", "'s'd"):
        texts.append((w + " ") * 400)
        texts.append(w * 300)
    for s in texts:
        got = t.encode(s).array
        want = k.oracle.encode_bytes(s.encode())
        assert not isinstance(want, int)
        assert np.array_equal(got, want), (len(s), s[:20])
    for s in texts[::5]:
        assert list(t.encode(s).array) == k.hf_ids(s), (len(s), s[:20])


@pytest.mark.parametrize("name", ["qwen3_8b", "llama_3_1_8b"])
def test_hot_pair_probe_matches_oracle(name):
    """TK_OPT_HOT_PAIRS on: the merges of pieces of 65..256 bytes probe the
    LDS copy of the lowest-ranked rules first (Llama: beside the
    unsafe-rank bitmap in the same LDS); the ids equal the option off and
    the oracle's."""
    from toktier_amd import _ffi, workloads
    k, t = kit(name), tok(name)
    text = workloads.config5(k.json, n_chars=300_000, n_runs=1, run_chars=2_000)
    want = k.oracle.encode_bytes(text.encode())
    assert not isinstance(want, int)
    try:
        t.engine.set_option(_ffi.TK_OPT_HOT_PAIRS, 1)
        on = t.encode(text).array
    finally:
        t.engine.set_option(_ffi.TK_OPT_HOT_PAIRS, 0)
    off = t.encode(text).array
    assert np.array_equal(on, want)
    assert np.array_equal(off, want)


# kimi: Han runs of every subclass, Han numbers inside and at the start of
# digit groups, other Han in punctuation runs, the tail without '/'
KIMI_BRANCHES = [
    "中文ABC def", "中ABCd", "a中文Abc", "Hello世界's", "世界's", "12〇〇34",
    "〇1234〇〇〇5678", "1〇2〇3〇4", "〡〢〣12", "!⺀x", " ⺀!", "⺀⺀中〇",
    "a!\n/b", "!\r\n/!", "x'S 中'S", "ǅungla ǅUNG", "é中", "中́",
    "々々ABC", "I'M HERE'LL", "12345678901",
]


@pytest.mark.family("kimi_k3")
def test_kimi_branches_match_hf():
    k, t = kit("kimi_k3"), tok("kimi_k3")
    for s in KIMI_BRANCHES:
        for pre in ("", "z", " ", "中", "1", "x" * 62):
            u = pre + s
            assert list(t.encode(u).array) == k.hf_ids(u), repr(u)


def _kimi_runs(rng):
    out = []
    for n in (20, 63, 64, 65, 1023, 1024, 1025, TILE - 1, TILE, TILE + 1, 9000):
        for lead in ("", "a", "1", "〇", "x" * 61, "y" * (TILE - 2)):
            digits = "".join("0123456789〇〡〢"[int(i)] for i in rng.integers(0, 13, n))
            out.append(lead + digits + " z")
            out.append(lead + "7" * n + "〇" + "8" * 5)
            han = "".join(chr(int(c)) for c in rng.integers(0x4E00, 0x9FA5, n))
            out.append(lead + han + "ABC d")
        out.append("!" + "⺀!" * n + "x")
        out.append("\n" + " " * n + "x")
    for _ in range(20):
        alpha = ["中", "〇", "⺀", "a", "A", "1", "2", "!", " ", "\n", "/", "'"]
        w = rng.dirichlet(np.ones(len(alpha)))
        n = int(rng.integers(1, 20_000))
        out.append("".join(alpha[int(i)] for i in rng.choice(len(alpha), size=n, p=w)))
    return out


@pytest.mark.family("kimi_k3")
def test_kimi_long_runs_match_oracle():
    """Digit groups counted in the automaton's state across words and
    tiles (a long digit run leaves no word function constant, so tiles
    compose theirs and look back), Han runs, punctuation runs."""
    k, t = kit("kimi_k3"), tok("kimi_k3")
    rng = np.random.default_rng(53)
    texts = _kimi_runs(rng)
    for s in texts:
        got = t.encode(s).array
        want = k.oracle.encode_bytes(s.encode())
        assert np.array_equal(got, want), (len(s), s[:20])
    for s in texts[::9]:
        assert list(t.encode(s).array) == k.hf_ids(s), (len(s), s[:20])


@pytest.mark.family("kimi_k3")
def test_kimi_documents_cut_inside_runs():
    k, t = kit("kimi_k3"), tok("kimi_k3")
    rng = np.random.default_rng(59)
    base = ("1" * 7000 + "〇" * 3 + "2" * 500 + " " +
            "".join(chr(int(c)) for c in rng.integers(0x4E00, 0x9FA5, 4000)) +
            "ABC" + "!⺀" * 2000 + "\n/" + "a" * 100)
    docs, at = [], 0
    while at < len(base):
        n = int(rng.integers(0, 4000))
        docs.append(base[at:at + n])
        at += n
    for d, r in zip(docs, t.encode_batch(docs)):
        assert np.array_equal(r.array, k.oracle.encode_bytes(d.encode())), len(d)


@pytest.mark.family("kimi_k3")
def test_kimi_million_digit_request_is_linear():
    """A 1,000,000-digit request: every tile composes its function (the
    digit states cycle, so no word fixes the state) and looks back over
    published tile functions (decoupled look-back), in linear time."""
    import time
    k, t = kit("kimi_k3"), tok("kimi_k3")
    s = "1234567890" * 100_000
    t.encode(s)
    t0 = time.perf_counter()
    got = t.encode(s).array
    dt = time.perf_counter() - t0
    assert np.array_equal(got, k.oracle.encode_bytes(s.encode()))
    assert dt < 0.25, dt


@pytest.mark.parametrize("name", ["qwen3_8b", "llama_3_1_8b", "gpt_oss_120b",
                                  "kimi_k3", "deepseek_v3"])
def test_long_whitespace_and_periodic_pieces(name):
    """Pieces of one repeated character or pair (whitespace runs, rules,
    repeated syllables): a 64-byte window of them is one or two tokens, so
    the cut selection finds no cut and the piece is one segment, merged by
    a workgroup (safe ranks in batch rounds). And runs of one letter led by
    a character that joins their piece ("!" + "QQ..."): the first window
    fixes the token parity, every later one pairs from an even offset, so
    removing a failed cut makes the next one fail, and from the fourth
    repair pass on each failed cut drops a fourfold wider ring of cuts. Against the oracle, and a
    40,000-space run and a 40,000-letter run in well under 50 ms."""
    import time
    k, t = kit(name), tok(name)
    texts = []
    for n in (513, 600, 1023, 5000, 40_000):
        texts += [" " * n + "x", "\t" * n + "y", "=" * n + "\n", "ab" * (n // 2) + " c",
                  " \t" * (n // 2) + "z", "x" + " " * n, "!" + "Q" * n + "é",
                  " " + "Q" * n, "xy!" + "Q" * n + "\u0301"]
    for s in texts:
        got = t.encode(s).array
        want = k.expected(s)  # (a mark after a letter fails the NFC quick check)
        assert not isinstance(want, int), (name, len(s), s[:4])
        assert np.array_equal(got, want), (name, len(s), s[:4])
    for s in (" " * 40_000 + "x", "!" + "Q" * 40_000 + "é"):
        t.encode(s)
        t0 = time.perf_counter()
        t.encode(s)
        dt = time.perf_counter() - t0
        assert t.engine.last_stats()["repair_passes"] <= 14, name
        assert dt < 0.05, (name, len(s), dt)


@pytest.mark.family("qwen3_8b")
def test_injected_fault_isolates_rows_and_writes_no_ids():
    """The error contract through the real path: with a fault marker set,
    a call whose input holds it fails as a whole after its pipeline ran;
    a batch is resolved by halving, so exactly the poisoned rows fail and
    every other row keeps the oracle's ids; a single call raises and no
    ids are returned."""
    import toktier_amd
    from toktier_amd import _ffi, workloads
    k, t = kit("qwen3_8b"), tok("qwen3_8b")
    base = workloads.config2(k.json, n_chars=40_000, sample=6)
    docs = [base[i * 300:(i + 1) * 300] for i in range(100)]
    poison = {3, 50, 51, 99}
    for d in poison:
        docs[d] = docs[d][:100] + "⁣POISON⁣" + docs[d][100:]
    try:
        t.engine.set_fault_marker("⁣POISON⁣".encode())
        with pytest.raises(toktier_amd.BatchError) as err:
            t.encode_batch(docs)
        assert sorted(err.value.rows) == sorted(poison)
        assert all(e.status == _ffi.TK_E_INTERNAL for e in err.value.errors)
        rows = t.encode_batch(docs, errors="return")
        for d, r in enumerate(rows):
            if d in poison:
                assert isinstance(r, _ffi.EngineError)
            else:
                assert np.array_equal(r.array, k.oracle.encode_bytes(docs[d].encode())), d
        with pytest.raises(_ffi.EngineError) as e1:
            t.engine.encode(docs[3].encode())
        assert e1.value.status == _ffi.TK_E_INTERNAL
        with pytest.raises(_ffi.EngineError):
            t.seed(docs[50])
        # clean inputs are untouched by the marker
        assert np.array_equal(t.encode(docs[0]).array,
                              k.oracle.encode_bytes(docs[0].encode()))
    finally:
        t.engine.set_fault_marker(b"")
    assert np.array_equal(t.encode(docs[3]).array, k.oracle.encode_bytes(docs[3].encode()))
