"""CPU: pin the oracle (oracle/toktier_oracle.c) before trusting it.

Each check is chosen so that a plausible restatement mistake fails it:
- table digests equal the reference's pinned sha256 values;
- published constants of the hash functions (FNV-1a offset basis,
  SplitMix64's first output) and the reference's own table fixtures
  (duplicate refusal, load factor, the non-monotone guard example);
- the split rules against the certified engine's pre-tokenizer offsets by
  brute force over every short string of an alphabet that reaches every
  branch of the rules, and over seeded fuzz;
- full encodes against the committed golden vectors (HF tokenizers 0.22.2
  on the stand-in artifacts) and against HF directly on larger texts;
- planted mistakes (a wrong digit group width, the wrong rule set) must
  make the comparison fail.
"""

from __future__ import annotations

import itertools
import json
from pathlib import Path

import numpy as np
import pytest

from conftest import FAMILY_NAMES, kit
from toktier_amd import bpe_tables, classes

GOLDEN = Path(__file__).resolve().parent / "golden" / "golden_ids.json"


def _golden():
    return json.loads(GOLDEN.read_text(encoding="utf-8"))


# ------------------------------------------------------------- tables

def test_class_table_matches_reference_digest():
    tab = classes.class_table()  # raises unless the pinned digest matches
    assert classes.npy_sha256(tab) == classes.CLASS_TABLE_SHA256
    assert np.bincount(tab, minlength=4).tolist() == [971148, 141028, 1911, 25]
    assert tab[ord("a")] == 1 and tab[ord("7")] == 2 and tab[ord(" ")] == 3
    assert tab[ord("!")] == 0 and tab[0x4E2D] == 1 and tab[0xA0] == 3


def test_deepseek_class_table_matches_reference_digest():
    tab = classes.deepseek_class_table()  # raises unless the digest matches
    assert classes.npy_sha256(tab) == classes.DEEPSEEK_TABLE_SHA256
    # pretok_classes_deepseek.v1.meta.json "class_histogram"
    assert np.bincount(tab, minlength=7).tolist() == [
        957230, 141028, 2501, 1911, 11417, 23, 2]
    assert tab[ord("a")] == 1 and tab[0x301] == 2 and tab[ord("7")] == 3
    assert tab[ord("!")] == 4 and tab[ord(" ")] == 5 and tab[ord("\n")] == 6
    assert tab[0x01] == 0 and tab[0x200D] == 0 and tab[0x309B] == 4


def test_nfc_table_matches_reference_digest():
    qc = classes.nfc_qc_table()
    assert classes.npy_sha256(qc) == classes.NFC_QC_SHA256
    assert qc[ord("a")] == 0 and qc[0xE9] == 0      # precomposed e-acute
    assert qc[0x301] == 255                          # composes with a base
    assert qc[0x212B] == 255                         # singleton (Angstrom)


def test_fnv1a64_published_constants():
    assert bpe_tables.fnv1a64(b"") == 0xCBF29CE484222325
    assert bpe_tables.fnv1a64(b"a") == 0xAF63DC4C8601EC8C
    assert bpe_tables.fnv1a64(b"foobar") == 0x85944171F73967E8


def test_splitmix64_published_first_output():
    # SplitMix64 seeded with 0 yields 0xE220A8397B1DCDAF first
    assert bpe_tables.splitmix64(0) == 0xE220A8397B1DCDAF


def test_hash_table_shape_and_determinism():
    keys = list(range(1000))
    vals = [k * 7 for k in keys]
    k1, v1 = bpe_tables.build_hash(keys, vals)
    k2, v2 = bpe_tables.build_hash(keys, vals)
    assert (k1 == k2).all() and (v1 == v2).all()
    assert k1.size >= 3 * len(keys) and k1.size & (k1.size - 1) == 0
    # every key is found by the probe the kernels use
    mask = k1.size - 1
    for key, val in zip(keys, vals):
        i = bpe_tables.splitmix64(key) & mask
        while int(k1[i]) != key:
            assert int(k1[i]) != 0xFFFFFFFFFFFFFFFF
            i = (i + 1) & mask
        assert int(v1[i]) == val


def test_hash_table_refuses_duplicates():
    with pytest.raises(ValueError, match="duplicate"):
        bpe_tables.build_hash([5, 5], [1, 2])


def test_unsafe_rank_fixtures():
    # reference fixtures (tests/gpu/test_bpe_tables.py:231-267)
    assert bpe_tables.unsafe_ranks([["a", "b"], ["ab", "c"]]) == []
    assert bpe_tables.unsafe_ranks([["xy", "z"], ["x", "y"]]) == [1]
    assert bpe_tables.unsafe_ranks(["xy z", "x y"]) == [1]


def test_byte_level_alphabet():
    b2u = bpe_tables.bytes_to_unicode()
    assert len(b2u) == 256 and len(set(b2u.values())) == 256
    assert b2u[ord("A")] == "A" and b2u[0x20] == "Ġ" and b2u[0x0A] == "Ċ"
    raw = bytes([0x00, 0x41, 0xC3, 0xA9, 0xFF])
    assert bpe_tables.token_to_raw("".join(b2u[b] for b in raw)) == raw


@pytest.mark.parametrize("name", FAMILY_NAMES)
def test_exported_tables_follow_the_artifact(name):
    k = kit(name)
    spec = json.loads(k.json)["model"]
    t = k.tables
    assert t.n_merges == len(spec["merges"])
    assert t.pair_count >= 3 * t.n_merges
    assert (t.byte_id >= 0).all()
    assert bool(t.ignore_merges) == k.family.ignore_merges


# ------------------------------------------------------- split rules

BRUTE_ALPHABET = ["a", "'", "s", "S", "ſ", "1", " ", "\t", "\r", "\n",
                  "!", "é", "中", " ", "r", "e"]


def _hf_split_starts(kit_, text: str) -> list[int]:
    pre = kit_.hf.pre_tokenizer
    offs = [o for _, o in pre.pre_tokenize_str(text)]
    starts = sorted({len(text[:a].encode("utf-8")) for a, _ in offs})
    return starts + [len(text.encode("utf-8"))]


@pytest.mark.parametrize("name", FAMILY_NAMES)
def test_split_rules_brute_force(name):
    """Every string of length <= 3 over the alphabet, plus every length-4
    string over a core subset, splits like the certified engine."""
    k = kit(name)
    core = ["a", "'", "s", " ", "\r", "\n", "!", "1", "r"]
    cases = itertools.chain(
        ("".join(p) for n in range(1, 4)
         for p in itertools.product(BRUTE_ALPHABET, repeat=n)),
        ("".join(p) for p in itertools.product(core, repeat=4)),
    )
    bad = []
    for s in cases:
        if k.oracle.pretokenize(s.encode("utf-8")) != _hf_split_starts(k, s):
            bad.append(s)
    assert not bad, bad[:10]


@pytest.mark.parametrize("name", FAMILY_NAMES)
def test_split_rules_fuzz(name):
    k = kit(name)
    rng = np.random.default_rng(5)
    alpha = BRUTE_ALPHABET + ["d", "m", "t", "l", "v", "L", "E", "T", "2",
                              "\U0001f600", "-", ".", "　", " "]
    for _ in range(3000):
        s = "".join(alpha[int(i)] for i in rng.integers(0, len(alpha), int(rng.integers(1, 30))))
        assert k.oracle.pretokenize(s.encode("utf-8")) == _hf_split_starts(k, s), s


#: every class of the DeepSeek split and its special members: ASCII and
#: other letters, a combining mark, CJK-range letters and non-letters
#: (U+309B symbol, U+30FB punctuation, unassigned U+3040), ASCII and other
#: digits, ASCII punctuation and symbols, a non-ASCII symbol, O characters
#: (ZWJ, a control), space / tab / CR / LF / other whitespace, a variation
#: selector
DS_ALPHABET = ["a", "Z", "é", "\u0301", "中", "か", "\u309b", "\u30fb",
               "\u3040", "1", "½", ".", "'", "!", "$", "\U0001f600",
               "\u200d", "\x01", " ", "\t", "\n", "\r", "\u00a0",
               "\u3000", "\ufe0f", "\u0663"]


def test_deepseek_split_brute_force():
    """Every string of length <= 3 over the DeepSeek alphabet, every
    length-5 string over a core subset, and seeded fuzz split like the
    certified engine's three-stage pre-tokenizer."""
    k = kit("deepseek_v3")
    core = ["a", "é", ".", " ", "\n", "1", "\x01", "中", "\u0301", "\t"]
    cases = itertools.chain(
        ("".join(p) for n in range(1, 4)
         for p in itertools.product(DS_ALPHABET, repeat=n)),
        ("".join(p) for p in itertools.product(core, repeat=5)),
    )
    bad = [s for s in cases
           if k.oracle.pretokenize(s.encode("utf-8")) != _hf_split_starts(k, s)]
    assert not bad, [repr(s) for s in bad[:10]]
    rng = np.random.default_rng(8)
    for _ in range(5000):
        s = "".join(DS_ALPHABET[int(i)] for i in
                    rng.integers(0, len(DS_ALPHABET), int(rng.integers(1, 40))))
        assert k.oracle.pretokenize(s.encode("utf-8")) == _hf_split_starts(k, s), repr(s)


def test_planted_deepseek_mistakes_are_caught():
    """The cl100k rules on the DeepSeek classes, or digit groups of one,
    must disagree with the certified engine on the DeepSeek cases."""
    from oracle.oracle import Oracle
    k = kit("deepseek_v3")
    texts = [".abc", "12345", "中文abc", "\x01\x02a", "!!\n\n x"]
    for rs, dm in ((0, 3), (3, 1)):
        wrong = Oracle(k.tables, classes.deepseek_class_table(), None, rs, dm, False)
        assert any(wrong.pretokenize(t.encode()) != _hf_split_starts(k, t)
                   for t in texts), (rs, dm)


def test_o200k_class_table_matches_reference_digest():
    tab = classes.o200k_class_table()  # raises unless the digest matches
    assert classes.npy_sha256(tab) == classes.O200K_TABLE_SHA256
    assert tab[ord("A")] == 1 and tab[0x1C5] == 1      # Lu, Lt
    assert tab[ord("b")] == 2 and tab[0x4E2D] == 3     # Ll, Lo
    assert tab[0x2B0] == 3 and tab[ord("7")] == 4      # Lm, N
    assert tab[ord(" ")] == 5 and tab[0x301] == 6 and tab[ord("!")] == 0


#: each o200k class and the characters its rules name: U, L, Lo, Lm, Lt,
#: a mark, a digit, P, space / tab / CR / LF, the apostrophe and the
#: contraction letters in both cases (and U+017F, which folds to s), "/"
O2K_ALPHABET = ["A", "b", "中", "ʰ", "ǅ", "\u0301", "1", ".", "!", " ", "\t",
                "\n", "\r", "'", "s", "S", "ſ", "r", "e", "/"]


def test_o200k_split_brute_force():
    """The o200k restatement (oracle ruleset 4) splits like the certified
    engine with the o200k pattern: every string of length <= 3 over the
    alphabet, every length-5 string over a 10-symbol core, seeded fuzz."""
    from tokenizers import Regex, pre_tokenizers
    from oracle.oracle import Oracle
    from toktier_amd.families import O200K_PATTERN
    pre = pre_tokenizers.Split(Regex(O200K_PATTERN), behavior="isolated",
                               invert=False)
    o = Oracle(kit("gpt2").tables, classes.o200k_class_table(), None, 4, 3, False)

    def hf(text):
        offs = [b for _, b in pre.pre_tokenize_str(text)]
        st = sorted({len(text[:a].encode("utf-8")) for a, _ in offs})
        return st + [len(text.encode("utf-8"))]

    core = ["A", "b", "中", "\u0301", ".", " ", "'", "s", "\n", "/"]
    cases = itertools.chain(
        ("".join(p) for n in range(1, 4)
         for p in itertools.product(O2K_ALPHABET, repeat=n)),
        ("".join(p) for p in itertools.product(core, repeat=5)),
    )
    bad = [s for s in cases if o.pretokenize(s.encode("utf-8")) != hf(s)]
    assert not bad, [repr(s) for s in bad[:10]]
    rng = np.random.default_rng(9)
    for _ in range(5000):
        s = "".join(O2K_ALPHABET[int(i)] for i in
                    rng.integers(0, len(O2K_ALPHABET), int(rng.integers(1, 40))))
        assert o.pretokenize(s.encode("utf-8")) == hf(s), repr(s)
    # planted: the cl100k rules on these classes disagree
    wrong = Oracle(kit("gpt2").tables, classes.o200k_class_table(), None, 0, 3, False)
    assert any(wrong.pretokenize(t.encode()) != hf(t)
               for t in ("HelloWorld", "ABCdef", "x'S", "!\n/"))


#: the kimi alphabet: the o200k one with the Han letter in the Han
#: classes, plus a Han number (U+3007) and other Han (U+2E80, a radical)
KIMI_ALPHABET = ["A", "b", "中", "ʰ", "ǅ", "\u0301", "1", "〇", "⺀", ".", "!",
                 " ", "\t", "\n", "\r", "'", "s", "S", "ſ", "r", "e", "/"]


def _hf_starts(pattern):
    from tokenizers import Regex, pre_tokenizers
    pre = pre_tokenizers.Split(Regex(pattern), behavior="isolated", invert=False)

    def hf(text):
        offs = [b for _, b in pre.pre_tokenize_str(text)]
        st = sorted({len(text[:a].encode("utf-8")) for a, _ in offs})
        return st + [len(text.encode("utf-8"))]
    return hf


def test_kimi_class_table():
    tab = classes.kimi_class_table()
    assert classes.npy_sha256(tab) == classes.KIMI_TABLE_SHA256
    # the o200k classes outside Han; Han letters, numbers and the rest
    o2 = classes.o200k_class_table()
    han = tab >= 7
    assert np.array_equal(tab[~han], o2[~han])
    assert tab[0x4E2D] == 7 and tab[0x3005] == 7   # Lo, Lm
    assert tab[0x3007] == 8 and tab[0x3021] == 8   # Nl
    assert tab[0x2E80] == 9                        # So
    assert np.bincount(tab, minlength=10)[7:].tolist() == [98685, 13, 332]


def test_kimi_split_brute_force():
    """The kimi restatement (oracle ruleset 5) splits like the certified
    engine with the Kimi pattern (``[\\p{Han}]+`` first, Han-free letter
    classes, a tail without '/'): every string of length <= 3 over the
    alphabet, every length-5 string over an 11-symbol core, seeded fuzz."""
    from oracle.oracle import Oracle
    from toktier_amd.families import KIMI_PATTERN
    hf = _hf_starts(KIMI_PATTERN)
    o = Oracle(kit("gpt2").tables, classes.kimi_class_table(), None, 5, 3, False)
    core = ["A", "b", "中", "〇", "⺀", "\u0301", ".", " ", "'", "1", "\n"]
    cases = itertools.chain(
        ("".join(p) for n in range(1, 4)
         for p in itertools.product(KIMI_ALPHABET, repeat=n)),
        ("".join(p) for p in itertools.product(core, repeat=5)),
    )
    bad = [s for s in cases if o.pretokenize(s.encode("utf-8")) != hf(s)]
    assert not bad, [repr(s) for s in bad[:10]]
    rng = np.random.default_rng(19)
    for _ in range(5000):
        s = "".join(KIMI_ALPHABET[int(i)] for i in
                    rng.integers(0, len(KIMI_ALPHABET), int(rng.integers(1, 40))))
        assert o.pretokenize(s.encode("utf-8")) == hf(s), repr(s)
    # planted: the o200k split (no Han branch, the '/' tail) disagrees
    wrong = Oracle(kit("gpt2").tables, classes.o200k_class_table(), None, 4, 3, False)
    assert all(wrong.pretokenize(t.encode()) != hf(t)
               for t in ("Hello世界's", "!\n/x", "12〇〇34"))
    # and the o200k rules cannot read the Han classes at all
    bad_cfg = Oracle(kit("gpt2").tables, classes.kimi_class_table(), None, 4, 3, False)
    with pytest.raises(ValueError):
        bad_cfg.pretokenize("中".encode())


def test_o200k_without_contractions_brute_force():
    """The o200k restatement with the contraction suffix off splits like
    the o200k pattern without it (the o200k families whose
    ``kernel_families.v1.json`` rows say contractions false)."""
    from oracle.oracle import Oracle
    from toktier_amd.families import O200K_PATTERN
    pat = O200K_PATTERN.replace("(?i:'s|'t|'re|'ve|'m|'ll|'d)?", "")
    assert pat != O200K_PATTERN
    hf = _hf_starts(pat.replace(r"\p{N}{1,3}", r"\p{N}"))
    o = Oracle(kit("gpt2").tables, classes.o200k_class_table(), None, 4, 1,
               False, contractions=False)
    for s in ("".join(p) for n in range(1, 4)
              for p in itertools.product(O2K_ALPHABET, repeat=n)):
        assert o.pretokenize(s.encode("utf-8")) == hf(s), repr(s)
    assert o.pretokenize(b"it's") != _hf_starts(O200K_PATTERN)("it's")


# ------------------------------------------------------------ encodes

#: the Qwen3.5 split's cases: letters (ASCII, Latin-1, Devanagari, Thai),
#: marks of three kinds (a combining accent, a Devanagari vowel sign and
#: virama, a Thai vowel mark), the contraction letters, digits,
#: punctuation, whitespace of four kinds
Q35_ALPHABET = ["a", "'", "s", "\u0301", "\u093f", "\u094d", "\u0e31", "क",
                "ก", "é", "1", " ", "\n", "!", "\t", "中"]


def _qwen35_oracle(table):
    from oracle.oracle import Oracle
    from toktier_amd import classes, families
    return Oracle(kit("qwen3_8b").tables, table, classes.nfc_qc_table(),
                  families.RULESET_CL100K, 1, False)


def test_m2l_class_table_matches_reference_digest():
    """The marks-as-letters table (cl100k_m2l_v3) probed here equals the
    reference's pin; it differs from the base table exactly at the Mark
    code points, all moved from P to L."""
    from toktier_amd import classes, tables_gen
    m2l, base = classes.m2l_class_table(), classes.class_table()
    assert classes.npy_sha256(m2l) == classes.M2L_TABLE_SHA256
    marks = tables_gen._probe_membership(r"\p{M}")
    assert ((m2l != base) == marks).all()
    assert (base[marks] == tables_gen.P).all() and (m2l[marks] == tables_gen.L).all()


def test_qwen35_split_brute_force():
    """The cl100k restatement over the marks-as-letters table splits like
    the certified engine's Split with the Qwen3.5 pattern: every string of
    length <= 3 over the alphabet, every length-5 string over a core, 3,000
    fuzz strings; over the plain table (the planted mistake) some split
    differently."""
    from tokenizers import Regex, pre_tokenizers
    from toktier_amd import classes, families
    split = pre_tokenizers.Split(Regex(families.QWEN35_PATTERN), behavior="isolated")

    def hf(text):
        offs = [o for _, o in split.pre_tokenize_str(text)]
        return (sorted({len(text[:a].encode("utf-8")) for a, _ in offs})
                + [len(text.encode("utf-8"))])
    o = _qwen35_oracle(classes.m2l_class_table())
    plain = _qwen35_oracle(classes.class_table())
    core = ["a", "\u0301", "\u093f", "!", " ", "'", "s", "1"]
    rng = np.random.default_rng(35)
    cases = itertools.chain(
        ("".join(p) for n in range(1, 4) for p in itertools.product(Q35_ALPHABET, repeat=n)),
        ("".join(p) for p in itertools.product(core, repeat=5)),
        ("".join(Q35_ALPHABET[int(i)] for i in rng.integers(0, len(Q35_ALPHABET),
                                                            int(rng.integers(1, 40))))
         for _ in range(3000)))
    bad, planted = [], 0
    for s in cases:
        want = hf(s)
        if o.pretokenize(s.encode("utf-8")) != want:
            bad.append(s)
        planted += plain.pretokenize(s.encode("utf-8")) != want
    assert not bad, bad[:10]
    assert planted > 0


def _expected(k, text: str, ids: list[int]):
    """Oracle result for text; an NFC family's failing quick check is
    answered segment by segment with the engine-normalized text, as the
    facade does."""
    return k.expected(text)


@pytest.mark.parametrize("name", FAMILY_NAMES)
def test_oracle_matches_golden_vectors(name):
    g = _golden()["families"][name]
    k = kit(name)
    from toktier_amd import standin
    assert g["artifact_sha256"] == standin.ARTIFACT_SHA256[name]
    for case in g["cases"]:
        got = _expected(k, case["text"], case["ids"])
        assert not isinstance(got, int), (case["text"], got)
        assert got.tolist() == case["ids"], case["text"]


@pytest.mark.parametrize("name", FAMILY_NAMES)
def test_oracle_matches_hf_on_mixed_text(name):
    from toktier_amd import workloads
    k = kit(name)
    gen = {"qwen3_8b": workloads.config2, "gpt2": workloads.config2,
           "llama_3_1_8b": workloads.config4,
           "laguna_s_2_1": workloads.config4,
           "gpt_oss_120b": lambda js, n_chars: workloads.config5(
               js, n_chars=n_chars, n_runs=4, run_chars=20_000),
           "kimi_k3": lambda js, n_chars: workloads.config5(
               js, n_chars=n_chars, n_runs=4, run_chars=20_000),
           "deepseek_v3": lambda js, n_chars: workloads.config5(
               js, n_chars=n_chars, n_runs=4, run_chars=20_000),
           "nemotron_3_nano_4b": lambda js, n_chars: workloads.config5(
               js, n_chars=n_chars, n_runs=4, run_chars=20_000),
           "qwen3_5_08b": _qwen35_mixed}[name]
    text = gen(k.json, n_chars=200_000)
    got = k.expected(text)
    assert not isinstance(got, int), got
    assert got.tolist() == k.hf_ids(text)


def _qwen35_mixed(js: str, n_chars: int) -> str:
    """Mixed text and lines dense in combining marks (Devanagari, Thai,
    stacked accents), NFC-normal as the engine receives it."""
    import unicodedata
    from toktier_amd import standin, workloads
    marks = "\n".join(standin._mark_corpus(5, 400))
    return unicodedata.normalize(
        "NFC", workloads.config2(js, n_chars=n_chars) + "\n" + marks)


def test_oracle_matches_hf_on_cjk_and_long_runs():
    from toktier_amd import workloads
    k = kit("qwen3_8b")
    text = workloads.config5(k.json, n_chars=120_000, n_runs=2, run_chars=8000)
    assert k.oracle.encode_bytes(text.encode()).tolist() == k.hf_ids(text)


def test_nfc_quick_check_is_sound():
    """A passing string is left unchanged by the engine's NFC."""
    from tokenizers import normalizers
    k = kit("qwen3_8b")
    nfc = normalizers.NFC()
    qc = classes.nfc_qc_table()
    rng = np.random.default_rng(3)
    pool = np.nonzero(qc != 255)[0]
    pool = pool[(pool < 0xD800) | (pool > 0xDFFF)]
    for _ in range(400):
        s = "".join(chr(int(c)) for c in rng.choice(pool, size=12))
        if k.oracle.nfc_qc(s.encode()):
            assert nfc.normalize_str(s) == s
    assert not k.oracle.nfc_qc("é".encode())        # composes
    assert not k.oracle.nfc_qc("ậ"[::-1].encode())
    assert k.oracle.nfc_qc("café 中文 \U0001f600".encode())


# --------------------------------------------------- planted mistakes

def test_planted_wrong_digit_width_is_caught():
    from oracle.oracle import Oracle
    k = kit("qwen3_8b")
    f = k.family
    wrong = Oracle(k.tables, classes.class_table(), classes.nfc_qc_table(),
                   f.ruleset, 3, f.needs_nfc)
    text = "year 2024 and 1234567 units"
    # the stand-in Qwen vocabulary has no multi-digit tokens, so the ids
    # cannot tell the groups apart; the split offsets can
    assert wrong.pretokenize(text.encode()) != _hf_split_starts(k, text)
    assert k.oracle.pretokenize(text.encode()) == _hf_split_starts(k, text)


def test_planted_wrong_ruleset_is_caught():
    from oracle.oracle import Oracle
    k = kit("gpt2")
    f = k.family
    wrong = Oracle(k.tables, classes.class_table(), None, 0, 1, False)
    text = "we're 12 'S  \n\n x!y"
    assert wrong.encode_bytes(text.encode()).tolist() != k.hf_ids(text)
    assert k.oracle.encode_bytes(text.encode()).tolist() == k.hf_ids(text)


def test_invalid_utf8_is_refused():
    k = kit("gpt2")
    for bad in (b"\xff", b"a\xc3", b"\xc0\x80", b"\xed\xa0\x80", b"\x80abc",
                b"\xf4\x90\x80\x80"):
        assert k.oracle.encode_bytes(bad) == -1, bad
