"""Added-token literals on the CPU: the oracle's split and the facade's host
splitter against the certified engine (HF tokenizers 0.22.2).

The differential shape is the reference's (tests/backend/
test_added_frontend.py:1-11): the whole artifact encoding a text is the
expectation; the subject is the split with each segment encoded by the same
artifact without its added tokens. The probe tables follow that file's
flag-free probes (special vs ordinary, leftmost-longest overlap,
:130-176); single_word / lstrip / rstrip tables are refused by the engine
(tests/test_gpu_added.py checks the refusal)."""

from __future__ import annotations

import json

import numpy as np
import pytest

from conftest import FAMILY_NAMES, kit

BIG_ID = 300_000

PROBES = [
    (["<sp>", "<or>"], ["a<sp>b", "a<or>b", "<sp><or>", "text <sp> tail",
                        "x<sp", "<or", "<sp>>", "<<or>"]),
    (["<t", "<t>", "<tt>", "ab", "abc", "bc"],
     ["<t>", "<tt>", "<t", "x<t>y", "x<tt>y", "<t<t>", "<t><tt>", "ab", "abc",
      "abcd", "aabc", "xabcbc", "ababc", "abcbc", "zab", "abz", "aabbcc",
      "<t<t<t>>", "ab" * 20 + "c", "<tt" * 9 + ">"]),
]


def with_added(json_text: str, contents: list[str]) -> str:
    spec = json.loads(json_text)
    spec["added_tokens"] = [
        {"id": BIG_ID + k, "content": c, "single_word": False,
         "lstrip": False, "rstrip": False, "normalized": False,
         "special": k % 2 == 0}
        for k, c in enumerate(contents)]
    return json.dumps(spec, ensure_ascii=False)


def bare(json_text: str) -> str:
    spec = json.loads(json_text)
    spec["added_tokens"] = []
    return json.dumps(spec, ensure_ascii=False)


def hf_assigned(json_text: str, contents: list[str]) -> list[int]:
    from tokenizers import Tokenizer
    t = Tokenizer.from_str(json_text)
    return [t.token_to_id(c) for c in contents]


def oracle_with(k, contents: list[str], ids: list[int]):
    from oracle.oracle import Oracle
    from toktier_amd import classes
    f = k.family
    o = Oracle(k.tables, classes.class_table(), classes.nfc_qc_table(),
               f.ruleset, f.digits_max, f.needs_nfc)
    o.set_added([c.encode() for c in contents], ids)
    return o


def spliced(splitter, hf_bare, text: str) -> list[int]:
    out: list[int] = []
    for seg, lit in splitter.split(text):
        out += [lit] if lit is not None else \
            hf_bare.encode(seg, add_special_tokens=False).ids
    return out


@pytest.mark.parametrize("probe", range(len(PROBES)))
def test_probe_tables_split_like_hf(probe):
    from tokenizers import Tokenizer
    import toktier_amd
    contents, docs = PROBES[probe]
    k = kit("gpt2")
    full = Tokenizer.from_str(with_added(k.json, contents))
    hf_bare = Tokenizer.from_str(bare(k.json))
    ids = [t.id for t in toktier_amd.added_tokens(with_added(k.json, contents))]
    assert ids == hf_assigned(with_added(k.json, contents), contents)
    o = oracle_with(k, contents, ids)
    sp = toktier_amd.LiteralSplitter(
        toktier_amd.added_tokens(with_added(k.json, contents)))
    for d in docs:
        want = full.encode(d, add_special_tokens=False).ids
        assert o.encode_bytes(d.encode()).tolist() == want, d
        assert spliced(sp, hf_bare, d) == want, d


@pytest.mark.parametrize("name", FAMILY_NAMES)
def test_family_literals_fuzz(name):
    """Random texts over literal fragments, whole literals and ordinary
    characters: oracle and host splitter against HF."""
    from tokenizers import Tokenizer
    import toktier_amd
    k = kit(name)
    lits = [t.content for t in k.added]
    rng = np.random.default_rng(17)
    frags = ["<", "|", ">", "<|", "|>", "im", "_end", "end", "of", "text",
             " ", "\n", "a", "é", "中", "'s", "1", "́", "\t"]
    hf_bare = Tokenizer.from_str(bare(k.json))
    sp = toktier_amd.LiteralSplitter(k.added)
    for _ in range(300):
        parts = []
        for _ in range(int(rng.integers(1, 14))):
            if rng.random() < 0.3:
                parts.append(lits[int(rng.integers(0, len(lits)))])
            else:
                parts.append(frags[int(rng.integers(0, len(frags)))])
        s = "".join(parts)
        want = k.hf_ids(s)
        got = k.expected(s)
        assert not isinstance(got, int), (s, got)
        assert got.tolist() == want, s
        if not k.family.needs_nfc:
            assert spliced(sp, hf_bare, s) == want, s


@pytest.mark.parametrize("name", FAMILY_NAMES)
def test_chat_text_oracle_matches_hf(name):
    from toktier_amd import workloads
    k = kit(name)
    text = workloads.chat(k.json, name, n_chars=60_000)
    assert k.oracle.encode_bytes(text.encode()).tolist() == k.hf_ids(text)


def test_literals_are_split_before_normalization():
    """A combining mark after a literal composes with the literal's last
    byte under a whole-text NFC ('>' + U+0338 is U+226F); HF extracts the
    literal first, so the mark stays a segment of its own."""
    k = kit("qwen3_8b")
    text = "<|im_end|≯x"
    want = k.hf_ids(text)
    assert want[0] == 151645
    assert k.expected(text).tolist() == want
    # the whole-text route would lose the literal
    from tokenizers import normalizers
    assert "<|im_end|>" not in normalizers.NFC().normalize_str(text)


def test_splitter_without_literals_is_one_segment():
    import toktier_amd
    sp = toktier_amd.LiteralSplitter([])
    assert sp.split("") == []
    assert sp.split("abc") == [("abc", None)]


@pytest.mark.parametrize("name", FAMILY_NAMES)
def test_family_ids_are_the_ones_hf_assigns(name):
    k = kit(name)
    assert [t.id for t in k.added] == hf_assigned(
        k.json, [t.content for t in k.added])
    from toktier_amd import standin
    assert [t.id for t in k.added] == [i for _, i, _ in
                                       standin.family_added_tokens(name)]


def test_id_assignment_rule_matches_hf():
    """The id field is ignored: vocabulary entries keep their id, new
    contents count up from the vocabulary size (or past the largest id
    given), repeats and empty contents are skipped."""
    import toktier_amd
    k = kit("gpt2")
    cases = [["<a>", "<b>", "ab", "<c>"], ["ab", "<a>"], ["<a>", "<a>", "<b>"],
             ["<|endoftext|>", "<x>"], ["hello", "<x>", "world", "<y>"],
             ["", "<z>"]]
    for contents in cases:
        js = with_added(k.json, contents)
        got = {t.content: t.id for t in toktier_amd.added_tokens(js)}
        want = dict(zip(contents, hf_assigned(js, contents)))
        want.pop("", None)
        assert got == want, contents


def test_added_tokens_parse_flags():
    import toktier_amd
    from toktier_amd import _ffi
    spec = {"added_tokens": [
        {"id": 5, "content": "<m>", "single_word": True, "lstrip": True,
         "rstrip": False, "normalized": True, "special": True}]}
    (t,) = toktier_amd.added_tokens(json.dumps(spec))
    assert t.flags == (_ffi.TK_ADDED_SPECIAL | _ffi.TK_ADDED_SINGLE_WORD
                       | _ffi.TK_ADDED_LSTRIP | _ffi.TK_ADDED_NORMALIZED)
