"""Deterministic stand-in tokenizer artifacts for offline work.

The real ``tokenizer.json`` files of Qwen3-8B, Llama-3.1-8B and GPT-2 are
not reachable from this environment (no network, none on disk). Token-id
parity is a property of an *artifact* plus the encode algorithm, so the
path is exercised on stand-ins that carry each family's exact
normalizer / pre-tokenizer / model configuration and its real vocabulary
size, trained with Hugging Face ``tokenizers`` (the certified oracle,
version 0.22.2) on a corpus assembled from text files of this image plus a
seeded synthetic multilingual part. Any real artifact can be dropped in
instead (``toktier_amd.load(family, tokenizer_json=path)``).

Shapes follow the real artifacts:

- ``qwen3_8b``: NFC normalizer; ``Split(Qwen2 regex, isolated)`` +
  ``ByteLevel(use_regex=False)``; BPE with 151,387 merges over a
  151,643-entry vocabulary; ``ignore_merges`` false.
- ``llama_3_1_8b``: no normalizer; ``Split(Llama-3 regex)`` + ``ByteLevel``;
  BPE with ``ignore_merges`` true over a 128,000-entry vocabulary, merges
  re-derived tiktoken-style (every split of a token into two vocabulary
  entries, ordered by the merged token's rank), which gives more merges
  than vocabulary entries and duplicate merged ids, as the real artifact
  has (``src/toktier/kernels/bpe_tables.py`` module notes).
- ``deepseek_v3``: an empty normalizer sequence; the three
  ``Split(isolated)`` stages (digits, CJK-range runs, main pattern) +
  ``ByteLevel(use_regex=False)``; BPE over a 128,000-entry vocabulary,
  ``ignore_merges`` false.
- ``gpt2``: ``ByteLevel(use_regex=True)`` pre-tokenizer; 50,000 merges,
  50,257 entries including ``<|endoftext|>``.
- ``kimi_k3``: no normalizer; ``Split(kimi regex, isolated)`` +
  ``ByteLevel(use_regex=False)``; BPE with ``ignore_merges`` true over
  163,584 regular entries, merges every two-way split of each token in
  the order of the Kimi conversion, and 256 marker ids above them.
- ``gpt_oss_120b``: no normalizer; ``Split(o200k regex, isolated)`` +
  ``ByteLevel(use_regex=False)``; BPE with ``ignore_merges`` true over
  199,998 regular entries, merges re-derived tiktoken-style as for
  Llama-3, and the harmony markers from id 199,998.
- ``qwen3_5_08b``: as ``qwen3_8b`` with the Qwen3.5 split (marks in the
  letter run), trained with text dense in combining marks; 151,643
  entries (the stand-in's size).
- ``nemotron_3_nano_4b``: as ``gpt_oss_120b`` with the Nemotron-3 split
  (no contraction suffix, single digits); 131,072 entries (the
  stand-in's size).

The committed artifacts live in ``toktier_amd/data/artifacts`` (xz
compressed); this module regenerates them (``python -m toktier_amd.standin``),
or only rewrites their added-token lists to the real families' ones
(``python -m toktier_amd.standin --added-only``).
Training is not bit-reproducible across machines, so the committed files
and their sha256 (``ARTIFACT_SHA256``) are the identity, not this script.
"""

from __future__ import annotations

import hashlib
import json
import lzma
import os
import sys
from pathlib import Path

import numpy as np

from .families import FAMILIES, family

DATA_DIR = Path(__file__).resolve().parent / "data" / "artifacts"

__all__ = ["artifact_path", "load_artifact_json", "ARTIFACT_SHA256"]

#: sha256 of the *uncompressed* committed stand-in tokenizer.json files.
ARTIFACT_SHA256: dict[str, str] = {}
_SHA_FILE = DATA_DIR / "SHA256SUMS.json"
if _SHA_FILE.exists():
    ARTIFACT_SHA256.update(json.loads(_SHA_FILE.read_text()))


def artifact_path(name: str) -> Path:
    return DATA_DIR / f"{name}.tokenizer.json.xz"


def load_artifact_json(name: str) -> str:
    """The committed stand-in ``tokenizer.json`` text, sha256-verified."""
    family(name)
    raw = lzma.decompress(artifact_path(name).read_bytes())
    want = ARTIFACT_SHA256.get(name)
    got = hashlib.sha256(raw).hexdigest()
    if want is not None and got != want:
        raise ValueError(
            f"stand-in artifact {name} sha256 {got} != recorded {want}"
        )
    return raw.decode("utf-8")


# ---------------------------------------------------------------- corpus

_TEXT_ROOTS = ("/usr/lib/python3.10", "/usr/local/lib/python3.10/dist-packages")


def _code_corpus(limit_bytes: int) -> list[str]:
    files: list[str] = []
    for root in _TEXT_ROOTS:
        for dirpath, dirnames, filenames in os.walk(root):
            dirnames.sort()
            for f in sorted(filenames):
                if f.endswith((".py", ".rst", ".md")):
                    files.append(os.path.join(dirpath, f))
    out: list[str] = []
    total = 0
    for path in files:
        try:
            size = os.path.getsize(path)
            if size > 2_000_000:
                continue
            with open(path, encoding="utf-8", errors="ignore") as fh:
                text = fh.read()
        except OSError:
            continue
        out.append(text)
        total += len(text)
        if total >= limit_bytes:
            break
    return out


_ACCENTED = "àáâãäåæçèéêëìíîïñòóôõöøùúûüýÿÀÁÂÃÄÅÇÈÉÊËÌÍÎÏÑÒÓÔÕÖØÙÚÛÜÝß"
_SYLL_C = "bcdfghjklmnpqrstvwxz"
_SYLL_V = "aeiouy"


def _latin1_words(rng: np.random.Generator, n: int) -> list[str]:
    words = []
    for _ in range(n):
        k = int(rng.integers(1, 4))
        w = []
        for _ in range(k):
            w.append(_SYLL_C[int(rng.integers(len(_SYLL_C)))])
            if rng.random() < 0.45:
                w.append(_ACCENTED[int(rng.integers(len(_ACCENTED)))])
            else:
                w.append(_SYLL_V[int(rng.integers(len(_SYLL_V)))])
        words.append("".join(w))
    return words


def _synthetic_corpus(seed: int, cjk_chars: int, latin1_words: int,
                      emoji_lines: int) -> list[str]:
    rng = np.random.default_rng(seed)
    out: list[str] = []
    if cjk_chars:
        han = np.arange(0x4E00, 0xA000)
        rng.shuffle(han)
        # Zipf-ish character frequencies; words are 1-4 characters
        ranks = np.minimum(rng.zipf(1.15, size=cjk_chars), len(han)) - 1
        chars = [chr(int(han[r])) for r in ranks]
        words_vocab = ["".join(chars[i:i + int(rng.integers(1, 5))])
                       for i in range(0, 60000)]
        wr = np.minimum(rng.zipf(1.1, size=cjk_chars // 2),
                        len(words_vocab)) - 1
        line: list[str] = []
        n = 0
        for r in wr:
            w = words_vocab[int(r)]
            line.append(w)
            n += len(w)
            if rng.random() < 0.08:
                line.append("\uff0c" if rng.random() < 0.7 else "\u3002")
            if n > 60:
                out.append("".join(line))
                line, n = [], 0
    if latin1_words:
        lex = _latin1_words(rng, 40000)
        wr = np.minimum(rng.zipf(1.1, size=latin1_words), len(lex)) - 1
        for i in range(0, len(wr), 12):
            out.append(" ".join(lex[int(r)] for r in wr[i:i + 12]))
    if emoji_lines:
        base = list(range(0x1F600, 0x1F64F)) + list(range(0x1F300, 0x1F3FF))
        for _ in range(emoji_lines):
            k = int(rng.integers(1, 6))
            seq = []
            for _ in range(k):
                e = chr(base[int(rng.integers(len(base)))])
                if rng.random() < 0.2:
                    e += "\u200d" + chr(base[int(rng.integers(len(base)))])
                if rng.random() < 0.2:
                    e += "\ufe0f"
                seq.append(e)
            out.append(" ".join(seq))
    return out


def _mark_corpus(seed: int, n_lines: int) -> list[str]:
    """Lines dense in combining marks, whose split differs between the
    Qwen2 pattern (marks outside the letter run) and Qwen3.5's (marks in
    it): Devanagari and Thai syllables (vowel signs, viramas, tone marks
    that NFC keeps), and Latin letters with stacked accents."""
    rng = np.random.default_rng(seed)
    deva_c = [chr(c) for c in range(0x0915, 0x0939)]
    deva_v = [chr(c) for c in (0x093E, 0x093F, 0x0940, 0x0941, 0x0942, 0x0947,
                               0x0948, 0x094B, 0x094C, 0x0902, 0x094D)]
    thai_c = [chr(c) for c in range(0x0E01, 0x0E2F)]
    thai_m = [chr(c) for c in (0x0E31, 0x0E34, 0x0E35, 0x0E36, 0x0E37, 0x0E38,
                               0x0E39, 0x0E47, 0x0E48, 0x0E49, 0x0E4A, 0x0E4B)]
    accents = [chr(c) for c in (0x0301, 0x0300, 0x0308, 0x0323, 0x0331, 0x0330)]
    out = []
    for _ in range(n_lines):
        words = []
        for _ in range(int(rng.integers(4, 12))):
            kind = rng.random()
            k = int(rng.integers(1, 5))
            if kind < 0.4:
                w = "".join(deva_c[int(rng.integers(len(deva_c)))]
                            + (deva_v[int(rng.integers(len(deva_v)))] if rng.random() < 0.7 else "")
                            for _ in range(k))
            elif kind < 0.75:
                w = "".join(thai_c[int(rng.integers(len(thai_c)))]
                            + (thai_m[int(rng.integers(len(thai_m)))] if rng.random() < 0.6 else "")
                            for _ in range(k))
            else:
                w = "".join("qxzk"[int(rng.integers(4))]
                            + "".join(accents[int(rng.integers(len(accents)))]
                                      for _ in range(int(rng.integers(1, 3))))
                            for _ in range(k))
            words.append(w)
        out.append(" ".join(words))
    return out


# -------------------------------------------------------------- training

def _train(name: str) -> dict:
    from tokenizers import (Regex, Tokenizer, decoders, models,
                            normalizers, pre_tokenizers, trainers)

    fam = family(name)
    tok = Tokenizer(models.BPE())
    if fam.needs_nfc:
        tok.normalizer = normalizers.NFC()
    if name == "gpt2":
        tok.pre_tokenizer = pre_tokenizers.ByteLevel(
            add_prefix_space=False, trim_offsets=True, use_regex=True)
    elif fam.ruleset_name == "deepseek":
        from .families import DEEPSEEK_STAGES
        tok.normalizer = normalizers.Sequence([])
        tok.pre_tokenizer = pre_tokenizers.Sequence(
            [pre_tokenizers.Split(Regex(p), behavior="isolated", invert=False)
             for p in DEEPSEEK_STAGES]
            + [pre_tokenizers.ByteLevel(add_prefix_space=False,
                                        trim_offsets=False, use_regex=False)])
    elif fam.ruleset_name == "laguna":
        from .families import LAGUNA_STAGE0
        tok.pre_tokenizer = pre_tokenizers.Sequence([
            pre_tokenizers.Split(Regex(LAGUNA_STAGE0),
                                 behavior="merged_with_next", invert=False),
            pre_tokenizers.Split(Regex(fam.pattern), behavior="isolated",
                                 invert=False),
            pre_tokenizers.ByteLevel(add_prefix_space=False,
                                     trim_offsets=False, use_regex=False),
        ])
    else:
        tok.pre_tokenizer = pre_tokenizers.Sequence([
            pre_tokenizers.Split(Regex(fam.pattern), behavior="isolated",
                                 invert=False),
            pre_tokenizers.ByteLevel(add_prefix_space=False,
                                     trim_offsets=False, use_regex=False),
        ])
    tok.decoder = decoders.ByteLevel()
    n_regular = fam.vocab_size - (1 if name == "gpt2" else 0)
    trainer = trainers.BpeTrainer(
        vocab_size=n_regular,
        initial_alphabet=pre_tokenizers.ByteLevel.alphabet(),
        show_progress=False,
    )
    corpus = _code_corpus(150_000_000 if name not in (
        "gpt2", "laguna_s_2_1", "qwen3_5_08b", "nemotron_3_nano_4b")
                          else 60_000_000)
    if name == "qwen3_8b":
        corpus += _synthetic_corpus(20261201, 6_000_000, 1_500_000, 40000)
    elif name == "llama_3_1_8b":
        corpus += _synthetic_corpus(20261202, 1_500_000, 800_000, 10000)
    elif name == "deepseek_v3":
        corpus += _synthetic_corpus(20261203, 8_000_000, 1_000_000, 40000)
    elif name == "gpt_oss_120b":
        corpus += _synthetic_corpus(20261204, 6_000_000, 1_500_000, 40000)
    elif name == "kimi_k3":
        corpus += _synthetic_corpus(20261205, 10_000_000, 1_500_000, 40000)
    elif name == "qwen3_5_08b":
        corpus += _synthetic_corpus(20261206, 3_000_000, 1_000_000, 20000)
        corpus += _mark_corpus(20261206, 300_000)
    elif name == "nemotron_3_nano_4b":
        corpus += _synthetic_corpus(20261207, 3_000_000, 1_000_000, 20000)
    tok.train_from_iterator(corpus, trainer)
    spec = json.loads(tok.to_str())
    model = spec["model"]
    vocab: dict[str, int] = model["vocab"]
    if len(vocab) != n_regular:
        raise RuntimeError(
            f"{name}: corpus too small: vocab {len(vocab)} < {n_regular}")
    model["ignore_merges"] = bool(fam.ignore_merges)
    if name in ("llama_3_1_8b", "gpt_oss_120b", "nemotron_3_nano_4b"):
        model["merges"] = _tiktoken_style_merges(vocab)
    elif name == "kimi_k3":
        model["merges"] = _tiktoken_style_merges(vocab, ties="cut")
    if name == "gpt2":
        vocab["<|endoftext|>"] = 50256
    spec["added_tokens"] = added_token_entries(name)
    return spec


def family_added_tokens(name: str) -> list[tuple[str, int, bool]]:
    """(content, id, special) of the family's added tokens, in the real
    artifacts' order: Qwen3's 26 chat / tool / vision / FIM markers
    (ids 151643-151668; the tool, FIM and think markers are not special),
    Llama-3.1's 256 (128000-128255, reserved slots included) and GPT-2's
    end-of-text marker."""
    if name == "gpt2":
        return [("<|endoftext|>", 50256, True)]
    if name == "deepseek_v3":
        # (the real artifact keeps its sentence markers at ids 0-2 inside
        # the vocabulary; the stand-in numbers its markers from 128000)
        names = ["<｜begin▁of▁sentence｜>", "<｜end▁of▁sentence｜>",
                 "<｜▁pad▁｜>", "<｜fim▁hole｜>", "<｜fim▁begin｜>",
                 "<｜fim▁end｜>", "<｜User｜>", "<｜Assistant｜>", "<|EOT|>",
                 "<｜tool▁calls▁begin｜>", "<｜tool▁calls▁end｜>",
                 "<｜tool▁call▁begin｜>", "<｜tool▁call▁end｜>",
                 "<｜tool▁outputs▁begin｜>", "<｜tool▁outputs▁end｜>",
                 "<｜tool▁output▁begin｜>", "<｜tool▁output▁end｜>",
                 "<｜tool▁sep｜>", "<think>", "</think>"]
        return [(c, 128000 + k, k < 3) for k, c in enumerate(names)]
    if name == "kimi_k3":
        # 256 ids above the 163,584 ranks: the named markers in the form of
        # the Kimi-K2 configuration, reserved spellings for the rest
        named = {163584: "[BOS]", 163585: "[EOS]", 163586: "<|im_end|>",
                 163587: "<|im_user|>", 163588: "<|im_assistant|>",
                 163590: "<|start_header_id|>", 163591: "<|end_header_id|>",
                 163593: "[EOT]", 163594: "<|im_system|>",
                 163595: "<|tool_calls_section_begin|>",
                 163596: "<|tool_calls_section_end|>",
                 163597: "<|tool_call_begin|>",
                 163598: "<|tool_call_argument_begin|>",
                 163599: "<|tool_call_end|>", 163601: "<|im_middle|>",
                 163838: "[UNK]", 163839: "[PAD]"}
        return [(named.get(i, f"<|reserved_token_{i}|>"), i, True)
                for i in range(163584, 163840)]
    if name == "gpt_oss_120b":
        # the harmony markers after the 199,998 regular tokens (the named
        # ones, and the reserved slots between them)
        named = {199998: "<|startoftext|>", 199999: "<|endoftext|>",
                 200002: "<|return|>", 200003: "<|constrain|>",
                 200005: "<|channel|>", 200006: "<|start|>",
                 200007: "<|end|>", 200008: "<|message|>", 200012: "<|call|>"}
        return [(named.get(i, f"<|reserved_{i}|>"), i, True)
                for i in range(199998, 200019)]
    if name == "qwen3_5_08b":
        # (the real list is not recorded offline; Qwen3's markers, numbered
        # after the stand-in's vocabulary)
        return family_added_tokens("qwen3_8b")
    if name == "nemotron_3_nano_4b":
        # (the real list is not recorded offline; the common control and
        # chat markers, numbered after the stand-in's vocabulary)
        names = ["<unk>", "<s>", "</s>", "<|im_start|>", "<|im_end|>",
                 "<think>", "</think>", "<SPECIAL_10>"]
        return [(c, 131072 + k, k < 3 or k == 7) for k, c in enumerate(names)]
    if name == "laguna_s_2_1":
        # (the real list is not recorded offline; chat and FIM markers in
        # the common form)
        names = ["<|endoftext|>", "<|im_start|>", "<|im_end|>",
                 "<|fim_prefix|>", "<|fim_middle|>", "<|fim_suffix|>",
                 "<think>", "</think>"]
        return [(c, 100000 + k, k < 3) for k, c in enumerate(names)]
    if name == "qwen3_8b":
        special = ["endoftext", "im_start", "im_end", "object_ref_start",
                   "object_ref_end", "box_start", "box_end", "quad_start",
                   "quad_end", "vision_start", "vision_end", "vision_pad",
                   "image_pad", "video_pad"]
        out = [(f"<|{t}|>", 151643 + k, True) for k, t in enumerate(special)]
        rest = ["<tool_call>", "</tool_call>", "<|fim_prefix|>",
                "<|fim_middle|>", "<|fim_suffix|>", "<|fim_pad|>",
                "<|repo_name|>", "<|file_sep|>", "<tool_response>",
                "</tool_response>", "<think>", "</think>"]
        out += [(t, 151657 + k, False) for k, t in enumerate(rest)]
        return out
    named = {128000: "begin_of_text", 128001: "end_of_text",
             128002: "reserved_special_token_0",
             128003: "reserved_special_token_1",
             128004: "finetune_right_pad_id",
             128005: "reserved_special_token_2",
             128006: "start_header_id", 128007: "end_header_id",
             128008: "eom_id", 128009: "eot_id", 128010: "python_tag"}
    return [(f"<|{named.get(i, f'reserved_special_token_{i - 128008}')}|>",
             i, True) for i in range(128000, 128256)]


def added_token_entries(name: str) -> list[dict]:
    return [{"id": i, "content": c, "single_word": False, "lstrip": False,
             "rstrip": False, "normalized": False, "special": sp}
            for c, i, sp in family_added_tokens(name)]


def patch_added_tokens(names: list[str]) -> None:
    """Rewrite the committed artifacts' added_tokens list (the merges and
    vocabulary stay as they are) and their recorded sha256."""
    sums = dict(ARTIFACT_SHA256)
    for name in names:
        spec = json.loads(load_artifact_json(name))
        spec["added_tokens"] = added_token_entries(name)
        raw = json.dumps(spec, ensure_ascii=False,
                         separators=(",", ":")).encode("utf-8")
        sums[name] = hashlib.sha256(raw).hexdigest()
        artifact_path(name).write_bytes(lzma.compress(raw, preset=9))
        ARTIFACT_SHA256[name] = sums[name]
        print(name, len(raw), sums[name], flush=True)
    _SHA_FILE.write_text(json.dumps(sums, indent=1, sort_keys=True) + "\n")


def _tiktoken_style_merges(vocab: dict[str, int],
                           ties: str = "ids") -> list[list[str]]:
    """Every split ``t = a + b`` with ``a, b`` in the vocabulary, ordered by
    the merged token's id, then by ``(id(a), id(b))`` (``ties="ids"``) or
    by the split position (``ties="cut"``, as the Kimi conversion orders
    them: ``src/toktier/artifacts/conversion.py`` ``convert_kimi_tiktoken``)."""
    merges: list[tuple[int, int, int, str, str]] = []
    for token, rank in vocab.items():
        if len(token) < 2:
            continue
        for k in range(1, len(token)):
            a, b = token[:k], token[k:]
            ia, ib = vocab.get(a), vocab.get(b)
            if ia is not None and ib is not None:
                merges.append((rank, ia, ib, a, b) if ties == "ids"
                              else (rank, k, 0, a, b))
    merges.sort()
    return [[a, b] for _, _, _, a, b in merges]


def main(argv: list[str]) -> None:
    if argv[:1] == ["--added-only"]:
        patch_added_tokens(argv[1:] or sorted(FAMILIES))
        return
    names = argv or sorted(FAMILIES)
    DATA_DIR.mkdir(parents=True, exist_ok=True)
    sums = dict(ARTIFACT_SHA256)
    for name in names:
        spec = _train(name)
        raw = json.dumps(spec, ensure_ascii=False,
                         separators=(",", ":")).encode("utf-8")
        sums[name] = hashlib.sha256(raw).hexdigest()
        artifact_path(name).write_bytes(lzma.compress(raw, preset=9))
        print(name, len(raw), sums[name], flush=True)
    _SHA_FILE.write_text(json.dumps(sums, indent=1, sort_keys=True) + "\n")


if __name__ == "__main__":
    main(sys.argv[1:])
