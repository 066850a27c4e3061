"""Seeded synthetic inputs for the five benchmark configurations.

Each config ``k`` draws from ``numpy.random.default_rng(20261201 + k)``.
Words are concatenations of 1-3 vocabulary tokens drawn Zipf(s=1.1) over
token rank (token id order), decoded to text, as the configurations
specify. The vocabulary is the family artifact the engine is opened with
(the committed stand-ins unless a real ``tokenizer.json`` is supplied).

- C1 ``qwen3_8b``, 65,536 chars, ASCII: single spaces between words, 8%
  punctuation tokens, 4% digit runs of 1-6, a newline every ~80 chars.
- C2 ``qwen3_8b``, 4,194,304 chars: 85% ASCII words (with the C1
  punctuation / digit mix), 10% Latin-1 accented words (NFC composed,
  U+00C0-U+00FF, two UTF-8 bytes each), 5% whitespace runs of 2-16 drawn
  from space, tab and CR LF.
- C3 ``gpt2``, 256 documents of U[1,024, 32,768] chars of C1-style ASCII.
- C4 ``llama_3_1_8b``, 4,194,304 chars of code: snake_case / camelCase
  identifiers from token concatenation, 20% operators and brackets,
  indentation runs of 4-32 spaces after newlines, 10% hex / decimal
  literals of 1-20 chars, string literals with escapes.
- C5 ``qwen3_8b``, 4,194,304 chars: 50% CJK ideographs (U+4E00-U+9FFF,
  sentences of CJK vocabulary tokens without spaces), 10% emoji including
  ZWJ sequences and VS16, 40% Latin token-concat text; plus ten unbroken
  65,536-char letter runs (five Latin, five CJK) with no whitespace.
"""

from __future__ import annotations

import json
from functools import lru_cache

import numpy as np

from .bpe_tables import token_to_raw

SEED_BASE = 20261201
CHARS_4M = 4_194_304

_ACC = {
    "a": "àáâãäå", "e": "èéêë", "i": "ìíîï", "o": "òóôõöø", "u": "ùúûü",
    "y": "ýÿ", "n": "ñ", "c": "ç", "A": "ÀÁÂÃÄÅ", "E": "ÈÉÊË", "O": "ÒÓÔÕÖØ",
}
_PUNCT = list(".,;:!?-()\"'[]/") + ["...", "--", "?!"]
_OPS = ["=", "==", "!=", "+", "-", "*", "/", "%", "<", ">", "<=", ">=", "+=",
        "-=", "->", "=>", "&&", "||", "(", ")", "[", "]", "{", "}", ",", ";",
        ":", ".", "::", "&", "|", "^", "~", "<<", ">>", "@", "#"]


@lru_cache(maxsize=8)
def _vocab_lists(tokenizer_json: str) -> dict[str, list[str]]:
    vocab = json.loads(tokenizer_json)["model"]["vocab"]
    words, cjk = [], []
    for tok, _tid in sorted(vocab.items(), key=lambda kv: kv[1]):
        try:
            s = token_to_raw(tok).decode("utf-8")
        except (KeyError, UnicodeDecodeError):
            continue
        w = s.strip(" ")
        if w and w.isascii() and w.isalpha():
            words.append(w)
        elif w and all(0x4E00 <= ord(ch) <= 0x9FFF for ch in w):
            cjk.append(w)
    return {"words": words, "cjk": cjk}


def _zipf_idx(rng: np.random.Generator, n: int, size: int) -> np.ndarray:
    out = np.empty(0, dtype=np.int64)
    while out.size < size:
        k = rng.zipf(1.1, size=2 * (size - out.size) + 16)
        out = np.concatenate([out, k[k <= n] - 1])
    return out[:size]


class _Words:
    def __init__(self, rng: np.random.Generator, toks: list[str]):
        self.rng, self.toks = rng, toks
        self._buf = np.empty(0, dtype=np.int64)

    def _next_idx(self) -> int:
        if self._buf.size == 0:
            self._buf = _zipf_idx(self.rng, len(self.toks), 65536)
        i = int(self._buf[0])
        self._buf = self._buf[1:]
        return i

    def word(self, joiner: str = "") -> str:
        k = int(self.rng.integers(1, 4))
        return joiner.join(self.toks[self._next_idx()] for _ in range(k))


def _accent(rng: np.random.Generator, w: str) -> str:
    chars = list(w)
    idx = [i for i, ch in enumerate(chars) if ch in _ACC]
    if not idx:
        return w + "é"
    for i in idx[: max(1, len(idx) // 2)]:
        opts = _ACC[chars[i]]
        chars[i] = opts[int(rng.integers(len(opts)))]
    return "".join(chars)


def _ascii_stream(rng: np.random.Generator, words: _Words, n_chars: int,
                  latin1: float = 0.0, ws_runs: float = 0.0) -> str:
    parts: list[str] = []
    total = 0
    col = 0
    while total < n_chars:
        r = rng.random()
        if r < ws_runs:
            k = int(rng.integers(2, 17))
            pool = [" ", "\t", "\r\n"]
            s = "".join(pool[int(x)] for x in rng.integers(0, 3, size=k))
            parts.append(s)
            total += len(s)
            col = 0 if "\n" in s else col + len(s)
            continue
        r2 = rng.random()
        if r2 < 0.08:
            s = _PUNCT[int(rng.integers(len(_PUNCT)))]
        elif r2 < 0.12:
            s = "".join(str(int(d)) for d in rng.integers(0, 10, size=int(rng.integers(1, 7))))
        else:
            s = words.word()
            if latin1 and rng.random() < latin1:
                s = _accent(rng, s)
        if col + len(s) + 1 > 80:
            sep = "\n"
            col = 0
        else:
            sep = " "
        piece = s + sep
        parts.append(piece)
        total += len(piece)
        col += len(piece)
    return "".join(parts)[:n_chars]


def config1(tokenizer_json: str, n_chars: int = 65_536) -> str:
    rng = np.random.default_rng(SEED_BASE + 1)
    return _ascii_stream(rng, _Words(rng, _vocab_lists(tokenizer_json)["words"]), n_chars)


def config2(tokenizer_json: str, n_chars: int = CHARS_4M, sample: int = 0) -> str:
    rng = np.random.default_rng(SEED_BASE + 2 + 1000 * sample)
    w = _Words(rng, _vocab_lists(tokenizer_json)["words"])
    # 85/10/5 of elements: ws-run share 5%, Latin-1 10/95 of the rest
    return _ascii_stream(rng, w, n_chars, latin1=0.10 / 0.95, ws_runs=0.05)


def config3(tokenizer_json: str, n_docs: int = 256, sample: int = 0) -> list[str]:
    rng = np.random.default_rng(SEED_BASE + 3 + 1000 * sample)
    w = _Words(rng, _vocab_lists(tokenizer_json)["words"])
    lens = rng.integers(1024, 32769, size=n_docs)
    return [_ascii_stream(rng, w, int(n)) for n in lens]


def config4(tokenizer_json: str, n_chars: int = CHARS_4M, sample: int = 0) -> str:
    rng = np.random.default_rng(SEED_BASE + 4 + 1000 * sample)
    w = _Words(rng, _vocab_lists(tokenizer_json)["words"])
    parts: list[str] = []
    total = 0
    line = 0
    while total < n_chars:
        r = rng.random()
        if r < 0.20:
            s = _OPS[int(rng.integers(len(_OPS)))]
        elif r < 0.30:
            k = int(rng.integers(1, 21))
            if rng.random() < 0.5 and k > 2:
                s = "0x" + "".join("0123456789abcdefABCDEF"[int(x)]
                                   for x in rng.integers(0, 22, size=k - 2))
            else:
                s = "".join(str(int(d)) for d in rng.integers(0, 10, size=k))
        elif r < 0.36:
            body = w.word(" ")
            esc = ["\\n", "\\t", '\\"', "\\\\"][int(rng.integers(4))]
            s = '"' + body + esc + w.word() + '"'
        else:
            toks = [w.word().lower() for _ in range(int(rng.integers(1, 4)))]
            if rng.random() < 0.5:
                s = "_".join(toks)
            else:
                s = toks[0] + "".join(t[:1].upper() + t[1:] for t in toks[1:])
        line += len(s)
        if line > 70:
            s = s + "\n" + " " * int(4 * rng.integers(1, 9))
            line = 0
        else:
            s = s + (" " if rng.random() < 0.7 else "")
        parts.append(s)
        total += len(s)
    return "".join(parts)[:n_chars]


_EMOJI = list(range(0x1F600, 0x1F64F)) + list(range(0x1F300, 0x1F3FF)) + \
    list(range(0x1F680, 0x1F6C5))


def config5(tokenizer_json: str, n_chars: int = CHARS_4M, sample: int = 0,
            n_runs: int = 10, run_chars: int = 65_536) -> str:
    rng = np.random.default_rng(SEED_BASE + 5 + 1000 * sample)
    lists = _vocab_lists(tokenizer_json)
    latin = _Words(rng, lists["words"])
    cjk = _Words(rng, lists["cjk"]) if lists["cjk"] else None

    def cjk_run(n: int) -> str:
        out, k = [], 0
        while k < n:
            if cjk is not None and rng.random() < 0.9:
                s = cjk.word()
            else:
                s = chr(int(rng.integers(0x4E00, 0xA000)))
            out.append(s)
            k += len(s)
        return "".join(out)[:n]

    def latin_run(n: int) -> str:
        out, k = [], 0
        while k < n:
            s = latin.word()
            out.append(s)
            k += len(s)
        return "".join(out)[:n]

    body = n_chars - n_runs * run_chars
    n_cjk_runs = n_runs // 2
    # character budgets of the body after the runs' own share: 50% CJK,
    # 10% emoji, 40% Latin over the whole request
    want = {"cjk": 0.5 * n_chars - n_cjk_runs * run_chars,
            "emoji": 0.1 * n_chars,
            "latin": 0.4 * n_chars - (n_runs - n_cjk_runs) * run_chars}
    have = {"cjk": 0.0, "emoji": 0.0, "latin": 0.0}
    parts: list[str] = []
    total = 0
    while total < body:
        # the category furthest below its budget, with a little noise
        kind = max(want, key=lambda c: (want[c] - have[c]) / max(want[c], 1.0)
                   + 0.05 * rng.random())
        if kind == "cjk":
            s = cjk_run(int(rng.integers(4, 60))) + ("\uff0c" if rng.random() < 0.6 else "\u3002")
        elif kind == "emoji":
            k = int(rng.integers(1, 4))
            em = []
            for _ in range(k):
                e = chr(_EMOJI[int(rng.integers(len(_EMOJI)))])
                if rng.random() < 0.25:
                    e += "\u200d" + chr(_EMOJI[int(rng.integers(len(_EMOJI)))])
                if rng.random() < 0.2:
                    e += "\ufe0f"
                em.append(e)
            s = "".join(em) + " "
        else:
            s = latin.word() + (" " if rng.random() < 0.9 else "\n")
        have[kind] += len(s)
        parts.append(s)
        total += len(s)
    text = "".join(parts)[:body]
    # embed the pathological runs at seeded positions, each between spaces
    cuts = sorted(int(x) for x in rng.integers(0, len(text), size=n_runs))
    out, prev = [], 0
    for i, c in enumerate(cuts):
        out.append(text[prev:c])
        run = latin_run(run_chars) if i % 2 == 0 else cjk_run(run_chars)
        out.append(run)
        prev = c
    out.append(text[prev:])
    return "".join(out)[:n_chars]


def chat(tokenizer_json: str, family: str, n_chars: int = CHARS_4M,
         sample: int = 0) -> str:
    """C2-style text laid out as chat turns in the family's template, so
    the request carries added-token literals: Qwen3 ``<|im_start|>role``
    ... ``<|im_end|>`` (assistant turns with a ``<think>`` block), Llama-3
    header / ``<|eot_id|>`` turns after ``<|begin_of_text|>``, DeepSeek
    ``<｜User｜>`` / ``<｜Assistant｜>`` turns after the sentence marker
    (assistant turns closed by ``<｜end▁of▁sentence｜>``), gpt-oss harmony
    ``<|start|>role<|message|>`` ... ``<|end|>`` turns (assistant turns on
    the final channel, some after an analysis one), Kimi
    ``<|im_role|>role<|im_middle|>`` ... ``<|im_end|>`` turns, GPT-2
    documents joined by ``<|endoftext|>``; Qwen3.5 as Qwen3, Nemotron-3 the
    Qwen3 turns after ``<s>``. Turns hold U[200, 3000] chars."""
    rng = np.random.default_rng(SEED_BASE + 6 + 1000 * sample)
    body = config2(tokenizer_json, n_chars=n_chars, sample=sample)
    roles = ["system", "user", "assistant"]
    out: list[str] = (["<|begin_of_text|>"] if family == "llama_3_1_8b" else
                      ["<｜begin▁of▁sentence｜>"] if family == "deepseek_v3" else
                      ["<s>"] if family == "nemotron_3_nano_4b" else [])
    total, at, turn = sum(map(len, out)), 0, 0
    while total < n_chars and at < len(body):
        n = int(rng.integers(200, 3001))
        content = body[at:at + n]
        at += n
        role = roles[0] if turn == 0 else roles[1 + (turn - 1) % 2]
        if family in ("qwen3_8b", "qwen3_5_08b", "nemotron_3_nano_4b"):
            if role == "assistant" and rng.random() < 0.5:
                content = "<think>\n" + content[: n // 3] + "\n</think>\n\n" + content[n // 3:]
            piece = f"<|im_start|>{role}\n{content}<|im_end|>\n"
        elif family == "llama_3_1_8b":
            piece = f"<|start_header_id|>{role}<|end_header_id|>\n\n{content}<|eot_id|>"
        elif family == "deepseek_v3":
            piece = (f"<｜Assistant｜>{content}<｜end▁of▁sentence｜>"
                     if role == "assistant" else
                     f"<｜User｜>{content}" if role == "user" else content)
        elif family == "kimi_k3":
            piece = (f"<|im_{role}|>{role}<|im_middle|>{content}<|im_end|>"
                     if role != "assistant" else
                     f"<|im_assistant|>assistant<|im_middle|>{content}<|im_end|>")
        elif family == "gpt_oss_120b":
            if role == "assistant":
                cut = n // 3 if rng.random() < 0.5 else 0
                piece = ((f"<|start|>assistant<|channel|>analysis<|message|>"
                          f"{content[:cut]}<|end|>" if cut else "") +
                         f"<|start|>assistant<|channel|>final<|message|>"
                         f"{content[cut:]}<|return|>")
            else:
                piece = f"<|start|>{role}<|message|>{content}<|end|>"
        else:
            piece = content + "<|endoftext|>"
        out.append(piece)
        total += len(piece)
        turn += 1
    return "".join(out)[:n_chars]


CONFIGS = {
    1: ("qwen3_8b", config1),
    2: ("qwen3_8b", config2),
    3: ("gpt2", config3),
    4: ("llama_3_1_8b", config4),
    5: ("qwen3_8b", config5),
}
