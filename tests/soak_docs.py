"""Documents and expected ids for the seeded parity soak
(``test_gpu_soak.py``), computed in worker processes that never touch the
GPU: each batch's documents are drawn from a seed, and the oracle's ids
for each are computed beside them.

A batch (about ``BATCH_CHARS`` characters) mixes:

- fuzz documents: random strings over the family's branch atoms (the
  characters and strings that reach each branch of its split, its
  added-token literals, digits, marks, CR/LF, long-s, title case);
- workload slices: cuts of one generated request per batch, C2 / C4 / C5
  or chat text (the sample seed changes per batch), anywhere in the text;
- long runs: letter runs (random and periodic), digit runs, whitespace,
  punctuation-and-mark alternations and C-letter runs of 500 - 70,000
  characters (pieces over 512 bytes: cut, segmented, certified);
- short documents: the empty string and the golden samples.

The expected ids follow the facade's contract: the oracle's encode, and for
a text that fails the NFC quick check, its literals split out and each
segment normalized (HF's NFC) and encoded alone.
"""

from __future__ import annotations

import sys
from functools import lru_cache
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
for p in (str(ROOT), str(HERE), str(HERE / "golden")):
    if p not in sys.path:
        sys.path.insert(0, p)

SOAK_SEED = 20261202
BATCH_CHARS = 2_000_000
MAX_DOCS = 1000  # a batch ends at BATCH_CHARS characters, well before this

_ATOMS_COMMON = [
    "a", "A", "'", "s", "S", "\u017f", "1", "2", "9", " ", "  ", "\t", "\r",
    "\n", "\r\n", "!", ".", "-", "/", "\u00e9", "e\u0301", "\u0301",
    "\u4e2d", "\u6587", "\u00a0", "\u3000", "\U0001f600", "\u200d", "\u01c5",
    "'s", "'S", "'ll", "'RE", "'ve", "'M", "'d", "\u0663", "\u00bd",
    "\u0915\u094d\u0937", "\u093f", "\u0e19\u0e49", "\u3007", "\u2e80",
    "\u30fb", "\u309b", "\u3099", "\x01", "Hello", "WORLD", "x", "0x1F",
]


@lru_cache(maxsize=None)
def _oracle(name: str):
    """The family's oracle and added-token literals (as the test kit builds
    them)."""
    import toktier_amd
    from toktier_amd import bpe_tables, classes, families, standin
    from oracle.oracle import Oracle
    fam = families.family(name)
    js = standin.load_artifact_json(name)
    tables = bpe_tables.load_tables(js)
    orc = Oracle(tables, classes.table_named(families.class_table_name(fam)),
                 classes.nfc_qc_table(), fam.ruleset, fam.digits_max,
                 fam.needs_nfc, contractions=fam.contractions)
    added = toktier_amd.added_tokens(js)
    orc.set_added([t.content.encode() for t in added], [t.id for t in added])
    return fam, js, orc, added


def expected(name: str, text: str) -> np.ndarray | int:
    """The oracle's ids for `text` under the facade's NFC contract."""
    fam, _, orc, added = _oracle(name)
    got = orc.encode_bytes(text.encode("utf-8"))
    if not (isinstance(got, int) and fam.needs_nfc):
        return got
    from tokenizers import normalizers
    from toktier_amd import LiteralSplitter
    nfc = normalizers.NFC()
    parts = []
    for seg, lit in LiteralSplitter(added).split(text):
        if lit is not None:
            parts.append(np.asarray([lit], dtype=np.uint32))
            continue
        ids = orc.encode_bytes(nfc.normalize_str(seg).encode("utf-8"),
                               normalized=True, literals=False)
        if isinstance(ids, int):
            return ids
        parts.append(ids)
    return np.concatenate(parts) if parts else np.zeros(0, np.uint32)


@lru_cache(maxsize=None)
def _atoms(name: str) -> list[str]:
    import make_golden as g
    _, _, _, added = _oracle(name)
    atoms = list(_ATOMS_COMMON) + [t.content for t in added][:40]
    extra = {"deepseek_v3": g.DEEPSEEK_CASES, "gpt_oss_120b": g.O200K_CASES,
             "nemotron_3_nano_4b": g.O200K_CASES + g.NEMOTRON_CASES,
             "kimi_k3": g.KIMI_CASES, "qwen3_5_08b": g.QWEN35_CASES}
    atoms += [s for s in extra.get(name, []) if len(s) < 40]
    return atoms


def _workload(name: str, js: str, index: int, n_chars: int) -> str:
    from toktier_amd import workloads
    kind = index % 4
    if kind == 0:
        return workloads.config2(js, n_chars=n_chars, sample=index)
    if kind == 1:
        return workloads.config4(js, n_chars=n_chars, sample=index)
    if kind == 2:
        return workloads.config5(js, n_chars=n_chars, n_runs=2,
                                 run_chars=20_000, sample=index)
    return workloads.chat(js, name, n_chars=n_chars, sample=index)


def _long_run(rng: np.random.Generator, letters: str) -> str:
    n = int(rng.integers(500, 70_000))
    kind = int(rng.integers(0, 7))
    if kind == 0:
        a = int(rng.integers(0, max(1, len(letters) - n)))
        run = letters[a:a + n]
    elif kind == 1:
        unit = letters[:int(rng.integers(1, 6))] or "ab"
        run = unit * (n // len(unit))
    elif kind == 2:
        run = "".join(str(int(d)) for d in rng.integers(0, 10, n))
    elif kind == 3:
        run = "".join(" \t\n"[int(i)] for i in rng.integers(0, 3, n))
    elif kind == 4:
        run = "!" + "\u0301!" * (n // 2)
    elif kind == 5:
        run = "".join(chr(int(c)) for c in rng.integers(0x4E00, 0x9FA5, n // 3))
    else:
        run = "\u0915\u094d\u0937\u093f" * (n // 4)
    lead = ["", " ", "a", "A", "1", "!", "中", "x" * 61][int(rng.integers(0, 8))]
    tail = ["", " z", "ABC d", "'s", "\n", "12"][int(rng.integers(0, 6))]
    return lead + run + tail


def batch(name: str, index: int) -> tuple[list[str], list[np.ndarray | int]]:
    """Batch `index` of family `name`: its documents and expected ids."""
    import make_golden as g
    from toktier_amd.families import FAMILIES
    fam_no = sorted(FAMILIES).index(name)
    rng = np.random.default_rng([SOAK_SEED, fam_no, index])
    _, js, _, _ = _oracle(name)
    atoms = _atoms(name)
    text = _workload(name, js, index, BATCH_CHARS // 2)
    letters = "".join(ch for ch in text[:200_000] if ch.isalpha())
    docs: list[str] = []
    total = 0
    while total < BATCH_CHARS and len(docs) < MAX_DOCS:
        r = rng.random()
        if r < 0.35:
            k = int(rng.integers(1, 600))
            d = "".join(atoms[int(i)] for i in rng.integers(0, len(atoms), k))
        elif r < 0.75:
            n = int(min(len(text), rng.lognormal(7.5, 1.5)))
            a = int(rng.integers(0, max(1, len(text) - n)))
            d = text[a:a + n]
        elif r < 0.85:
            d = _long_run(rng, letters)
        else:
            pool = g.SAMPLES
            d = pool[int(rng.integers(0, len(pool)))]
        docs.append(d)
        total += len(d)
    return docs, [expected(name, d) for d in docs]


_CURRENT: list[str] = []


def work(job: tuple[str, int]):
    """Pool entry: (family, batch index) -> (index, documents, expected
    ids). A worker keeps one family's oracle at a time."""
    name, index = job
    if _CURRENT and _CURRENT[0] != name:
        _oracle.cache_clear()
        _atoms.cache_clear()
    _CURRENT[:] = [name]
    docs, want = batch(name, index)
    return index, docs, want
