"""Probe the certified engine (HF ``tokenizers`` 0.22.2) for the two
per-codepoint tables the device path reads.

1. **Character classes** over the whole codepoint space (0x110000 entries,
   ``uint8``): ``P=0`` (none of the below), ``L=1`` (``\\p{L}``), ``N=2``
   (``\\p{N}``), ``S=3`` (``\\s``), as the split regexes' engine sees them.
   Same class encoding as the reference table ``pretok_classes_cl100k.v3.npy``
   (``src/toktier/kernels/pretok_kernel.cu:63``,
   ``src/toktier/kernels/tables/kernel_families.v1.json:4-13``). The method
   (probe every codepoint through the engine's own regex) follows
   ``tools/generate_class_tables.py:375-444``, ``:556-572``; the code is this
   project's own.
2. **NFC quick check**: ``0`` = starter that is safe, ``1..K`` = rank of the
   canonical combining class of a non-starter that composes with nothing,
   ``255`` = unsafe (changes under NFC on its own, or may compose with a
   preceding character). Predicate: a string passes iff it holds no 255 and
   no adjacent pair with ``v[i-1] > v[i] != 0``; a passing string is left
   unchanged by the engine's NFC normalizer
   (``src/toktier/kernels/tables/nfc_quick_check.v1.meta.json``). Probed with
   ``normalizers.NFC``/``NFD`` over the whole codepoint space.

Surrogates (U+D800-DFFF) cannot occur in valid UTF-8 and are given class P
and QC 255.

Run ``python -m toktier_amd.tables_gen`` to regenerate
``toktier_amd/data/tables/{classes,nfc_qc}.npz``.
"""

from __future__ import annotations

import sys
import unicodedata
from pathlib import Path

import numpy as np

TABLE_DIR = Path(__file__).resolve().parent / "data" / "tables"
PLANE = 0x110000
P, L, N, S = 0, 1, 2, 3


def _valid(cp: int) -> bool:
    return not (0xD800 <= cp <= 0xDFFF)


def _probe_membership(pattern: str) -> np.ndarray:
    """Boolean per codepoint: does the single character match ``pattern``."""
    from tokenizers import Regex, pre_tokenizers

    # "removed" drops every match; the surviving char offsets are the misses
    split = pre_tokenizers.Split(Regex(pattern), behavior="removed")
    out = np.zeros(PLANE, dtype=bool)
    step = 1 << 14
    for lo in range(0, PLANE, step):
        cps = [c for c in range(lo, min(PLANE, lo + step)) if _valid(c)]
        text = "".join(chr(c) for c in cps)
        keep = np.zeros(len(cps), dtype=bool)
        for _piece, (a, b) in split.pre_tokenize_str(text):
            keep[a:b] = True
        for c, k in zip(cps, keep):
            if not k:
                out[c] = True
    return out


def build_classes() -> np.ndarray:
    ws = _probe_membership(r"\s")
    let = _probe_membership(r"\p{L}")
    num = _probe_membership(r"\p{N}")
    if (ws & let).any() or (ws & num).any() or (let & num).any():
        raise RuntimeError("class probes overlap")
    tab = np.full(PLANE, P, dtype=np.uint8)
    tab[num] = N
    tab[let] = L
    tab[ws] = S
    return tab


def build_cl100k_m2l(base: np.ndarray) -> np.ndarray:
    """The four-class table with the Mark code points moved into L: the
    Qwen3.5 split runs letters as ``[\p{L}\p{M}]+`` and leaves marks out
    of its punctuation run, and both differences are this one change to the
    table (the reference's generator ``class_tables:cl100k_m2l``,
    ``tools/generate_class_tables.py:574-597``)."""
    tab = base.copy()
    tab[_probe_membership(r"\p{M}")] = L
    return tab


#: DeepSeek seven-class encoding (the reference's
#: pretok_classes_deepseek.v1.meta.json enum)
DS_O, DS_L, DS_M, DS_N, DS_PS, DS_WS, DS_CRLF = range(7)


def build_deepseek_classes() -> np.ndarray:
    """Seven classes for the DeepSeek V3 split patterns: O (none of the
    below), L (``\p{L}``), M (``\p{M}``), N (``\p{N}``), PS
    (``[\p{P}\p{S}]``), WS (``\s`` other than CR / LF), CRLF. Surrogates
    (never in valid UTF-8) take PS, as in the reference table (whose sha256
    this reproduces, ``kernel_families.v1.json`` ``deepseek_v1``)."""
    ws = _probe_membership(r"\s")
    let = _probe_membership(r"\p{L}")
    mark = _probe_membership(r"\p{M}")
    num = _probe_membership(r"\p{N}")
    ps = _probe_membership(r"[\p{P}\p{S}]")
    crlf = _probe_membership(r"[\r\n]")
    sets = (ws, let, mark, num, ps)
    for i in range(len(sets)):
        for j in range(i + 1, len(sets)):
            if (sets[i] & sets[j]).any():
                raise RuntimeError("class probes overlap")
    tab = np.full(PLANE, DS_O, dtype=np.uint8)
    tab[let] = DS_L
    tab[mark] = DS_M
    tab[num] = DS_N
    tab[ps] = DS_PS
    tab[ws] = DS_WS
    tab[crlf] = DS_CRLF
    tab[0xD800:0xE000] = DS_PS
    return tab


#: o200k seven-class encoding (kimi meta "class_enum" order, first seven)
OK_P, OK_U, OK_L, OK_C, OK_N, OK_S, OK_M = range(7)


def build_o200k_classes() -> np.ndarray:
    """Seven classes for the o200k split: U (``\p{Lu}``, ``\p{Lt}``), L
    (``\p{Ll}``), C (``\p{Lm}``, ``\p{Lo}``: both letter sets of the
    pattern), N, S (``\s``), M and P (the rest). Reproduces the reference
    table's sha256 (``kernel_families.v1.json`` ``o200k_v4``)."""
    tab = np.full(PLANE, OK_P, dtype=np.uint8)
    for val, pats in ((OK_U, (r"\p{Lu}", r"\p{Lt}")), (OK_L, (r"\p{Ll}",)),
                      (OK_C, (r"\p{Lm}", r"\p{Lo}")), (OK_N, (r"\p{N}",)),
                      (OK_S, (r"\s",)), (OK_M, (r"\p{M}",))):
        for pat in pats:
            tab[_probe_membership(pat)] = val
    return tab


#: kimi's three Han subclasses on top of the o200k seven
OK_HL, OK_HN, OK_HP = 7, 8, 9


def build_kimi_classes(o200k: np.ndarray) -> np.ndarray:
    """Ten classes for the kimi split: the o200k seven with every
    ``\p{Han}`` codepoint moved to HL (Han and ``\p{Lm}`` or ``\p{Lo}``:
    only the Han branch takes it), HN (Han and ``\p{N}``: the digit
    branch takes it too) or HP (Han and neither: the punctuation branch
    takes it), since the pattern's letter classes exclude Han.
    Reproduces the reference table's sha256 (``kernel_families.v1.json``
    ``kimi_v1``; subclass sizes ``pretok_classes_kimi.v1.meta.json``)."""
    han = _probe_membership(r"\p{Han}")
    lm_lo = _probe_membership(r"\p{Lm}") | _probe_membership(r"\p{Lo}")
    let = _probe_membership(r"\p{L}")
    num = _probe_membership(r"\p{N}")
    tab = o200k.copy()
    tab[han & lm_lo] = OK_HL
    tab[han & num] = OK_HN
    tab[han & ~let & ~num] = OK_HP
    if ((tab >= OK_HL) != han).any():
        raise RuntimeError("the Han subclasses do not cover \\p{Han}")
    return tab


def _batch_norm(norm, items: list[str]) -> list[str]:
    """Normalize many short strings at once, separated by U+0020 (a starter
    with no composition or decomposition role)."""
    out: list[str] = []
    step = 4096
    for i in range(0, len(items), step):
        chunk = items[i:i + step]
        res = norm.normalize_str(" ".join(chunk)).split(" ")
        if len(res) != len(chunk):
            raise RuntimeError("separator interacted with the probe")
        out.extend(res)
    return out


#: Marks that Unicode 10-15 gave a non-zero canonical combining class but
#: that the engine's normalization data (older) still treats as plain
#: starters. They are flagged unsafe so that an engine built on newer
#: Unicode data could never see a string this table passes change under
#: NFC. (Unicode Character Database, DerivedCombiningClass.txt, 15.0.)
NEWER_NONSTARTERS = (
    (0x07FD, 0x07FD), (0x0898, 0x089F), (0x08CA, 0x08D3), (0x09FE, 0x09FE),
    (0x0C3C, 0x0C3C), (0x0D3B, 0x0D3C), (0x0EBA, 0x0EBA), (0x1715, 0x1715),
    (0x1ABF, 0x1ACE), (0x1DF6, 0x1DFA), (0xA82C, 0xA82C), (0x10D24, 0x10D27),
    (0x10EAB, 0x10EAC), (0x10EFD, 0x10EFF), (0x10F46, 0x10F50),
    (0x10F82, 0x10F85), (0x11070, 0x11070), (0x1133B, 0x1133B),
    (0x1145E, 0x1145E), (0x11839, 0x1183A), (0x1193D, 0x1193E),
    (0x11943, 0x11943), (0x119E0, 0x119E0), (0x11A34, 0x11A34),
    (0x11A47, 0x11A47), (0x11A99, 0x11A99), (0x11D42, 0x11D42),
    (0x11D44, 0x11D45), (0x11D97, 0x11D97), (0x11F41, 0x11F42),
    (0x16FF0, 0x16FF1), (0x1E08F, 0x1E08F), (0x1E130, 0x1E136),
    (0x1E2AE, 0x1E2AE), (0x1E2EC, 0x1E2EF), (0x1E4EC, 0x1E4EF),
)


def build_nfc_qc() -> np.ndarray:
    from tokenizers import normalizers

    nfc, nfd = normalizers.NFC(), normalizers.NFD()
    # U+0020 is the probe separator; it is a plain starter (v = 0)
    cps = [c for c in range(PLANE) if _valid(c) and c != 0x20]
    chars = [chr(c) for c in cps]
    v = np.zeros(PLANE, dtype=np.uint8)
    v[0xD800:0xE000] = 255

    # (1) changes on its own under NFC (QC = No)
    alone = _batch_norm(nfc, chars)
    for c, ch, r in zip(cps, chars, alone):
        if r != ch:
            v[c] = 255

    # (2) may compose with a preceding character (QC = Maybe): the last
    # character of the canonical decomposition of every primary composite
    decomp = _batch_norm(nfd, chars)
    second: set[int] = set()
    for c, ch, d in zip(cps, chars, decomp):
        if len(d) >= 2 and v[c] != 255:
            # ch is NFC-stable and decomposes: it is a primary composite
            second.add(ord(d[-1]))
    for c in second:
        v[c] = 255

    # (3) canonical combining class order of the remaining non-starters,
    # measured through NFD reordering against one representative mark per
    # class value
    reps: dict[int, int] = {}
    for c in cps:
        k = unicodedata.combining(chr(c))
        if k and k not in reps:
            if nfd.normalize_str(chr(c)) == chr(c):
                reps[k] = c

    def swaps(a: str, b: str) -> bool:
        return a != b and nfd.normalize_str(a + b) == b + a

    # keep only the class values the engine itself knows: a representative
    # must reorder against U+0301 (class 230) in the direction its class says
    acute = "\u0301"
    order = [k for k in sorted(reps)
             if k == 230
             or (k < 230 and swaps(acute, chr(reps[k])))
             or (k > 230 and swaps(chr(reps[k]), acute))]
    rep_chars = [chr(reps[k]) for k in order]

    # sanity: representatives must be strictly ordered by the engine too
    for i in range(len(order) - 1):
        if not swaps(rep_chars[i + 1], rep_chars[i]):
            raise RuntimeError("representative marks not ordered")
    top, bottom = rep_chars[-1], rep_chars[0]
    for c, ch, d in zip(cps, chars, decomp):
        if v[c] == 255 or d != ch:
            continue
        nonstarter = swaps(top, ch) or swaps(ch, bottom) or ch in rep_chars
        if not nonstarter:
            continue
        # rank = number of representatives whose class is <= class(ch)
        lo, hi = 0, len(rep_chars)
        while lo < hi:           # first rep that swaps before ch
            mid = (lo + hi) // 2
            if swaps(rep_chars[mid], ch):
                hi = mid
            else:
                lo = mid + 1
        pos = lo                  # reps[0:pos] have class <= class(ch)
        if pos == 0 or swaps(ch, rep_chars[pos - 1]):
            v[c] = 255            # a class value with no representative
        else:
            v[c] = pos
    for lo, hi in NEWER_NONSTARTERS:
        v[lo:hi + 1] = 255
    return v


def main() -> None:
    TABLE_DIR.mkdir(parents=True, exist_ok=True)
    cls = build_classes()
    np.savez_compressed(TABLE_DIR / "classes.npz", cl100k=cls)
    print("classes", np.bincount(cls, minlength=4), flush=True)
    m2l = build_cl100k_m2l(cls)
    np.savez_compressed(TABLE_DIR / "classes_m2l.npz", cl100k_m2l=m2l)
    print("m2l classes", np.bincount(m2l, minlength=4), flush=True)
    ds = build_deepseek_classes()
    np.savez_compressed(TABLE_DIR / "classes_deepseek.npz", deepseek=ds)
    print("deepseek classes", np.bincount(ds, minlength=7), flush=True)
    ok = build_o200k_classes()
    np.savez_compressed(TABLE_DIR / "classes_o200k.npz", o200k=ok)
    print("o200k classes", np.bincount(ok, minlength=7), flush=True)
    km = build_kimi_classes(ok)
    np.savez_compressed(TABLE_DIR / "classes_kimi.npz", kimi=km)
    print("kimi classes", np.bincount(km, minlength=10), flush=True)
    qc = build_nfc_qc()
    np.savez_compressed(TABLE_DIR / "nfc_qc.npz", nfc_qc=qc)
    print("nfc_qc 0:", int((qc == 0).sum()), "1..K:",
          int(((qc > 0) & (qc < 255)).sum()), "255:", int((qc == 255).sum()),
          "K:", int(qc[qc < 255].max()), flush=True)


if __name__ == "__main__":
    main()
    sys.exit(0)
