r"""CPU model of the o200k and kimi split automaton (the device's
``o2k_char`` with the state carried across lanes, words and tiles in
``k_pretok<4, ...>`` / ``k_pretok<5, ...>``).

The o200k split (oracle ruleset 4) is a left-to-right automaton over eight
states (the whitespace match shares the state that ends a match: a
whitespace character after another one reads it as the former; the
contraction letters share one state: the character before a letter tells
whether another follows): each character maps the state after the character before it to the
state after itself and says, per previous state, whether it starts a
piece; digits take the group rule instead. The model here is that
automaton character by character. Checked: it splits every string of
length <= 4 over the o200k alphabet of the oracle's brute-force test, every
length-5 string over a ten-symbol core, seeded fuzz with document starts
(each document split on its own), and composing the transitions in blocks
(as the wave scan and the tile look-back do) gives the same states. Planted
mistakes in the transitions (a C letter resetting LBL, the tail dropping
'/', a two-letter contraction taking one letter, the whitespace rule
ignoring the CR/LF before it) each split some string differently.

kimi adds three states, eleven in all (in a Han run; one or two digits into a
\p{N}{1,3} group, since a Han number continues a group but opens a Han
run at a group's start) and the same checks run against oracle ruleset 5
over an alphabet with a Han letter, a Han number and other Han.
"""

from __future__ import annotations

import itertools

import numpy as np
import pytest

from conftest import kit
from test_oracle import KIMI_ALPHABET, O2K_ALPHABET

P, U, L, C, N, S, M, HL, HN, HP = range(10)
W = (U, L, C, M)
PUN, TAIL, LPRE, LU, LBL, LBN, CONTR, FRESH, HAN, D1, D2 = range(11)


def _nstate(kimi):
    return 11 if kimi else 8


def _classes(kimi=False):
    from toktier_amd import classes
    return classes.kimi_class_table() if kimi else classes.o200k_class_table()


def _fold(c: int) -> int:
    if 65 <= c <= 90:
        return c + 32
    return ord("s") if c == 0x17F else c


def _crlf(c: int) -> bool:
    return c in (10, 13)


def transitions(cps, ds, plant=None, kimi=False):
    """Per character (f, g): f[s] the state after it, g[s] its start bit
    (None: the digit group rule, o200k), for the previous state s. FRESH
    is also the whitespace match's state: a whitespace character after
    another one reads it as such (the character before it tells)."""
    cls = _classes(kimi)
    nstate = _nstate(kimi)
    n = len(cps)
    cl = [int(cls[c]) for c in cps]

    def nxt(j):
        q = j + 1
        return None if q >= n or ds[q] else q

    out = []
    for j in range(n):
        k, c = cl[j], cps[j]
        n1 = nxt(j)
        n2 = nxt(n1) if n1 is not None else None
        k1 = cl[n1] if n1 is not None else None
        has_prev = j > 0 and not ds[j]
        prev_s = has_prev and cl[j - 1] == S
        prev_ap = has_prev and cps[j - 1] == ord("'")
        han = kimi and k >= HL
        pm = k in (P, M) or (kimi and k == HP)
        if han:
            ns = HAN
        elif k == N:
            ns = D1 if kimi else FRESH
        elif k in (U, L):
            ns = LU if k == U else LBL
        elif k in (C, M):
            ns = LBN
        elif k == P or (k == S and not _crlf(c)):
            ns = (LPRE if k1 in W else
                  PUN if k == P or (c == 32 and (k1 == P or (kimi and k1 == HP)))
                  else FRESH)
        else:
            ns = FRESH
        ap = False  # an apostrophe that a contraction takes
        if c == ord("'") and n1 is not None:
            a = _fold(cps[n1])
            if chr(a) in "stmd":
                ap = True
            elif n2 is not None and (chr(a), chr(_fold(cps[n2]))) in (
                    ("r", "e"), ("v", "e"), ("l", "l")):
                ap = True
        f1 = False  # every character from j to the letter run's end is U
        if k == U:
            q = nxt(j)
            while q is not None and cl[q] == U:
                q = nxt(q)
            f1 = q is None or cl[q] not in W
        f3 = True  # no CR/LF from j to the whitespace run's end
        q = j
        while q is not None and cl[q] == S:
            if _crlf(cps[q]):
                f3 = False
                break
            q = nxt(q)
        prev_crlf = (has_prev and _crlf(cps[j - 1]) and plant != "ws_no_crlf")
        f, g = [ns] * nstate, [1] * nstate
        for s in range(nstate):
            if ds[j]:
                continue
            st, nx = 1, ns
            if s == PUN:
                if pm:
                    st, nx = 0, PUN
                elif _crlf(c):
                    st, nx = 0, TAIL
            elif s == TAIL:
                if _crlf(c) or (c == ord("/") and not kimi
                                and plant != "tail_no_slash"):
                    st, nx = 0, TAIL
            elif s == LPRE:
                if k in W:
                    st = 0
            elif s in (LU, LBL, LBN):
                if k == U:
                    st, nx = (1 if s == LBL else f1 if s == LBN else 0), LU
                elif k == L:
                    st, nx = 0, LBL
                elif k in (C, M):
                    keep = s if plant != "c_resets" else LBN
                    st, nx = 0, (LBN if s == LU else keep)
                elif ap:
                    st, nx = 0, CONTR
            elif s == CONTR:
                two = prev_ap and chr(_fold(c)) in "rvl"
                if plant == "two_takes_one":
                    two = False
                st, nx = 0, (CONTR if two else FRESH)
            elif s == FRESH and k == S and prev_s:
                # inside a whitespace match
                if _crlf(c):
                    st, nx = 0, FRESH
                else:
                    st = f3 if prev_crlf else (n1 is not None and k1 != S)
                    nx = ns if st else FRESH
            elif s == HAN and han:
                st, nx = 0, HAN
            elif s in (D1, D2) and k in (N, HN):
                st, nx = 0, (D2 if s == D1 else FRESH)
            f[s], g[s] = nx, (None if k == N and not kimi else int(st))
        out.append((tuple(f), tuple(g)))
    return out, cl


def split(text: str, docs=(), plant=None, block: int = 0, kimi=False):
    """Piece starts (char indices) of `text` with documents starting at
    the indices `docs`; block > 0: the states come from compositions of
    `block` transitions at a time (the state after each block from its
    composed function, the states inside it from prefix compositions)."""
    cps = [ord(ch) for ch in text]
    n = len(cps)
    ds = [i == 0 or i in docs for i in range(n)]
    fg, cl = transitions(cps, ds, plant, kimi)
    nstate = _nstate(kimi)
    states = [0] * n
    if block:
        s = FRESH
        for a in range(0, n, block):
            F = tuple(range(nstate))
            for j in range(a, min(n, a + block)):
                F = tuple(fg[j][0][F[x]] for x in range(nstate))
                states[j] = F[s]
            s = F[s]
    else:
        s = FRESH
        for j in range(n):
            s = fg[j][0][s]
            states[j] = s
    out, run = [], 0
    for j in range(n):
        prev = states[j - 1] if j else FRESH
        st = fg[j][1][prev]
        if cl[j] == N and not kimi:
            run = 0 if ds[j] or cl[j - 1] != N else run
            st = int(ds[j] or run % 3 == 0)
            run += 1
        if st:
            out.append(j)
    return out


def _oracle(kimi=False):
    from oracle.oracle import Oracle
    return Oracle(kit("gpt2").tables, _classes(kimi), None, 5 if kimi else 4,
                  3, False)


def oracle_split(o, text: str, docs=()) -> list[int]:
    cuts = [0, *sorted(d for d in docs if 0 < d < len(text)), len(text)]
    out = []
    for a, b in zip(cuts, cuts[1:]):
        seg = text[a:b]
        idx = {len(seg[:i].encode()): i for i in range(len(seg) + 1)}
        out += [a + idx[x] for x in o.pretokenize(seg.encode())[:-1]]
    return out


CORE = ["A", "b", "中", "́", ".", " ", "'", "s", "\n", "/"]


@pytest.mark.slow
def test_automaton_splits_like_the_oracle_exhaustively():
    o = _oracle()
    cases = itertools.chain(
        ("".join(p) for n in range(1, 5)
         for p in itertools.product(O2K_ALPHABET, repeat=n)),
        ("".join(p) for p in itertools.product(CORE, repeat=5)))
    bad = [t for t in cases if split(t) != oracle_split(o, t)]
    assert not bad, [repr(t) for t in bad[:10]]


def test_automaton_splits_like_the_oracle():
    o = _oracle()
    for t in ("".join(p) for n in range(1, 4)
              for p in itertools.product(O2K_ALPHABET, repeat=n)):
        assert split(t) == oracle_split(o, t), repr(t)
    rng = np.random.default_rng(11)
    for _ in range(3000):
        n = int(rng.integers(1, 60))
        t = "".join(O2K_ALPHABET[int(i)] for i in rng.integers(0, len(O2K_ALPHABET), n))
        docs = sorted(set(int(x) for x in rng.integers(1, n + 1, size=int(rng.integers(0, 4)))))
        want = oracle_split(o, t, docs)
        assert split(t, docs) == want, (repr(t), docs)
        assert split(t, docs, block=int(rng.integers(1, 9))) == want, (repr(t), docs)


def test_automaton_on_long_runs():
    """Runs no fixed context resolves: C letters after an L letter or not,
    P / M alternations after one P or two, whitespace runs after a CR/LF."""
    o = _oracle()
    texts = ["a" + "中" * 200 + "ABC d", "中" * 200 + "ABC d", "中" * 200 + "ABCd",
             "!" + "́!" * 100 + "x", "!!" + "́!" * 100 + "x",
             "\n" + " " * 150 + "x", "\n" + " " * 150 + "\n x",
             "x" + "'" * 99 + "s", "It'" + "s" * 50 + "'LL", "a!\n/\n/" * 30]
    for t in texts:
        assert split(t) == oracle_split(o, t), repr(t)
        assert split(t, block=64) == oracle_split(o, t), repr(t)


PLANTS = ["c_resets", "tail_no_slash", "two_takes_one", "ws_no_crlf"]


@pytest.mark.parametrize("plant", PLANTS)
def test_planted_transition_mistakes_are_caught(plant):
    o = _oracle()
    hits = [t for t in ("".join(p) for n in range(1, 5)
                        for p in itertools.product(CORE + ["r", "e", "\t"], repeat=n))
            if split(t, plant=plant) != oracle_split(o, t)]
    found = {"c_resets": "b中Ad", "tail_no_slash": "./\n/",
             "ws_no_crlf": "\n \t\t"}.get(plant)
    assert hits, plant
    if found:
        assert split(found, plant=plant) != oracle_split(o, found), plant


KIMI_CORE = ["A", "b", "中", "〇", "⺀", "\u0301", ".", " ", "'", "1", "\n"]


def test_kimi_automaton_splits_like_the_oracle():
    o = _oracle(kimi=True)
    for t in itertools.chain(
            ("".join(p) for n in range(1, 4)
             for p in itertools.product(KIMI_ALPHABET, repeat=n)),
            ("".join(p) for p in itertools.product(KIMI_CORE, repeat=4))):
        assert split(t, kimi=True) == oracle_split(o, t), repr(t)
    rng = np.random.default_rng(13)
    for _ in range(3000):
        n = int(rng.integers(1, 60))
        t = "".join(KIMI_ALPHABET[int(i)] for i in rng.integers(0, len(KIMI_ALPHABET), n))
        docs = sorted(set(int(x) for x in rng.integers(1, n + 1, size=int(rng.integers(0, 4)))))
        want = oracle_split(o, t, docs)
        assert split(t, docs, kimi=True) == want, (repr(t), docs)
        assert split(t, docs, block=int(rng.integers(1, 9)), kimi=True) == want, (repr(t), docs)


@pytest.mark.slow
def test_kimi_automaton_splits_like_the_oracle_exhaustively():
    o = _oracle(kimi=True)
    cases = itertools.chain(
        ("".join(p) for p in itertools.product(KIMI_ALPHABET, repeat=4)),
        ("".join(p) for p in itertools.product(KIMI_CORE, repeat=5)))
    bad = [t for t in cases if split(t, kimi=True) != oracle_split(o, t)]
    assert not bad, [repr(t) for t in bad[:10]]


def test_kimi_automaton_on_long_runs():
    """Digit runs with Han numbers inside and at group starts, Han runs of
    every subclass, the tail without '/'."""
    o = _oracle(kimi=True)
    texts = ["1" * 40 + "〇" * 7 + "2" * 11, "〇1234〇〇〇5678", "12〇〇34" * 20,
             "中" * 100 + "〇⺀中1234", "!⺀!" * 30 + "x", " ⺀" * 40,
             "a!\n/\n/b" * 20, "x" + "1〇" * 60]
    for t in texts:
        assert split(t, kimi=True) == oracle_split(o, t), repr(t)
        assert split(t, block=64, kimi=True) == oracle_split(o, t), repr(t)
