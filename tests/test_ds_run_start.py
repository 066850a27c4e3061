"""CPU model of DeepSeek's letter-after-run decision on the device
(``ds_run_led``, ``ds_stop_hbm`` and the ``FAST_FAR`` search in
``k_pretok<3, ...>``).

DeepSeek's main pattern starts ``[ascii punct][A-Za-z]+``. So a letter or
mark right after an ASCII-letter run starts a piece exactly when that
alternative took the run. That holds when no document starts inside the
run, and the character before the run is ASCII punctuation that starts its
own match: no P/S character and no U+0020 before it in its region, or a
document start at it. The answer therefore needs only ``s``, the highest
position below the run that is not an ASCII letter or that opens a
document, however far back the run begins.

The device finds ``s`` in one of three ways:
- inside the lane's 64-byte word, from the word's byte masks;
- else the wave searches the tile's staged bytes, 64 a step;
- past those, it searches the text in HBM, one 64-byte chunk per lane in
  4 KiB steps.

There is no wait on another tile. The model restates each of the three
with the device's index arithmetic: word and tile geometry, chunk masks,
and lane order. It checks, against the oracle's split, every such position
in texts with runs of 3 to 9,000 letters placed at shifting offsets across
words and 2816-byte tiles, with document starts inside the runs, at their
punctuation and just before it. It checks both tiles that decide a
position near a tile edge: its own tile, and the tile before it, whose
recomputed word after the tile reaches the span end through the general
walk. Planted mistakes must each decide some position differently: document
starts ignored in the HBM chunks, the first chunk's mask one byte short,
the character before the punctuation not read, and the LDS search stopping
a step early.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import kit

PT_TILE, PT_PAD, PT_HALO = 2816, 80, 64  # tk_device.h / tk_device.hip
PT_SPAN = PT_TILE + 2 * PT_HALO
DS_O, DS_L, DS_M, DS_N, DS_PS, DS_WS, DS_CR = range(7)


def ascii_alpha(b: int) -> bool:
    return 0 <= (b | 32) - 97 < 26


def ascii_punct(c: int) -> bool:
    return (0x21 <= c <= 0x2F or 0x3A <= c <= 0x40 or 0x5B <= c <= 0x60
            or 0x7B <= c <= 0x7E)


def ds_cjk(c: int) -> bool:
    return 0x4E00 <= c <= 0x9FA5 or 0x3040 <= c <= 0x30FF


class Text:
    def __init__(self, data: bytes, docs, cls):
        self.data = data
        self.docs = set(docs) | {0}
        self.cls = cls

    def ds(self, p: int) -> bool:
        return p in self.docs

    def char_at(self, p: int) -> tuple[int, int]:
        """(code point, class) of the character whose lead byte is p
        (U+FFFD for a byte that starts no valid character)."""
        b = self.data[p]
        n = 1 if b < 0x80 else 2 if 0xC0 <= b < 0xE0 else 3 if 0xE0 <= b < 0xF0 \
            else 4 if 0xF0 <= b < 0xF8 else 0
        try:
            cp = ord(self.data[p:p + n].decode("utf-8")) if n else 0xFFFD
        except UnicodeDecodeError:
            cp = 0xFFFD
        return cp, int(self.cls[cp])

    def prev(self, s: int) -> int:
        """Start of the character before the one at s (-1 at a document
        start): at most three continuation bytes back, not below 0."""
        if self.ds(s):
            return -1
        q = s - 1
        k = 0
        while q > 0 and k < 3 and (self.data[q] & 0xC0) == 0x80:
            q -= 1
            k += 1
        return q

    def docword(self, w: int) -> int:
        m = 0
        for j in range(64):
            if self.ds(64 * w + j):
                m |= 1 << j
        return m


def run_led(t: Text, s: int, plant=None) -> bool:
    """ds_run_led: the character whose last byte is s leads the run."""
    if s < 0:
        return False
    b = t.data[s]
    if not (b < 0x80 and ascii_punct(b)):
        return False
    q = t.prev(s)
    if q < 0:
        return True
    if plant == "no_arrival":
        return True
    cp, cl = t.char_at(q)
    region = 2 if cl == DS_N else 1 if ds_cjk(cp) else 0
    return region != 0 or (cl != DS_PS and cp != 0x20)


def stop_hbm(t: Text, q: int, plant=None) -> int:
    """ds_stop_hbm: lane l takes chunk (cq - l) of each 4 KiB step."""
    assert q >= 0
    cq = q >> 6
    while True:
        for lane in range(64):
            ch = cq - lane
            if ch < 0:
                continue
            m = 0
            for j in range(64):
                if not ascii_alpha(t.data[64 * ch + j]):
                    m |= 1 << j
            if plant != "no_docs_hbm":
                m |= t.docword(ch)
            if ch == 0:
                m |= 1
            if ch == q >> 6:
                h = (q & 63) - (1 if plant == "chunk_mask_short" else 0)
                m &= (2 << h) - 1 if h >= 0 else 0
            if m:  # the lowest such lane holds the highest stop
                return 64 * ch + m.bit_length() - 1
        cq -= 64


def stop_tile(t: Text, base: int, frm: int, plant=None) -> int:
    """The ds_stop lambda of k_pretok's start words: the staged bytes
    [base - PT_PAD, ...) 64 a step, then the HBM search."""
    st0 = base - PT_PAD
    lo_st = max(st0, 0)
    top = frm
    floor = lo_st + (64 if plant == "lds_short" else 0)
    while top >= floor:
        hits = [top - lane for lane in range(64)
                if top - lane >= lo_st and (not ascii_alpha(t.data[top - lane])
                                            or t.ds(top - lane))]
        if hits:
            return max(hits)
        top -= 64
    return stop_hbm(t, lo_st - 1, plant)


def decide(t: Text, i: int, base: int, plant=None) -> bool:
    """The device's answer at position i (a letter / mark after an ASCII
    letter, no document start at i) when tile ``base`` computes it."""
    k = (i - base) // 64
    lane = (i - base) % 64
    lo = base - PT_HALO
    li = i - lo
    # the fixed context's next-character check fails at the span's end:
    # the general walk (start_deepseek) then runs down the run in the span
    fwd = len(t.data[i:i + 4].decode("utf-8", errors="ignore")[:1].encode()) or 1
    if li + fwd >= PT_SPAN:
        q = i - 1
        while True:
            if t.ds(q):
                return False
            r = q - 1
            if not (0 <= r - lo < PT_SPAN):
                return run_led(t, stop_tile(t, base, r, plant), plant)
            if not ascii_alpha(t.data[r]):
                return run_led(t, r, plant)
            q = r
    wstart = base + 64 * k
    for p in range(i - 1, wstart - 1, -1):  # stop bits below the lane
        if not ascii_alpha(t.data[p]) or t.ds(p):
            return run_led(t, p, plant)
    assert lane == i - wstart and wstart > 0
    return run_led(t, stop_tile(t, base, wstart - 1, plant), plant)


def candidates(t: Text):
    """Positions of a letter / mark (region 0, not an ASCII letter) right
    after an ASCII letter, with no document start at them."""
    d = t.data
    out = []
    for i in range(1, len(d)):
        if (d[i] & 0xC0) == 0x80 or t.ds(i) or not ascii_alpha(d[i - 1]):
            continue
        cp, cl = t.char_at(i)
        if cl in (DS_L, DS_M) and not ascii_alpha(cp) and not ds_cjk(cp):
            out.append(i)
    return out


def oracle_starts(o, t: Text) -> set[int]:
    cuts = sorted(t.docs | {len(t.data)})
    out = set()
    for a, b in zip(cuts, cuts[1:]):
        out.update(a + s for s in o.pretokenize(t.data[a:b])[:-1])
    return out


PREFIXES = ["", "!", "a!", " !", "!!", "中!", "\n!", "é!", "1!", "。!",
            "٣!", "\t!", "x "]
TAILS = ["́", "️", "é", "ā"]
LENGTHS = [3, 5, 63, 64, 65, 130, 2815, 2816, 2817, 3 * PT_TILE + 17, 9000]


def _texts(seed: int, n: int = 6):
    """Texts of run cases at random offsets, with document starts in and
    around some of the runs."""
    rng = np.random.default_rng(seed)
    for _ in range(n):
        parts, docs, pos = [], [], 0
        filler = "".join(rng.choice(list("ab c,!é中\n1"), size=int(rng.integers(0, 3000))))
        parts.append(filler)
        pos += len(filler.encode())
        for _ in range(int(rng.integers(2, 6))):
            pre = PREFIXES[int(rng.integers(len(PREFIXES)))]
            nrun = LENGTHS[int(rng.integers(len(LENGTHS)))]
            tail = TAILS[int(rng.integers(len(TAILS)))]
            run = "".join(rng.choice(list("QabZ"), size=nrun))
            case = pre + run + tail
            cb = len(pre.encode())
            how = int(rng.integers(0, 5))
            if how == 1 and cb:  # at the punctuation
                docs.append(pos + cb - 1)
            elif how == 2 and cb > 1:  # just before it
                docs.append(pos + cb - 2)
            elif how == 3:  # inside the run
                docs.append(pos + cb + int(rng.integers(0, nrun)))
            parts.append(case)
            pos += len(case.encode())
            gap = " " * int(rng.integers(0, 2)) + "".join(
                rng.choice(list("xy!. "), size=int(rng.integers(0, 200))))
            parts.append(gap)
            pos += len(gap.encode())
        data = "".join(parts).encode()
        yield data, sorted(d for d in set(docs) if 0 < d < len(data)
                           and (data[d] & 0xC0) != 0x80)


@pytest.fixture(scope="module")
def dsk():
    from toktier_amd import classes
    return kit("deepseek_v3").oracle, classes.deepseek_class_table()


def _check(o, cls, data, docs, plant=None):
    t = Text(data, docs, cls)
    want = oracle_starts(o, t)
    bad = []
    for i in candidates(t):
        tiles = {(i // PT_TILE) * PT_TILE}
        if i % PT_TILE < 64 and i >= PT_TILE:  # the tile before recomputes it
            tiles.add((i // PT_TILE - 1) * PT_TILE)
        for base in tiles:
            if decide(t, i, base, plant) != (i in want):
                bad.append((i, base))
    return bad


@pytest.mark.parametrize("seed", range(8))
def test_run_start_decision_matches_the_oracle(dsk, seed):
    o, cls = dsk
    n = 0
    for data, docs in _texts(20261210 + seed):
        assert _check(o, cls, data, docs) == [], seed
        n += 1
    assert n


def test_run_start_decision_at_every_tile_offset(dsk):
    """A run that ends at each byte of the 64 around a tile edge, led by
    punctuation that does or does not start its own match, runs long
    enough to reach the HBM search, and a document start inside one."""
    o, cls = dsk
    for end in range(-40, 40, 3):
        for pre, n in (("!", 5000), (" !", 5000), ("!", 40), ("a!", 200)):
            head = "y" * 700 + pre
            # the run's last letter at byte end - 1 of tile 4's start
            shift = 4 * PT_TILE + end - (len(head) + n)
            data = ("z" * shift + head + "Q" * n + "\u0301").encode()
            for docs in ([], [len(data) - 40], [shift + len(head) - 1]):
                assert _check(o, cls, data, docs) == [], (end, pre, n, docs)


def _pinned(plant: str):
    """A text whose decision the planted mistake changes, built for it:
    tile 3 decides the letter after a run that reaches below its staged
    bytes (base - PT_PAD) or starts just inside them."""
    base = 3 * PT_TILE
    run = "Q" * 300 + "é"
    if plant == "chunk_mask_short":  # the stop is the search's first byte
        return ("a" * (base - PT_PAD - 1) + "!" + run).encode(), []
    if plant == "lds_short":  # the stop is in the staged bytes' last step
        return ("a" * (base - 71) + "!" + run).encode(), []
    if plant == "no_docs_hbm":  # a document starts inside the run, far back
        return ("a" * 99 + "!" + "Q" * (base - 100) + run).encode(), [2000]
    return ("a" * 99 + " !" + "Q" * (base - 101) + run).encode(), []


@pytest.mark.parametrize("plant", ["no_docs_hbm", "chunk_mask_short",
                                   "no_arrival", "lds_short"])
def test_planted_search_mistakes_are_caught(dsk, plant):
    o, cls = dsk
    data, docs = _pinned(plant)
    assert _check(o, cls, data, docs) == []
    assert _check(o, cls, data, docs, plant) != [], plant
