"""CPU model of the long-piece certification (the device's cut / segment /
certify path, ``k_long_segments`` + ``k_certify``).

A piece is cut into segments; each segment is merged alone, recording its
merge rounds (rank, whether the round changed the segment's first / last
token, its product). A cut holds
when, walking the two adjacent segments' rounds in the order the whole
piece would run them (the left segment's next round first when its rank is
at most the right one's), the pair across the cut always loses to one of
the two heads. The property checked here: whenever every cut of a piece
holds, the concatenated segment merges equal the whole piece's merge in the
HF order (lowest rank first, leftmost on ties), on the non-monotone Llama
stand-in (ranks whose product an earlier rule consumes) and on the
monotone Qwen stand-in, with single-merge rounds (the lane-per-byte wave
merge) and guarded batch rounds (the wide merge: every leftmost
non-overlapping occurrence of a rank that no earlier rule consumes the
product of, else its leftmost one alone). A batch round needs no check of
the states inside it: its product is consumed only by later rules, so the
pair it leaves across a cut ranks above it (checked here too). Planted
mistakes in the walk (ties to the right segment, the right-hand comparison
made strict, the left token never updated) let a cut set through with
wrong ids (pinned counterexamples found by a seeded search).
"""

from __future__ import annotations

import json
from functools import lru_cache

import numpy as np
import pytest

INF = 1 << 62


@lru_cache(maxsize=4)
def _model(family: str):
    from toktier_amd import bpe_tables, standin
    js = standin.load_artifact_json(family)
    m = json.loads(js)["model"]
    vocab = m["vocab"]
    rules = {}
    for r, (a, b) in enumerate(bpe_tables._merge_pairs(m["merges"])):
        rules.setdefault((vocab[a], vocab[b]), (r, vocab[a + b]))
    unsafe = set(bpe_tables.unsafe_ranks(m["merges"]))
    b2u = bpe_tables.bytes_to_unicode()
    byte_id = [vocab[b2u[b]] for b in range(256)]
    return rules, unsafe, byte_id


def _rank(rules, a, b):
    v = rules.get((a, b))
    return v[0] if v else INF


def merge(rules, unsafe, ids, batch: bool):
    """The segment's merge in rounds; returns (final ids, rounds) with a
    round = (rank, first, last, product, multi)."""
    ids = list(ids)
    rounds = []
    while len(ids) > 1:
        ranks = [_rank(rules, ids[i], ids[i + 1]) for i in range(len(ids) - 1)]
        r = min(ranks)
        if r == INF:
            break
        prod = rules[(ids[ranks.index(r)], ids[ranks.index(r) + 1])][1]
        sel = []
        i = 0
        while i < len(ranks):
            if ranks[i] == r:
                sel.append(i)
                if not batch or r in unsafe:
                    break
                i += 2
            else:
                i += 1
        first = sel[0] == 0
        last = sel[-1] == len(ids) - 2
        for i in reversed(sel):
            ids[i:i + 2] = [prod]
        rounds.append((r, first, last, prod, len(sel) > 1))
    return ids, rounds


def walk(rules, L, R, ra_list, rb_list, ties_left=True):
    """The device's cut check over the two segments' rounds (k_certify,
    cert mode 2). True when the pair across the cut never merges."""
    i = j = 0
    while True:
        ra = ra_list[i][0] if i < len(ra_list) else INF
        rb = rb_list[j][0] if j < len(rb_list) else INF
        rho = _rank(rules, L, R)
        if rho < ra and rho <= rb:
            return False
        if ra == INF and rb == INF:
            return True
        if (ra <= rb) if ties_left else (ra < rb):
            e = ra_list[i]
            i += 1
            if e[2]:
                L = e[3]
        else:
            e = rb_list[j]
            j += 1
            if e[1]:
                R = e[3]


def walk_events(rules, L, R, ra_list, rb_list):
    """The first / last-token event walk (cert mode 1), exact only for
    monotone tables: events alone, no other heads."""
    ea = [e for e in ra_list if e[2]]
    eb = [e for e in rb_list if e[1]]
    i = j = 0
    while True:
        ra = ea[i][0] if i < len(ea) else INF
        rb = eb[j][0] if j < len(eb) else INF
        rho = _rank(rules, L, R)
        if rho < ra and rho <= rb:
            return False
        if ra == INF and rb == INF:
            return True
        if ra <= rb:
            L = ea[i][3]
            i += 1
        if rb <= ra:
            R = eb[j][3]
            j += 1


def _pieces(family: str, n: int, seed: int):
    from toktier_amd import standin, workloads
    js = standin.load_artifact_json(family)
    text = workloads.config5(js, n_chars=60_000, n_runs=2, run_chars=4_000,
                             sample=seed)
    letters = "".join(ch for ch in text if ch.isalpha())
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        k = int(rng.integers(12, 60))
        a = int(rng.integers(0, len(letters) - k))
        out.append(letters[a:a + k].encode("utf-8"))
    return out, rng


def _trial(family, data, cuts, batch, walker):
    rules, unsafe, byte_id = _model(family)
    ids = [byte_id[b] for b in data]
    whole, _ = merge(rules, unsafe, ids, False)
    bounds = [0, *cuts, len(ids)]
    segs = [merge(rules, unsafe, ids[a:b], batch)
            for a, b in zip(bounds, bounds[1:])]
    ok = all(walker(rules, ids[c - 1], ids[c], segs[k][1], segs[k + 1][1])
             for k, c in enumerate(cuts))
    cat = [t for s in segs for t in s[0]]
    return ok, cat == whole


def _cuts(rng, n):
    k = int(rng.integers(1, 4))
    return sorted(set(int(x) for x in rng.integers(1, n, size=k)))


def _true_cuts(family, data, rng):
    """Cuts at the whole piece's own token boundaries (a random subset)."""
    rules, unsafe, byte_id = _model(family)
    whole, _ = merge(rules, unsafe, [byte_id[b] for b in data], False)
    rules_len = []
    at = 0
    for t in whole[:-1]:
        at += _token_len(family, t)
        rules_len.append(at)
    if not rules_len:
        return []
    k = int(rng.integers(1, min(4, len(rules_len)) + 1))
    return sorted(set(int(x) for x in rng.choice(rules_len, size=k)))


@lru_cache(maxsize=4)
def _lengths(family: str):
    from toktier_amd import standin
    from oracle.oracle import token_byte_lengths
    return token_byte_lengths(standin.load_artifact_json(family))


def _token_len(family, t):
    return int(_lengths(family)[t])


@pytest.mark.parametrize("family,batch", [("llama_3_1_8b", False),
                                          ("llama_3_1_8b", True),
                                          ("qwen3_8b", False),
                                          ("qwen3_8b", True)])
def test_a_cut_set_that_holds_gives_the_whole_piece(family, batch):
    rules, unsafe, _ = _model(family)
    if family == "llama_3_1_8b":
        assert unsafe, "the Llama stand-in is the non-monotone case"
    pieces, rng = _pieces(family, 300, 5)
    held = 0
    for data in pieces:
        # random cuts: sound (a set that holds gives the whole piece)
        cuts = _cuts(rng, len(data))
        ok, same = _trial(family, data, cuts, batch, walk)
        assert not ok or same, (family, data, cuts)
        held += ok
        # cuts at the piece's own token boundaries: no merge ever crosses
        # them, and with one merge per round the walk is exact, so they hold
        cuts = _true_cuts(family, data, rng)
        ok, same = _trial(family, data, cuts, batch, walk)
        assert same, (family, data, cuts)
        assert ok or batch, (family, data, cuts)
        held += ok
    # the check is not vacuous: many cut sets hold
    assert held > 300, held


def test_guarded_batch_rounds_equal_the_hf_order():
    rules, unsafe, byte_id = _model("llama_3_1_8b")
    pieces, _ = _pieces("llama_3_1_8b", 300, 6)
    for data in pieces:
        ids = [byte_id[b] for b in data]
        assert merge(rules, unsafe, ids, True)[0] == merge(rules, unsafe, ids, False)[0]


def test_batch_round_products_rank_above_their_round():
    """The pair a batch round leaves across a cut while it goes on (left
    token, the round's product) never ranks at or below the round."""
    rules, unsafe, byte_id = _model("llama_3_1_8b")
    pieces, _ = _pieces("llama_3_1_8b", 300, 7)
    vocab_ids = sorted({t for (a, b) in rules for t in (a, b)})
    consumers: dict[int, int] = {}
    for (a, b), (r, _) in rules.items():
        consumers[b] = min(consumers.get(b, INF), r)
    for data in pieces:
        _, rounds = merge(rules, unsafe, [byte_id[b] for b in data], True)
        for r, first, last, prod, multi in rounds:
            if multi:
                assert r not in unsafe
                assert consumers.get(prod, INF) > r
    assert vocab_ids


def walk_planted(rules, L, R, A, B, mistake):
    """``walk`` with one planted mistake: ties to the right segment, the
    right-hand comparison made strict, or the left token never updated."""
    i = j = 0
    while True:
        ra = A[i][0] if i < len(A) else INF
        rb = B[j][0] if j < len(B) else INF
        rho = _rank(rules, L, R)
        if rho < ra and (rho < rb if mistake == "strict_b" else rho <= rb):
            return False
        if ra == INF and rb == INF:
            return True
        if (ra < rb) if mistake == "ties_right" else (ra <= rb):
            e = A[i]
            i += 1
            if e[2] and mistake != "stale_left":
                L = e[3]
        else:
            e = B[j]
            j += 1
            if e[1]:
                R = e[3]


# counterexamples found by a seeded search over the Llama stand-in's letter
# runs (pieces of _pieces(), random cuts): each planted walk lets its cut
# set through with ids that differ from the whole piece
PLANTED = [
    ("ties_right", b"kresXAAAAAAAAAAAAAAAAAAAAAAAAAAAAAAAAFSreAAD"
                   b"\xe5\xa6\xb4\xe9\x92\xbf\xe5\xa6\xb4", [15, 44]),
    ("strict_b", b"\xe6\x8a\x89\xe5\xa6\xb4\xe5\xa6\xb4\xe5\xa6\xb4\xe6\x8a\x89"
                 b"\xe9\x88\xb0\xe7\xb6\x8d\xe7\xb4\xb9\xe6\x8a\x89\xe9\x88\xb0"
                 b"\xe7\xb6\x8d\xe7\xb4\xb9HykSeparsi", [6]),
    ("stale_left", b"\xe9\x88\xb0\xe7\xb6\x8d\xe5\x90\xa8\xe7\xb4\xb9\xe9\x90\xa4"
                   b"\xe6\xaf\xa8\xe5\xa6\xb4\xe5\xa6\xb4\xe5\xa6\xb4\xe9\x92\xbf"
                   b"\xe5\x90\xa8\xe6\xb4\xbd\xe7\xbe\x90\xe8\x80\xbd\xe7\xb6\x8d"
                   b"\xe5\xa6\xb4\xe9\x92\xbf\xe5\xa6\xb4\xe9\x92\xbf\xe5\xa6\xb4"
                   b"onsenowryallKeysVERSIONSBarg", [8, 44]),
]


@pytest.mark.parametrize("mistake,data,cuts", PLANTED)
def test_planted_walk_mistakes_are_caught(mistake, data, cuts):
    planted = _trial("llama_3_1_8b", data, cuts, False,
                     lambda *a: walk_planted(*a, mistake))
    assert planted == (True, False), mistake  # holds, with wrong ids
    ok, same = _trial("llama_3_1_8b", data, cuts, False, walk)
    assert same or not ok, mistake  # the correct walk refuses it


# ------------------------------------------------------- the repair passes

def window_cuts(family, ids, lens, off):
    """k_long_windows on a piece whose first byte is text position `off`:
    every 64-byte window of both grids (text positions 64v and 64v - 32),
    clipped to the piece, merged alone; the token starts in its central 32
    bytes become cuts (piece offsets)."""
    rules, unsafe, _ = _model(family)
    n = len(ids)
    cuts = set()
    for ws in range((off // 32) * 32 - 32, off + n, 32):
        a, b = max(ws, off), min(ws + 64, off + n)
        if a >= b:
            continue
        toks, _ = merge(rules, unsafe, ids[a - off:b - off], True)
        pos = a
        for t in toks:
            if ws + 16 <= pos < ws + 48 and off < pos:
                cuts.add(pos - off)
            pos += lens[t]
    return sorted(cuts)


def repair(family, data, off, widen_from=None, limit=10_000, first_max=None,
           stats=None):
    """The certification and its repair passes on one piece: certify every
    cut, drop the failed ones, redo the segments, until none fails (cert 1,
    a monotone table). From pass `widen_from` on, each failed cut also
    drops its 4^(p - widen_from + 1) nearest cuts on each side
    (k_fail_widen). With `first_max`, the first pass fails both cuts around
    every segment longer than that instead of merging it (the device's
    first segment pass: fail_segment_cuts past 64 bytes), and a segment
    with no cut to fail still makes the repair pass run. Returns (ids,
    passes)."""
    rules, unsafe, byte_id = _model(family)
    lens = _lengths(family)
    ids = [byte_id[b] for b in data]
    cuts = window_cuts(family, ids, lens, off)
    passes = 0
    while True:
        bounds = [0, *cuts, len(ids)]
        # (the first pass leaves a segment over first_max unmerged: its
        # bytes, no events)
        segs = [(list(ids[a:b]), []) if first_max and passes == 0 and b - a > first_max
                else merge(rules, unsafe, ids[a:b], True)
                for a, b in zip(bounds, bounds[1:])]
        failed = [k for k, c in enumerate(cuts)
                  if not walk_events(rules, ids[c - 1], ids[c], segs[k][1], segs[k + 1][1])]
        forced = False
        if first_max and passes == 0:
            extra = set()
            for k, (a, b) in enumerate(zip(bounds, bounds[1:])):
                if b - a > first_max:
                    forced = True
                    extra.update(j for j in (k - 1, k) if 0 <= j < len(cuts))
            failed = sorted(set(failed) | extra)
            if stats is not None:
                stats["long_first"] = stats.get("long_first", 0) + int(forced)
        if (not failed and not forced) or passes >= limit:
            return [t for s in segs for t in s[0]], passes
        passes += 1
        width = 4 ** (passes - widen_from + 1) if widen_from and passes >= widen_from else 0
        drop = set()
        for k in failed:
            drop.update(range(max(0, k - width), min(len(cuts), k + width + 1)))
        cuts = [c for k, c in enumerate(cuts) if k not in drop]


def test_repair_passes_cascade_on_periodic_runs_and_widening_ends_them():
    """A run of one letter led by a character that joins its piece ("!"
    + "QQQ...": one piece under the Qwen2 pattern) fixes the token parity
    at its first window, while every later window pairs the letters from
    an even text position. Removing the one cut that fails makes the next
    one fail: one cut per pass, so the passes grow with the run. Dropping a
    fourfold wider ring of cuts around each failed one from pass 4 on (the
    device's REPAIR_WIDEN) ends them within about log4 of the run's cuts,
    with the whole piece's ids."""
    family = "qwen3_8b"
    rules, unsafe, byte_id = _model(family)
    for n in (300, 600, 1200, 4000):
        data = b"!" + b"Q" * n
        whole, _ = merge(rules, unsafe, [byte_id[b] for b in data], True)
        if n <= 1200:
            ids, passes = repair(family, data, off=64)
            assert ids == whole
            assert passes >= n // 2 - 40, (n, passes)  # one cut per pass
        ids, passes = repair(family, data, off=64, widen_from=4)
        assert ids == whole and passes <= 3 + 8, (n, passes)


def test_widened_repair_keeps_the_ids_of_ordinary_pieces():
    """Letter runs of C5's text (monotone Qwen table) at shifting text
    offsets: the widened repair loop gives the whole piece's ids, widened
    from the first pass too."""
    family = "qwen3_8b"
    rules, unsafe, byte_id = _model(family)
    from toktier_amd import standin, workloads
    js = standin.load_artifact_json(family)
    text = workloads.config5(js, n_chars=40_000, n_runs=2, run_chars=3_000, sample=9)
    letters = "".join(ch for ch in text if ch.isalpha()).encode("utf-8")
    rng = np.random.default_rng(21)
    for _ in range(12):
        k = int(rng.integers(513, 1500))
        a = int(rng.integers(0, len(letters) - k))
        while a < len(letters) and (letters[a] & 0xC0) == 0x80:
            a += 1
        data = letters[a:a + k]
        while data and (data[-1] & 0xC0) == 0x80 or (data and data[-1] >= 0xC0):
            data = data[:-1]
        whole, _ = merge(rules, unsafe, [byte_id[b] for b in data], True)
        for widen in (1, 4):
            ids, passes = repair(family, data, off=int(rng.integers(0, 64)),
                                 widen_from=widen)
            assert ids == whole, (widen, passes)


def test_first_pass_long_segments_left_to_the_repair_passes():
    """The device's first segment pass fails the cuts around a segment over
    64 bytes instead of merging it there (k_long_segments:
    fail_segment_cuts), and the repair passes join and merge it. The ids
    stay the whole piece's: space runs and periodic runs, where the windows
    find few cuts and segments run past 64 bytes, C5 letter runs, and the
    cascading "!" + "QQQ..." run."""
    family = "qwen3_8b"
    rules, unsafe, byte_id = _model(family)
    from toktier_amd import standin, workloads
    js = standin.load_artifact_json(family)
    text = workloads.config5(js, n_chars=40_000, n_runs=2, run_chars=3_000, sample=5)
    letters = "".join(ch for ch in text if ch.isalpha()).encode("utf-8")
    cases = [b" " * 1500, b"ab" * 700, b"\t\n " * 400, b"!" + b"Q" * 900,
             letters[:1200], letters[3000:4100]]
    stats = {}
    for data in cases:
        while data and (data[-1] & 0xC0) == 0x80 or (data and data[-1] >= 0xC0):
            data = data[:-1]
        whole, _ = merge(rules, unsafe, [byte_id[b] for b in data], True)
        for off in (0, 37):
            ids, passes = repair(family, data, off=off, widen_from=4, first_max=64,
                                 stats=stats)
            assert ids == whole, (data[:8], off, passes)
    assert stats.get("long_first", 0) > 0  # the path ran
