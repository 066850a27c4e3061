"""CPU model of the workgroup merge of segments over 512 bytes
(``block_bpe`` in ``k_seg_block``), transcribed step by step: per 1024-byte
chunk the lowest key (rank << 32 | offset), then per round the global
minimum, the selection of its rank's pairs by the two-state automaton
carried across chunks, the merges, and the recomputed pairs and minima of
the chunks the merges touched.

It equals the oracle on letter runs of the non-monotone Llama stand-in,
whose guarded ranks merge one occurrence a round (hundreds of rounds a
piece).

Planted: the race the device had. Thread 0 stored the last recomputed
chunk minimum after the barriers of the block-wide minimum, and the next
round's threads read their chunk's minimum before any barrier. A round
that sees the old minimum of that chunk picks the pair a round before it
merged. The model shows the consequence: a merge through a dead symbol's
stale links (the device's ``merge`` then wrote ``dirty[(q - a) / 1024]``
with ``q = -1``, far out of bounds) or wrong ids. The fix is a barrier at
the end of each round, and a guard that reports a dead link instead of
writing through it.
"""

from __future__ import annotations

import json
from functools import lru_cache

import numpy as np
import pytest

T = 1024  # SEGB_TPB: bytes per chunk
INV = 0xFFFFFFFF
NOPAIR = 0xFFFFFFFE
NOSYM = (1 << 64) - 1


@lru_cache(maxsize=2)
def _model(family: str):
    from toktier_amd import bpe_tables, standin
    m = json.loads(standin.load_artifact_json(family))["model"]
    vocab = m["vocab"]
    rules = {}
    for r, (a, b) in enumerate(bpe_tables._merge_pairs(m["merges"])):
        rules.setdefault((vocab[a], vocab[b]), (r, vocab[a + b]))
    unsafe = set(bpe_tables.unsafe_ranks(m["merges"]))
    b2u = bpe_tables.bytes_to_unicode()
    return rules, unsafe, [vocab[b2u[b]] for b in range(256)]


class DeadLink(Exception):
    """A merge reached a symbol without a live right neighbour."""


def block_bpe(data: bytes, family: str, stale_last_min: bool = False):
    """The merge; ``stale_last_min`` plants the race: each round's global
    minimum sees the minimum the last chunk the round before recomputed
    had before that recompute."""
    rules, unsafe, byte_id = _model(family)
    n = len(data)
    nch = (n + T - 1) // T
    tok = [byte_id[b] for b in data]
    nx = [i + 1 if i + 1 < n else -1 for i in range(n)]
    pv = [i - 1 for i in range(n)]
    pair = [rules.get((tok[i], tok[i + 1])) if i + 1 < n else None for i in range(n)]

    def chunk_min(c):
        best = NOSYM
        for i in range(c * T, min(n, c * T + T)):
            if tok[i] != INV:
                p = pair[i]
                best = min(best, ((NOPAIR if p is None else p[0]) << 32) | i)
        return best
    cmin = [chunk_min(c) for c in range(nch)]
    selr = [0] * n
    dirty = [0] * nch
    last = None  # (chunk, its minimum before the last recompute)
    rnd = 0
    while True:
        rnd += 1
        seen = list(cmin)
        if stale_last_min and last is not None and last[0] != 0:
            seen[last[0]] = last[1]  # thread c read before thread 0 stored
        m = min(seen)
        R = m >> 32
        if R >= NOPAIR:
            break
        s0 = m & 0xFFFFFFFF
        if pair[s0] is None or tok[s0] == INV:
            raise DeadLink(s0)
        prod = pair[s0][1]
        if R in unsafe:
            sel = [s0]
        else:
            sel, carry = [], 0
            for c in range(nch):
                if (cmin[c] >> 32) != R:
                    if cmin[c] != NOSYM:
                        carry = 0
                    continue
                for i in range(c * T, min(n, c * T + T)):
                    if tok[i] == INV:
                        continue
                    if pair[i] is not None and pair[i][0] == R:
                        carry = 0 if carry else 1
                        if carry:
                            sel.append(i)
                    else:
                        carry = 0
        for i in sel:
            q = nx[i]
            if q < 0 or tok[q] == INV:
                raise DeadLink(i)
            nn = nx[q]
            tok[i], tok[q], nx[i] = prod, INV, nn
            if nn >= 0:
                pv[nn] = i
            selr[i] = rnd
            for x in (i, q, pv[i]):
                if x >= 0:
                    dirty[x // T] = rnd
        last = None
        for c in range(nch):
            if dirty[c] != rnd:
                continue
            for i in range(c * T, min(n, c * T + T)):
                if tok[i] == INV:
                    continue
                q = nx[i]
                if selr[i] == rnd or (q >= 0 and selr[q] == rnd):
                    pair[i] = rules.get((tok[i], tok[q])) if q >= 0 else None
            last = (c, cmin[c])
            cmin[c] = chunk_min(c)
    return [t for t in tok if t != INV]


def _runs(n_pieces: int, seed: int):
    """Letter runs of 2,500-4,000 bytes from C5's text (three or four
    chunks each, so the last recomputed chunk is rarely chunk 0)."""
    from toktier_amd import standin, workloads
    js = standin.load_artifact_json("llama_3_1_8b")
    text = workloads.config5(js, n_chars=60_000, n_runs=2, run_chars=6_000, sample=seed)
    letters = "".join(ch for ch in text if ch.isalpha() and ord(ch) < 0x3000)
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n_pieces):
        k = int(rng.integers(2_500, 4_000))
        a = int(rng.integers(0, len(letters) - k))
        out.append(letters[a:a + k].encode("utf-8"))
    return out


@pytest.fixture(scope="module")
def llama():
    from conftest import kit
    return kit("llama_3_1_8b")


def test_block_merge_equals_the_oracle_on_guarded_runs(llama):
    rules, unsafe, _ = _model("llama_3_1_8b")
    assert unsafe, "the Llama stand-in has guarded ranks"
    for data in _runs(4, 31):
        assert block_bpe(data, "llama_3_1_8b") == list(llama.oracle.encode_bytes(data))


def test_stale_chunk_minimum_breaks_the_merge(llama):
    """The planted race: some piece merges through a dead link or ends
    with ids that differ from the oracle's."""
    broken = 0
    for data in _runs(4, 31):
        try:
            got = block_bpe(data, "llama_3_1_8b", stale_last_min=True)
        except DeadLink:
            broken += 1
            continue
        broken += got != list(llama.oracle.encode_bytes(data))
    assert broken > 0
