"""CPU model of the device's cross-workgroup look-backs: ``k_pretok``'s
digit-run count and o200k automaton state per tile, and ``k_compact``'s
running totals per block.

Each protocol works the same way:
- a workgroup publishes a word tagged with the call number;
- later workgroups read their predecessors' words, waiting until the tag
  is the current call's;
- every wait is bounded, and a wait that runs out reports a stall (a
  status bit that names the stage) instead of hanging.

A waiting workgroup holds its slot. Liveness therefore rests on two rules:
1. The hardware dispatches a launch's workgroups to the eight XCDs in
   turn, and in order inside each XCD.
2. A workgroup publishes what its successors need before it waits on
   anything.

The model runs each workgroup as a sequence of steps: local work, publish,
polls. A scheduler keeps a bounded number of slots per XCD, dispatches in
that order, and advances a random resident workgroup at each step. It
plays two calls back to back over the same status words, so the second
call finds the first call's words in memory.

Checked, for random texts, slot counts and interleavings:
- every workgroup finishes with no stall;
- the values read equal a sequential computation;
- no workgroup ever waits on a predecessor that is itself blocked in a
  wait with nothing published, so waits never chain.

Planted mistakes must each be caught:
- publishing after the look-back (waits chain: a workgroup polls a
  blocked one);
- a path that returns without publishing (the successor's wait runs out:
  a stall);
- reading a word without checking its call tag (the previous call's value
  is read: a wrong count).
"""

from __future__ import annotations

import random

import pytest

XCDS = 8


class Stall(Exception):
    pass


class Sim:
    """Workgroups of one launch over shared status words."""

    def __init__(self, n, slots, rng, words, seq, bound=4000):
        self.n, self.slots, self.rng = n, slots, rng
        self.words, self.seq, self.bound = words, seq, bound
        self.state = ["new"] * n  # new / work / wait / done
        self.chained = []  # (waiter, waited-on) where the latter was waiting

    def poll(self, me, u):
        """One poll of workgroup u's word; records a wait on a workgroup
        that has not published this call's word and is itself waiting."""
        v = self.words.get(u)
        if self.state[u] == "wait" and (v is None or v[0] != self.seq):
            self.chained.append((me, u))
        return v

    def run(self, program):
        """program(sim, k) -> generator yielding "work" / "wait" per step."""
        queues = [[k for k in range(self.n) if k % XCDS == x] for x in range(XCDS)]
        resident: dict[int, object] = {}
        polls = {}
        while any(queues) or resident:
            for x in range(XCDS):  # in-order dispatch per XCD into free slots
                while queues[x] and sum(1 for k in resident if k % XCDS == x) < self.slots:
                    k = queues[x].pop(0)
                    resident[k] = program(self, k)
                    self.state[k] = "work"
                    polls[k] = 0
            k = self.rng.choice(sorted(resident))
            try:
                what = next(resident[k])
                self.state[k] = what
                if what == "wait":
                    polls[k] += 1
                    if polls[k] > self.bound:
                        raise Stall(k)
            except StopIteration:
                self.state[k] = "done"
                del resident[k]


# ------------------------------------------------ digit-run count (k_pretok)

def digit_tiles(rng, n):
    """Per tile: whether the run at its start reaches back past its halo
    (its halo is all digits), the run's N characters at its end, and
    whether the run spans the tile whole."""
    tiles = []
    for _ in range(n):
        kind = rng.random()
        if kind < 0.4:  # all digits: a long run passes through
            tiles.append((True, 44 * 64, True))
        elif kind < 0.7:  # digits at the end after a break
            tiles.append((rng.random() < 0.5, rng.randrange(0, 300), False))
        else:
            tiles.append((False, 0, False))
    return tiles


def digit_program(tiles, out, plant=None):
    def prog(sim, k):
        needs, cnt, full = tiles[k]
        yield "work"  # stage, decode, word ballots, thread 0's counts
        publish = not (plant == "skip_publish" and not needs)
        if publish and plant != "publish_after":
            sim.words[k] = (sim.seq, full, cnt)
        c0 = 0
        if needs and k > 0:
            for u in range(k - 1, -1, -1):
                while True:
                    v = sim.poll(k, u)
                    if v is not None and (v[0] == sim.seq or plant == "no_tag"):
                        break
                    yield "wait"
                c0 += v[2]
                if not v[1]:
                    break
        if publish and plant == "publish_after":
            sim.words[k] = (sim.seq, full, cnt)
        out[k] = c0
        yield "work"
    return prog


def digit_expected(tiles):
    out, run = [], 0
    for needs, cnt, full in tiles:
        out.append(run if needs else 0)
        run = run + cnt if full else cnt
    return out


def run_digits(seed, plant=None, n=120):
    rng = random.Random(seed)
    words = {}
    results = []
    for seq in (1, 2):  # two calls over the same words
        tiles = digit_tiles(rng, n)
        out = [None] * n
        sim = Sim(n, rng.choice([1, 2, 3, 8]), rng, words, seq)
        sim.run(digit_program(tiles, out, plant))
        results.append((out, digit_expected(tiles), sim.chained))
    return results


@pytest.mark.parametrize("seed", range(30))
def test_digit_run_lookback_is_live_and_exact(seed):
    for out, want, chained in run_digits(seed):
        assert out == want
        assert chained == []


def _caught(runner, plant, seeds=range(40)):
    for seed in seeds:
        try:
            res = runner(seed, plant)
        except Stall:
            return "stall"
        for out, want, chained in res:
            if out != want:
                return "wrong"
            if chained:
                return "chained"
    return None


def test_digit_run_planted_mistakes_are_caught():
    assert _caught(run_digits, "publish_after") == "chained"
    assert _caught(run_digits, "skip_publish") == "stall"
    assert _caught(run_digits, "no_tag") == "wrong"


# ------------------------------------------ o200k automaton state (k_pretok)

NST = 8


def o2k_tiles(rng, n):
    """Per tile: its function over the automaton's states (a tuple), and
    whether the word before it is constant (the fast path: no look-back)."""
    tiles = []
    for _ in range(n):
        if rng.random() < 0.5:
            f = tuple([rng.randrange(NST)] * NST)  # constant (ordinary text)
        else:
            f = tuple(rng.randrange(NST) for _ in range(NST))
        tiles.append((f, rng.random() < 0.3))
    return tiles


def o2k_program(tiles, out, plant=None):
    FRESH = 7

    def prog(sim, k):
        f, fast = tiles[k]
        yield "work"
        if k == 0 or fast:
            # the entry comes from the word before the tile; the state after
            # is published when the tile's last wave has carried it through
            entry = FRESH if k == 0 else out["halo"][k]
            out[k] = entry
            yield "work"
            sim.words[k] = (sim.seq, "INCL", f[entry])
            return
        if plant != "publish_after":
            sim.words[k] = (sim.seq, "AGG", f)  # before looking back
        g = tuple(range(NST))  # the function of the tiles after u up to k
        entry = None
        for u in range(k - 1, -1, -1):
            while True:
                v = sim.poll(k, u)
                if v is not None and (v[0] == sim.seq or plant == "no_tag"):
                    break
                yield "wait"
            if v[1] == "INCL":
                entry = g[v[2]]
                break
            g = tuple(g[v[2][s]] for s in range(NST))  # g after u's function
            if len(set(g)) == 1:
                entry = g[0]
                break
        if entry is None:
            entry = g[FRESH]
        out[k] = entry
        sim.words[k] = (sim.seq, "INCL", f[entry])
        yield "work"
    return prog


def o2k_expected(tiles):
    out, state = [], 7
    for f, _ in tiles:
        out.append(state)
        state = f[state]
    return out


def run_o2k(seed, plant=None, n=100):
    rng = random.Random(seed)
    words = {}
    results = []
    for seq in (1, 2):
        tiles = o2k_tiles(rng, n)
        want = o2k_expected(tiles)
        out = {"halo": want}  # a fast tile's halo word gives its entry
        sim = Sim(n, rng.choice([1, 2, 4, 8]), rng, words, seq)
        sim.run(o2k_program(tiles, out, plant))
        results.append(([out[k] for k in range(n)], want, sim.chained))
    return results


@pytest.mark.parametrize("seed", range(30))
def test_o200k_lookback_is_live_and_exact(seed):
    for out, want, chained in run_o2k(seed):
        assert out == want
        assert chained == []


def test_o200k_planted_mistakes_are_caught():
    assert _caught(run_o2k, "publish_after") == "chained"
    assert _caught(run_o2k, "no_tag") == "wrong"


# ------------------------------------------ compaction totals (k_compact)

def compact_program(counts, out, plant=None):
    def prog(sim, b):
        yield "work"  # count the block's ids, stage them
        tot = counts[b]
        if b == 0:
            sim.words[0] = (sim.seq, True, tot)
            out[0] = 0
            return
        if plant != "publish_after":
            sim.words[b] = (sim.seq, False, tot)  # the count, before waiting
        base = 0
        for j in range(b - 1, -1, -1):
            while True:
                v = sim.poll(b, j)
                if v is not None and (v[0] == sim.seq or plant == "no_tag"):
                    break
                yield "wait"
            base += v[2]
            if v[1]:
                break
        out[b] = base
        sim.words[b] = (sim.seq, True, base + tot)
        yield "work"
    return prog


def run_compact(seed, plant=None, n=150):
    rng = random.Random(seed)
    words = {}
    results = []
    for seq in (1, 2):
        counts = [rng.randrange(0, 5000) for _ in range(n)]
        out = [None] * n
        sim = Sim(n, rng.choice([1, 2, 4]), rng, words, seq)
        sim.run(compact_program(counts, out, plant))
        want = [sum(counts[:b]) for b in range(n)]
        results.append((out, want, sim.chained))
    return results


@pytest.mark.parametrize("seed", range(20))
def test_compaction_lookback_is_live_and_exact(seed):
    for out, want, chained in run_compact(seed):
        assert out == want
        assert chained == []


def test_compaction_planted_mistakes_are_caught():
    assert _caught(run_compact, "publish_after") == "chained"
    assert _caught(run_compact, "no_tag") == "wrong"


def test_dispatch_out_of_order_would_hang():
    """Why the in-order dispatch rule matters: with workgroups dispatched
    from the highest index down into one slot per XCD, the correct
    protocol's first waiter holds the only slot its predecessor needs,
    and the wait runs out."""
    rng = random.Random(1)
    tiles = [(True, 44 * 64, True)] * 16
    out = [None] * 16

    class Reversed(Sim):
        def run(self, program):
            order = list(range(self.n - 1, -1, -1))
            resident = {}
            polls = {}
            while order or resident:
                while order and len(resident) < self.slots:
                    k = order.pop(0)
                    resident[k] = program(self, k)
                    polls[k] = 0
                k = self.rng.choice(sorted(resident))
                try:
                    if next(resident[k]) == "wait":
                        polls[k] += 1
                        if polls[k] > self.bound:
                            raise Stall(k)
                except StopIteration:
                    del resident[k]

    with pytest.raises(Stall):
        Reversed(16, 1, rng, {}, 1).run(digit_program(tiles, out))
