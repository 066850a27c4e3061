"""Batch failure isolation (``resolve_failed_chunk``) against a stand-in
chunk encoder, as the reference tests its own search
(``crates/toktier-routing-core/src/gpu.rs:1820-1960``): any chunk holding a
poisoned document fails as a whole, every other chunk answers with ids
that are a function of the document alone."""

from __future__ import annotations

import pytest

from toktier_amd import resolve_failed_chunk


class Poison:
    def __init__(self, texts, poison):
        self.texts = texts
        self.poison = set(poison)
        self.attempts: list[int] = []

    @staticmethod
    def ids_of(text):
        return [ord(c) for c in text]

    def __call__(self, idx):
        self.attempts.append(len(idx))
        if any(self.texts[i] in self.poison for i in idx):
            raise RuntimeError("batched guard tripped")
        return [self.ids_of(self.texts[i]) for i in idx]


def run(size, faults):
    texts = ["poison" if i in faults else f"row-{i}" for i in range(size)]
    enc = Poison(texts, ["poison"])
    idx = list(range(size))
    with pytest.raises(RuntimeError) as err:
        enc(idx)  # the caller's own attempt over the whole chunk
    rows = resolve_failed_chunk(enc, idx, err.value)
    assert all(r is not None for r in rows)
    return rows, enc.attempts, texts


def test_halving_fails_exactly_the_faulting_row_wherever_it_sits():
    for size in (2, 3, 5, 8, 17, 64, 128, 512):
        for fault in {0, 1, size // 3, size // 2, size - 2, size - 1}:
            rows, _, texts = run(size, {fault})
            failed = [i for i, r in enumerate(rows) if isinstance(r, Exception)]
            assert failed == [fault], (size, fault)
            for i, r in enumerate(rows):
                if i != fault:
                    assert r == Poison.ids_of(texts[i]), (size, fault, i)


def test_halving_fails_exactly_n_rows_for_n_faults():
    cases = [(128, {0, 127}), (128, {3, 4}), (128, {7, 63, 64, 65}),
             (64, set(range(8))), (16, set(range(0, 16, 2))), (8, set(range(8)))]
    for size, faults in cases:
        rows, _, _ = run(size, faults)
        failed = {i for i, r in enumerate(rows) if isinstance(r, Exception)}
        assert failed == faults, (size, faults)


def test_halving_probes_a_chunk_instead_of_redoing_it():
    _, attempts, _ = run(128, {70})
    probes = attempts[1:]  # the first is the caller's own failed attempt
    assert len(probes) <= 2 * 8 and len(probes) < 128
    assert all(p < 128 for p in probes)
    assert 1 in probes  # the faulting row ends as a batch of one


def test_a_chunk_of_one_is_not_probed_again():
    rows, attempts, _ = run(1, {0})
    assert attempts == [1] and isinstance(rows[0], Exception)
    assert resolve_failed_chunk(lambda idx: [], [], RuntimeError("x")) == []
