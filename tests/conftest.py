"""Shared fixtures. GPU tests carry ``@pytest.mark.gpu``; everything else
runs on the CPU (the oracle, the table export, the host logic and the
C-ABI symbol surface)."""

from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

FAMILY_NAMES = ("qwen3_8b", "llama_3_1_8b", "gpt2")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long-running CPU test")


def _gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


class FamilyKit:
    """Everything a parity test needs for one family."""

    def __init__(self, name: str):
        from toktier_amd import bpe_tables, classes, families, standin
        from oracle.oracle import Oracle

        self.name = name
        self.family = families.family(name)
        self.json = standin.load_artifact_json(name)
        self.tables = bpe_tables.load_tables(self.json)
        self.oracle = Oracle(self.tables, classes.class_table(),
                             classes.nfc_qc_table(), self.family.ruleset,
                             self.family.digits_max, self.family.needs_nfc)
        # the artifact's added-token literals, split out as HF does
        import toktier_amd
        self.added = toktier_amd.added_tokens(self.json)
        self.oracle.set_added([t.content.encode() for t in self.added],
                              [t.id for t in self.added])
        self._hf = None

    @property
    def hf(self):
        if self._hf is None:
            from tokenizers import Tokenizer
            self._hf = Tokenizer.from_str(self.json)
        return self._hf

    def hf_ids(self, text: str) -> list[int]:
        return self.hf.encode(text, add_special_tokens=False).ids

    def expected(self, text: str):
        """The oracle's ids for ``text``; when a segment fails the NFC
        quick check, the text is split at its literals, each segment is
        normalized by the certified engine's NFC and encoded alone, and the
        literal ids are spliced back in (what the facade does)."""
        got = self.oracle.encode_bytes(text.encode("utf-8"))
        if not (isinstance(got, int) and self.family.needs_nfc):
            return got
        import numpy as np
        from tokenizers import normalizers
        from toktier_amd import LiteralSplitter
        nfc = normalizers.NFC()
        parts = []
        for seg, lit in LiteralSplitter(self.added).split(text):
            if lit is not None:
                parts.append(np.asarray([lit], dtype=np.uint32))
                continue
            ids = self.oracle.encode_bytes(
                nfc.normalize_str(seg).encode("utf-8"), normalized=True,
                literals=False)
            if isinstance(ids, int):
                return ids
            parts.append(ids)
        return np.concatenate(parts) if parts else np.zeros(0, np.uint32)


_KITS: dict[str, FamilyKit] = {}


def kit(name: str) -> FamilyKit:
    if name not in _KITS:
        _KITS[name] = FamilyKit(name)
    return _KITS[name]


@pytest.fixture(params=FAMILY_NAMES)
def family_kit(request) -> FamilyKit:
    return kit(request.param)


@pytest.fixture(scope="session", autouse=True)
def _oracle_built():
    from oracle import oracle
    if not oracle.LIB.exists():
        oracle.build()
