"""toktier_amd -- MI355X-native fresh-encode path of TokTier.

Facade shape mirrors the reference (``src/toktier/facade/api.py:1620-1659``
``load``; ``Tokenizer.encode/encode_batch/explain`` ``:611-705``,
``:705-830``): ``toktier_amd.load(family).encode(text).ids`` gives token ids
bit-identical to a from-scratch HF ``tokenizers`` encode of ``text`` with
``add_special_tokens=False``. Every encode runs on the gfx950 engine
(``libtoktier_hip.so``); there is no CPU fallback. A text that fails the
device NFC quick check is normalized exactly with the certified engine's
NFC normalizer and encoded again on the device, which is what the
reference host does for every non-ASCII text (``gpu.rs:1446-1461``).
"""

from __future__ import annotations

import hashlib
import json
import threading
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

from . import bpe_tables, classes, families, standin
from ._ffi import (TK_ABI_VERSION, TK_E_NEEDS_NFC, TK_FLAG_NORMALIZED,
                   Engine, EngineError, TkConfig)

__all__ = ["load", "Tokenizer", "Encoding", "EngineError", "families"]
__version__ = "0.1.0"


@dataclass(frozen=True)
class Encoding:
    """Result of one encode: ``ids`` as a tuple of ints (reference shape);
    ``array`` holds the same ids as ``uint32``."""

    array: np.ndarray

    @property
    def ids(self) -> tuple[int, ...]:
        return tuple(self.array.tolist())

    def __len__(self) -> int:
        return int(self.array.size)


@dataclass
class _Counters:
    executions: int = 0
    renormalized: int = 0
    last_bytes: int = 0
    last_ids: int = 0
    last_stage_us: list = field(default_factory=list)


class Tokenizer:
    """A family's tokenizer bound to one GPU engine."""

    def __init__(self, family: str, tokenizer_json: str, device: int = 0,
                 expected_architecture: str | None = "gfx950"):
        self.family = families.family(family)
        self._json = tokenizer_json
        self.artifact_sha256 = hashlib.sha256(
            tokenizer_json.encode("utf-8")).hexdigest()
        self.tables = bpe_tables.load_tables(tokenizer_json)
        fam = self.family
        if bool(self.tables.ignore_merges) != fam.ignore_merges:
            raise ValueError(
                f"artifact ignore_merges={self.tables.ignore_merges} does not "
                f"match family {fam.name}")
        cfg = TkConfig(
            abi_version=TK_ABI_VERSION, device_ordinal=device,
            ruleset=fam.ruleset, digits_max=fam.digits_max,
            contractions=1, needs_nfc=int(fam.needs_nfc),
            ignore_merges=int(self.tables.ignore_merges),
            pair_count=self.tables.pair_count,
            vocab_count=self.tables.vocab_count,
            family=fam.name.encode(), artifact_sha256=self.artifact_sha256.encode(),
            expected_architecture=(expected_architecture.encode()
                                   if expected_architecture else None))
        nfc = classes.nfc_qc_table() if fam.needs_nfc else None
        self.engine = Engine(cfg, classes.class_table(), self.tables, nfc)
        self._lock = threading.Lock()
        self._counters = _Counters()
        self._nfc = None

    # -- exact normalization for texts that fail the device quick check
    def _normalize(self, text: str) -> str:
        if self._nfc is None:
            from tokenizers import normalizers
            self._nfc = normalizers.NFC()
        return self._nfc.normalize_str(text)

    def encode_bytes(self, data: bytes) -> np.ndarray:
        try:
            ids = self.engine.encode(data)
        except EngineError as err:
            if err.status != TK_E_NEEDS_NFC:
                raise
            data = self._normalize(data.decode("utf-8")).encode("utf-8")
            ids = self.engine.encode(data, TK_FLAG_NORMALIZED)
            with self._lock:
                self._counters.renormalized += 1
        with self._lock:
            c = self._counters
            c.executions += 1
            c.last_bytes = len(data)
            c.last_ids = int(ids.size)
        return ids

    def encode(self, text: str) -> Encoding:
        return Encoding(self.encode_bytes(text.encode("utf-8")))

    def encode_batch(self, texts: list[str]) -> list[Encoding]:
        """Row ``i`` equals ``encode(texts[i])``
        (``docs/contracts/api.md:106`` in the reference)."""
        docs = [t.encode("utf-8") for t in texts]
        ids, rows, status = self.engine.encode_batch(docs)
        out: list[Encoding | None] = [None] * len(docs)
        redo = []
        for d in range(len(docs)):
            if status[d] == 0:
                out[d] = Encoding(ids[int(rows[d]):int(rows[d + 1])].copy())
            elif status[d] == TK_E_NEEDS_NFC:
                redo.append(d)
            else:
                raise EngineError(int(status[d]), "tk_engine_encode_batch",
                                  f"row {d} failed")
        if redo:
            nd = [self._normalize(texts[d]).encode("utf-8") for d in redo]
            ids2, rows2, status2 = self.engine.encode_batch(nd, TK_FLAG_NORMALIZED)
            for k, d in enumerate(redo):
                if status2[k] != 0:
                    raise EngineError(int(status2[k]), "tk_engine_encode_batch",
                                      f"row {d} failed after normalization")
                out[d] = Encoding(ids2[int(rows2[k]):int(rows2[k + 1])].copy())
            with self._lock:
                self._counters.renormalized += len(redo)
        with self._lock:
            self._counters.executions += 1
        return out  # type: ignore[return-value]

    def explain(self) -> dict:
        """Route and execution report (reference ``explain()`` fields that
        apply to the fresh-encode path)."""
        from ._build import MANIFEST
        manifest = {}
        if MANIFEST.exists():
            manifest = json.loads(MANIFEST.read_text())
        c = self._counters
        return {
            "family": self.family.name,
            "artifact_sha256": self.artifact_sha256,
            "plan": ["gpu"],
            "route": "gpu",
            "kernel_delivery": self.engine.delivery,
            "architectures": [self.engine.architecture],
            "code_object_sha256": manifest.get("sha256"),
            "ruleset": self.family.ruleset_name,
            "digits_max": self.family.digits_max,
            "needs_nfc": self.family.needs_nfc,
            "ignore_merges": bool(self.tables.ignore_merges),
            "gpu_backend": {"loaded": True, "load_error": None},
            "execution_counts": {"gpu": c.executions},
            "fallback_counts": {},
            "nfc_renormalized": c.renormalized,
            "last_execution": {"bytes": c.last_bytes, "ids": c.last_ids},
        }

    def close(self) -> None:
        self.engine.close()


def load(family: str, tokenizer_json: str | Path | None = None,
         device: int = 0) -> Tokenizer:
    """Open ``family`` on GPU ``device``. Without ``tokenizer_json`` the
    committed stand-in artifact of the family is used."""
    if tokenizer_json is None:
        text = standin.load_artifact_json(family)
    else:
        p = Path(tokenizer_json)
        text = p.read_text(encoding="utf-8") if p.exists() else str(tokenizer_json)
    return Tokenizer(family, text, device=device)
