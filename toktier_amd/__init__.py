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

Added tokens (the artifact's ``added_tokens``, e.g. ``<|im_end|>``) are
split out on the device, the way HF does it before normalization and
pretokenization; the reference instead routes every input that holds one
to its CPU engine (``frontend/added.py:503-555``, ``runtime.rs:641-662``).
"""

from __future__ import annotations

import hashlib
import json
import threading
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

from . import bpe_tables, classes, families, registry, standin
from ._ffi import (TK_ABI_VERSION, TK_ADDED_LSTRIP, TK_ADDED_NORMALIZED,
                   TK_ADDED_RSTRIP, TK_ADDED_SINGLE_WORD, TK_ADDED_SPECIAL,
                   TK_E_NEEDS_NFC, TK_FLAG_NO_ADDED, TK_FLAG_NORMALIZED,
                   Engine, EngineError, TkConfig)

__all__ = ["load", "Tokenizer", "Encoding", "EngineError", "BatchError",
           "resolve_failed_chunk", "families"]
__version__ = "0.1.0"


class BatchError(RuntimeError):
    """Rows of a batch that failed on their own: ``rows`` their indices,
    ``errors`` the ``EngineError`` of each."""

    def __init__(self, rows: list[int], errors: list):
        self.rows = rows
        self.errors = errors
        super().__init__(f"{len(rows)} row(s) failed: {rows[:8]}"
                         + (f"; first: {errors[0]}" if errors else ""))


def resolve_failed_chunk(encode_chunk, indices: list[int], error) -> list:
    """Rows of a chunk whose batched attempt failed as a whole, found by
    halving (``crates/toktier-routing-core/src/gpu.rs:1567-1639``): a half
    that succeeds is adopted whole and never split again, a half that still
    fails is divided, and a half of one document is that row's attempt, so
    its error is the row's. ``encode_chunk(indices)`` returns one entry per
    index or raises; ``error`` is the failure of the whole chunk. Returns
    the rows in order (an entry per index, the error for the rows that
    fail alone). A document's ids do not depend on the other documents of
    its batch, so the ids are those of encoding each document alone."""
    out: list = [None] * len(indices)
    if len(indices) <= 1:
        if indices:
            out[0] = error
        return out
    mid = len(indices) // 2
    pending = [(mid, len(indices)), (0, mid)]  # popped from the end: left first
    while pending:
        lo, hi = pending.pop()
        try:
            rows = encode_chunk(indices[lo:hi])
        except Exception as err:  # noqa: BLE001 -- the chunk's own failure
            if hi - lo <= 1:
                out[lo] = err
            else:
                m = lo + (hi - lo) // 2
                pending.append((m, hi))
                pending.append((lo, m))
            continue
        if len(rows) != hi - lo:
            bad = RuntimeError("batch returned the wrong row count")
            for k in range(lo, hi):
                out[k] = bad
            continue
        out[lo:hi] = rows
    return out


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
    last_literals: int = 0
    last_stats: dict = field(default_factory=dict)


@dataclass(frozen=True)
class AddedToken:
    """One ``added_tokens`` entry of a tokenizer.json."""

    content: str
    id: int
    flags: int  # TK_ADDED_* bits


def added_tokens(tokenizer_json: str) -> list[AddedToken]:
    """The artifact's added tokens in artifact order, with their flags and
    the ids HF tokenizers 0.22.2 gives them when it loads the file: the
    ``id`` field is not used; a content that is a model vocabulary entry
    keeps that entry's id, any other takes the vocabulary size, or one
    more than the largest id given so far when that is not below it; an
    empty or repeated content is skipped (the first one stands)."""
    spec = json.loads(tokenizer_json)
    vocab = (spec.get("model") or {}).get("vocab") or {}
    size = len(vocab)
    given: dict[str, int] = {}
    out = []
    for t in spec.get("added_tokens") or []:
        content = str(t["content"])
        if not content or content in given:
            continue
        if content in vocab:
            tid = int(vocab[content])
        else:
            top = max(given.values(), default=None)
            tid = size if top is None or top < size else top + 1
        given[content] = tid
        fl = ((TK_ADDED_SPECIAL if t.get("special") else 0)
              | (TK_ADDED_SINGLE_WORD if t.get("single_word") else 0)
              | (TK_ADDED_LSTRIP if t.get("lstrip") else 0)
              | (TK_ADDED_RSTRIP if t.get("rstrip") else 0)
              | (TK_ADDED_NORMALIZED if t.get("normalized") else 0))
        out.append(AddedToken(content, tid, fl))
    return out


class LiteralSplitter:
    """HF's added-token split on the host, for the texts the device sends
    back for exact normalization: scanning left to right, the first
    position where a literal matches takes the longest literal matching
    there, and the scan goes on after it (the same split the device does;
    the reference's scan / assemble, ``frontend/added.py:503-555``). A
    regex alternation tried longest first is exactly that: Python's
    alternation takes the first alternative that matches at the leftmost
    position where any does."""

    def __init__(self, tokens: list[AddedToken]):
        import re
        self._ids = {t.content: t.id for t in tokens}
        by_len = sorted(tokens, key=lambda t: -len(t.content))
        self._pat = (re.compile("|".join(re.escape(t.content) for t in by_len))
                     if tokens else None)

    def split(self, text: str) -> list[tuple[str, int | None]]:
        """Ordered ``(segment, None)`` / ``(literal, id)`` spans."""
        if self._pat is None:
            return [(text, None)] if text else []
        out: list[tuple[str, int | None]] = []
        at = 0
        for m in self._pat.finditer(text):
            if m.start() > at:
                out.append((text[at:m.start()], None))
            out.append((m.group(), self._ids[m.group()]))
            at = m.end()
        if at < len(text):
            out.append((text[at:], None))
        return out


#: token stride between span checkpoints of a session seed
#: (``crates/toktier-store-core/src/tail.rs:17-18``)
SPAN_CHECKPOINT_STRIDE = 4096


@dataclass(frozen=True)
class Seed:
    """A session seed: ``ids`` and, for every token index ``k * stride``,
    ``checkpoints[k] = (byte, anchor_byte, anchor_char)``: the token's first
    byte, the first byte of the character holding it, that character's
    index (``tail.rs:20-31``)."""

    ids: np.ndarray
    checkpoints: np.ndarray
    stride: int


class Tokenizer:
    """A family's tokenizer bound to one GPU engine."""

    def __init__(self, family: str, tokenizer_json: str, device: int = 0,
                 expected_architecture: str | None = "gfx950",
                 policy: str = registry.POLICY_EXPERIMENTAL):
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
            contractions=int(fam.ruleset != families.RULESET_DEEPSEEK
                             and fam.contractions),
            needs_nfc=int(fam.needs_nfc),
            ignore_merges=int(self.tables.ignore_merges),
            pair_count=self.tables.pair_count,
            vocab_count=self.tables.vocab_count,
            family=fam.name.encode(), artifact_sha256=self.artifact_sha256.encode(),
            expected_architecture=(expected_architecture.encode()
                                   if expected_architecture else None))
        nfc = classes.nfc_qc_table() if fam.needs_nfc else None
        self.engine = Engine(cfg, classes.table_named(families.class_table_name(fam)),
                             self.tables, nfc)
        self._lock = threading.Lock()
        self._counters = _Counters()
        self._nfc = None
        self.added_tokens = added_tokens(tokenizer_json)
        if self.added_tokens:
            try:
                self.engine.set_added(
                    [t.content.encode("utf-8") for t in self.added_tokens],
                    [t.id for t in self.added_tokens],
                    [t.flags for t in self.added_tokens])
            except EngineError:
                self.engine.close()
                raise
        self._splitter = None
        self.admission = self._admit(policy)
        if not self.admission.admitted:
            self.engine.close()
            codes = [r.code for r in self.admission.refusals]
            raise EngineError(
                -1, "route admission",
                f"the gfx950 route is not admitted under policy {policy!r}: "
                f"{codes}")

    def _admit(self, policy: str) -> "registry.Admission":
        """The gfx950 route's admission from the committed registry rows
        (reference planner checks, ``routing/plan.py:1-39``)."""
        from ._build import MANIFEST, verify
        try:
            reg = registry.load_registry()
        except (OSError, ValueError):
            reg = None
        build_key = None
        if MANIFEST.exists():
            build_key = json.loads(MANIFEST.read_text()).get("build_key")
        facts = registry.Facts(
            library_loaded=True, build_key=build_key, build_failed=False,
            architectures=(self.engine.architecture,),
            driver_version=self.engine.driver_version,
            build_mismatch=verify())
        return registry.admit(reg, self.artifact_sha256, facts, policy)

    # -- exact normalization for texts that fail the device quick check
    def _normalize(self, text: str) -> str:
        if self._nfc is None:
            from tokenizers import normalizers
            self._nfc = normalizers.NFC()
        return self._nfc.normalize_str(text)

    # -- texts that fail the device quick check: split at the literals,
    # normalize each segment exactly, encode the segments as one batch
    # (literal extraction off: they are the text between literals) and
    # splice the literal ids back in (frontend/added.py:544-555)
    def split_literals(self, text: str) -> list[tuple[str, int | None]]:
        if self._splitter is None:
            self._splitter = LiteralSplitter(self.added_tokens)
        return self._splitter.split(text)

    def _encode_normalized(self, text: str) -> np.ndarray:
        plan = self.split_literals(text)
        segs = [self._normalize(t).encode("utf-8") for t, i in plan if i is None]
        ids, rows, status = self.engine.encode_batch(
            segs, TK_FLAG_NORMALIZED | TK_FLAG_NO_ADDED)
        parts, k = [], 0
        for t, i in plan:
            if i is not None:
                parts.append(np.asarray([i], dtype=np.uint32))
                continue
            if status[k] != 0:
                raise EngineError(int(status[k]), "tk_engine_encode_batch",
                                  "segment failed after normalization")
            parts.append(ids[int(rows[k]):int(rows[k + 1])])
            k += 1
        with self._lock:
            self._counters.renormalized += 1
        return (np.concatenate(parts) if parts
                else np.zeros(0, dtype=np.uint32))

    def encode_bytes(self, data: bytes) -> np.ndarray:
        try:
            ids = self.engine.encode(data)
        except EngineError as err:
            if err.status != TK_E_NEEDS_NFC:
                raise
            ids = self._encode_normalized(data.decode("utf-8"))
        with self._lock:
            c = self._counters
            c.executions += 1
            c.last_bytes = len(data)
            c.last_ids = int(ids.size)
            c.last_literals = self.engine.last_literals()
            c.last_stats = self.engine.last_stats()
        return ids

    def encode(self, text: str) -> Encoding:
        return Encoding(self.encode_bytes(text.encode("utf-8")))

    def seed(self, text: str, stride: int = SPAN_CHECKPOINT_STRIDE) -> "Seed":
        """Ids plus the sparse span checkpoints the session store adopts
        (``crates/toktier-store-core/src/tail.rs:173-205``), computed on the
        device (``tk_engine_encode_seed_host``: host buffers in, engine-owned
        device buffers, host ids and checkpoints out). A text that fails the NFC
        quick check raises (``TK_E_NEEDS_NFC``): the store seeds the
        normalized text it holds."""
        data = text.encode("utf-8")
        ids, pts = self.engine.encode_seed_host(data, stride)
        with self._lock:
            c = self._counters
            c.executions += 1
            c.last_bytes = len(data)
            c.last_ids = int(ids.size)
            c.last_literals = self.engine.last_literals()
            c.last_stats = self.engine.last_stats()
        return Seed(ids, pts, stride)

    def encode_batch(self, texts: list[str], errors: str = "raise"
                     ) -> list[Encoding]:
        """Row ``i`` equals ``encode(texts[i])``
        (``docs/contracts/api.md:106`` in the reference). A row whose text
        fails on its own (invalid UTF-8) is that row's error; a batch that
        fails as a whole (a device guard, an injected fault) is resolved by
        halving (``resolve_failed_chunk``), so only the documents that fail
        alone end in an error and the others keep their ids. Rows that end
        in an error raise ``BatchError`` (``errors="raise"``, naming every
        failed row; no ids are returned), or stand as ``EngineError``
        entries in the returned list (``errors="return"``)."""
        docs = [t.encode("utf-8") for t in texts]
        out: list = [None] * len(docs)
        redo: list[int] = []

        def chunk(idx: list[int]) -> list:
            ids, rows, status = self.engine.encode_batch([docs[d] for d in idx])
            res = []
            for j, d in enumerate(idx):
                if status[j] == 0:
                    res.append(Encoding(ids[int(rows[j]):int(rows[j + 1])].copy()))
                elif status[j] == TK_E_NEEDS_NFC:
                    redo.append(d)
                    res.append(None)
                else:
                    res.append(EngineError(int(status[j]), "tk_engine_encode_batch",
                                           f"row {d} failed"))
            return res

        idx = list(range(len(docs)))
        try:
            rows = chunk(idx)
        except EngineError as err:
            rows = resolve_failed_chunk(chunk, idx, err)
        for d, r in zip(idx, rows):
            out[d] = r
        for d in redo:
            try:
                out[d] = Encoding(self._encode_normalized(texts[d]))
            except EngineError as err:
                out[d] = err
        with self._lock:
            self._counters.executions += 1
        failed = [d for d, r in enumerate(out) if isinstance(r, EngineError)]
        if failed and errors == "raise":
            raise BatchError(failed, [out[d] for d in failed])
        return out

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
            "admission": self.admission.as_dict(),
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
            "added_tokens": len(self.added_tokens),
            "added_token_frontend": "device" if self.added_tokens else None,
            "last_execution": {**c.last_stats,
                               "bytes": c.last_bytes, "ids": c.last_ids,
                               "added_literals": c.last_literals},
        }

    def close(self) -> None:
        self.engine.close()


def load(family: str, tokenizer_json: str | Path | None = None,
         device: int = 0, policy: str = registry.POLICY_EXPERIMENTAL
         ) -> Tokenizer:
    """Open ``family`` on GPU ``device``. Without ``tokenizer_json`` the
    committed stand-in artifact of the family is used. ``policy``:
    ``experimental`` (default) runs the gfx950 route past waivable
    refusals and reports them in ``explain()["admission"]``;
    ``certified`` refuses any route the registry has not certified for
    this artifact, device and build."""
    if tokenizer_json is None:
        text = standin.load_artifact_json(family)
    elif isinstance(tokenizer_json, str) and tokenizer_json.lstrip().startswith("{"):
        text = tokenizer_json  # the artifact's text itself
    else:
        p = Path(tokenizer_json)
        text = p.read_text(encoding="utf-8") if p.exists() else str(tokenizer_json)
    return Tokenizer(family, text, device=device, policy=policy)
