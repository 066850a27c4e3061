"""Export a ``tokenizer.json`` into the lookup tables the engine consumes.

The arrays and their encodings are the reference's kernel-input ABI
(``src/toktier/kernels/bpe_tables.py:1-30`` format notes, ``:284-390``
export, ``:435-501`` non-monotone guard), kept identical so that a caller
of the reference engine constructor can hand the same buffers to this one:

``pair_keys`` / ``pair_vals`` (uint64)
    open-addressed merge hash, ``key = id_left << 32 | id_right`` (empty
    ``~0``), ``val = rank << 32 | id_merged``; slot = ``splitmix64(key) &
    mask``, linear probing, size = smallest power of two ``>= 3 * n``.
``byte_id`` (int32[256])
    raw byte -> initial id through the byte-level alphabet, ``-1`` if the
    artifact has no id for that byte (the byte is then dropped before
    merging, as the engine does).
``vocab_keys`` / ``vocab_vals`` (uint64) + ``vocab_blob`` (uint8)
    whole-piece vocabulary hash for ``ignore_merges`` families:
    ``key = fnv1a64(raw bytes)``, ``val = blob_off << 30 | len << 20 | id``.
``unsafe_bits`` (uint32)
    bit ``r`` set iff merge rank ``r`` produces a token that a
    lower-ranked rule consumes (empty array for monotone tables).

The engine re-packs these into its own device layout at open time; this
module only produces the boundary format. No torch dependency.
"""

from __future__ import annotations

import hashlib
import json
import os
from dataclasses import dataclass
from pathlib import Path
from typing import Any

import numpy as np

__all__ = [
    "BpeTables", "export_tables", "bytes_to_unicode", "token_to_raw",
    "fnv1a64", "splitmix64", "build_hash", "unsafe_ranks", "load_tables",
]

MASK64 = 0xFFFFFFFFFFFFFFFF
EMPTY = MASK64
FNV_OFFSET = 0xCBF29CE484222325
FNV_PRIME = 0x100000001B3
TABLE_FORMAT = 1


def bytes_to_unicode() -> dict[int, str]:
    """GPT-2 byte-level alphabet: printable Latin-1 bytes map to themselves,
    the remaining 68 bytes to U+0100 upwards in byte order."""
    keep = set(range(0x21, 0x7F)) | set(range(0xA1, 0xAD)) | set(range(0xAE, 0x100))
    table: dict[int, str] = {}
    extra = 0
    for b in range(256):
        if b in keep:
            table[b] = chr(b)
        else:
            table[b] = chr(0x100 + extra)
            extra += 1
    return table


_B2U = bytes_to_unicode()
_U2B = {u: b for b, u in _B2U.items()}


def token_to_raw(token: str) -> bytes:
    """Byte-level token string -> the raw bytes it stands for."""
    return bytes(_U2B[ch] for ch in token)


def fnv1a64(data: bytes) -> int:
    h = FNV_OFFSET
    for b in data:
        h = ((h ^ b) * FNV_PRIME) & MASK64
    return h


def splitmix64(x: int) -> int:
    x = (x + 0x9E3779B97F4A7C15) & MASK64
    x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
    x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & MASK64
    return x ^ (x >> 31)


def _splitmix64_np(x: np.ndarray) -> np.ndarray:
    x = x.astype(np.uint64) + np.uint64(0x9E3779B97F4A7C15)
    x = (x ^ (x >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    x = (x ^ (x >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return x ^ (x >> np.uint64(31))


def build_hash(keys: list[int] | np.ndarray, values: list[int] | np.ndarray
               ) -> tuple[np.ndarray, np.ndarray]:
    """Open addressing, load <= 1/3, inserted in the given order."""
    keys = np.asarray(keys, dtype=np.uint64)
    values = np.asarray(values, dtype=np.uint64)
    size = 1
    while size < len(keys) * 3:
        size *= 2
    mask = size - 1
    slots = (_splitmix64_np(keys) & np.uint64(mask)).astype(np.int64).tolist()
    kl = keys.tolist()
    table_k = [EMPTY] * size
    table_v = [0] * size
    for key, val, slot in zip(kl, values.tolist(), slots):
        while table_k[slot] != EMPTY:
            if table_k[slot] == key:
                raise ValueError(f"duplicate key {key}")
            slot = (slot + 1) & mask
        table_k[slot] = key
        table_v[slot] = val
    return (np.array(table_k, dtype=np.uint64),
            np.array(table_v, dtype=np.uint64))


def _merge_pairs(merges: list[Any]) -> list[tuple[str, str]]:
    out = []
    for m in merges:
        if isinstance(m, list):
            a, b = m
        else:
            a, b = m.split(" ", 1)
        out.append((a, b))
    return out


def unsafe_ranks(merges: list[Any]) -> list[int]:
    """Ranks whose merged token is consumed by an earlier (lower) rank."""
    pairs = _merge_pairs(merges)
    first_use: dict[str, int] = {}
    for r, (a, b) in enumerate(pairs):
        first_use.setdefault(a, r)
        first_use.setdefault(b, r)
    return [r for r, (a, b) in enumerate(pairs)
            if first_use.get(a + b, r) < r]


@dataclass(frozen=True)
class BpeTables:
    pair_keys: np.ndarray
    pair_vals: np.ndarray
    byte_id: np.ndarray
    vocab_keys: np.ndarray
    vocab_vals: np.ndarray
    vocab_blob: np.ndarray
    unsafe_bits: np.ndarray
    ignore_merges: bool
    n_merges: int
    vocab_size: int
    source_sha256: str

    @property
    def pair_count(self) -> int:
        return int(self.pair_keys.size)

    @property
    def vocab_count(self) -> int:
        return int(self.vocab_keys.size)


def export_tables(tokenizer_json: str) -> BpeTables:
    """Build every boundary array from the text of a ``tokenizer.json``."""
    sha = hashlib.sha256(tokenizer_json.encode("utf-8")).hexdigest()
    model = json.loads(tokenizer_json)["model"]
    if model.get("type", "BPE") != "BPE":
        raise ValueError("only BPE models are supported")
    vocab: dict[str, int] = model["vocab"]
    pairs = _merge_pairs(model["merges"])
    ignore = bool(model.get("ignore_merges", False))
    if len(pairs) >= (1 << 27):
        raise ValueError("merge count exceeds the rank packing")

    pk = [(vocab[a] << 32) | vocab[b] for a, b in pairs]
    pv = [(r << 32) | vocab[a + b] for r, (a, b) in enumerate(pairs)]
    pair_keys, pair_vals = build_hash(pk, pv)

    byte_id = np.full(256, -1, dtype=np.int32)
    for b in range(256):
        tid = vocab.get(_B2U[b])
        if tid is not None:
            byte_id[b] = tid
    if ignore and (byte_id < 0).any():
        raise ValueError("ignore_merges needs full byte-alphabet coverage")

    referenced = {t for a, b in pairs for t in (a, b, a + b)}
    blob = bytearray()
    vk: list[int] = []
    vv: list[int] = []
    seen: dict[int, bytes] = {}
    for token, tid in vocab.items():
        try:
            raw = token_to_raw(token)
        except KeyError:
            if token in referenced:
                raise ValueError(
                    f"a merge references undecodable token {token!r}") from None
            continue
        if len(raw) >= 1024 or tid >= (1 << 20):
            raise ValueError("vocabulary entry exceeds the packing limits")
        key = fnv1a64(raw)
        if key in seen:
            if seen[key] != raw:
                raise ValueError("vocabulary hash collision")
            continue
        seen[key] = raw
        vk.append(key)
        vv.append((len(blob) << 30) | (len(raw) << 20) | tid)
        blob.extend(raw)
    vocab_keys, vocab_vals = build_hash(vk, vv)

    bits = np.zeros((len(pairs) + 31) // 32, dtype=np.uint32)
    flagged = unsafe_ranks(model["merges"])
    for r in flagged:
        bits[r >> 5] |= np.uint32(1 << (r & 31))
    if not flagged:
        bits = np.zeros(0, dtype=np.uint32)

    return BpeTables(
        pair_keys=pair_keys, pair_vals=pair_vals, byte_id=byte_id,
        vocab_keys=vocab_keys, vocab_vals=vocab_vals,
        vocab_blob=np.frombuffer(bytes(blob), dtype=np.uint8).copy(),
        unsafe_bits=bits, ignore_merges=ignore, n_merges=len(pairs),
        vocab_size=len(vocab), source_sha256=sha,
    )


def _cache_dir() -> Path:
    base = os.environ.get("XDG_CACHE_HOME") or os.path.join(
        os.path.expanduser("~"), ".cache")
    return Path(base) / "toktier_amd"


def load_tables(tokenizer_json: str) -> BpeTables:
    """``export_tables`` with an on-disk cache keyed by the artifact sha256."""
    sha = hashlib.sha256(tokenizer_json.encode("utf-8")).hexdigest()
    path = _cache_dir() / f"bpe_tables.{sha[:24]}.v{TABLE_FORMAT}.npz"
    if path.exists():
        try:
            with np.load(path, allow_pickle=False) as z:
                if str(z["source_sha256"]) == sha:
                    meta = z["meta"]
                    return BpeTables(
                        pair_keys=z["pair_keys"], pair_vals=z["pair_vals"],
                        byte_id=z["byte_id"], vocab_keys=z["vocab_keys"],
                        vocab_vals=z["vocab_vals"], vocab_blob=z["vocab_blob"],
                        unsafe_bits=z["unsafe_bits"],
                        ignore_merges=bool(meta[0]), n_merges=int(meta[1]),
                        vocab_size=int(meta[2]), source_sha256=sha)
        except (OSError, KeyError, ValueError):
            pass
    t = export_tables(tokenizer_json)
    try:
        path.parent.mkdir(parents=True, exist_ok=True)
        tmp = path.with_suffix(f".tmp{os.getpid()}.npz")
        np.savez(tmp, pair_keys=t.pair_keys, pair_vals=t.pair_vals,
                 byte_id=t.byte_id, vocab_keys=t.vocab_keys,
                 vocab_vals=t.vocab_vals, vocab_blob=t.vocab_blob,
                 unsafe_bits=t.unsafe_bits,
                 meta=np.array([int(t.ignore_merges), t.n_merges,
                                t.vocab_size], dtype=np.int64),
                 source_sha256=np.array(sha))
        os.replace(tmp, path)
    except OSError:
        pass
    return t
