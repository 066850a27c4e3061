"""ctypes wrapper of the CPU restatement (``liboracle.so``).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` as the parity checker. The
product path (``toktier_amd``) never imports this module.
"""

from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"

E_UTF8, E_NOMEM, E_NEEDS_NFC, E_CAP = -1, -2, -3, -4


class _Tables(C.Structure):
    _fields_ = [
        ("cls", C.c_void_p), ("pair_keys", C.c_void_p),
        ("pair_vals", C.c_void_p), ("pair_count", C.c_uint64),
        ("byte_id", C.c_void_p), ("vocab_keys", C.c_void_p),
        ("vocab_vals", C.c_void_p), ("vocab_count", C.c_uint64),
        ("vocab_blob", C.c_void_p), ("nfc_qc", C.c_void_p),
        ("ruleset", C.c_int32), ("digits_max", C.c_int32),
        ("ignore_merges", C.c_int32), ("needs_nfc", C.c_int32),
        ("contractions", C.c_int32),
    ]


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = C.CDLL(str(LIB))
        L.tko_pretokenize.restype = C.c_int64
        L.tko_pretokenize.argtypes = [C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p]
        L.tko_bpe.restype = C.c_int64
        L.tko_bpe.argtypes = [C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p]
        L.tko_nfc_qc.restype = C.c_int
        L.tko_nfc_qc.argtypes = [C.c_void_p, C.c_void_p, C.c_int64]
        L.tko_encode.restype = C.c_int64
        L.tko_encode.argtypes = [C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p, C.c_int64]
        L.tko_encode_added.restype = C.c_int64
        L.tko_encode_added.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p,
                                       C.c_int64, C.c_void_p, C.c_int64]
        L.tko_utf8_decode.restype = C.c_int64
        L.tko_utf8_decode.argtypes = [C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p]
        _lib = L
    return _lib


class _Added(C.Structure):
    _fields_ = [("blob", C.c_void_p), ("offsets", C.c_void_p),
                ("ids", C.c_void_p), ("n", C.c_int64)]


class Oracle:
    """Sequential restatement bound to one family's tables."""

    def __init__(self, tables, cls: np.ndarray, nfc_qc: np.ndarray | None,
                 ruleset: int, digits_max: int, needs_nfc: bool,
                 contractions: bool = True):
        self._keep = [tables.pair_keys, tables.pair_vals, tables.byte_id,
                      tables.vocab_keys, tables.vocab_vals,
                      tables.vocab_blob, cls, nfc_qc]
        blob = tables.vocab_blob if tables.vocab_blob.size else np.zeros(1, np.uint8)
        self._keep.append(blob)
        self._t = _Tables(
            cls.ctypes.data, tables.pair_keys.ctypes.data,
            tables.pair_vals.ctypes.data, tables.pair_keys.size,
            tables.byte_id.ctypes.data, tables.vocab_keys.ctypes.data,
            tables.vocab_vals.ctypes.data, tables.vocab_keys.size,
            blob.ctypes.data,
            nfc_qc.ctypes.data if nfc_qc is not None else None,
            ruleset, digits_max, int(tables.ignore_merges), int(needs_nfc),
            int(contractions))
        self._lib = lib()
        self._added = None

    def set_added(self, contents: list[bytes], ids: list[int]) -> None:
        """Added-token literals split out before encoding (no flags)."""
        if not contents:
            self._added = None
            return
        blob = np.frombuffer(b"".join(contents), dtype=np.uint8).copy()
        offs = np.zeros(len(contents) + 1, dtype=np.uint64)
        offs[1:] = np.cumsum([len(c) for c in contents], dtype=np.uint64)
        idv = np.asarray(ids, dtype=np.uint32)
        self._added_keep = (blob, offs, idv)
        self._added = _Added(blob.ctypes.data, offs.ctypes.data,
                             idv.ctypes.data, len(contents))

    def pretokenize(self, data: bytes) -> list[int]:
        """Piece start byte offsets, followed by len(data)."""
        starts = np.zeros(len(data) + 1, dtype=np.int64)
        n = self._lib.tko_pretokenize(C.byref(self._t), data, len(data),
                                      starts.ctypes.data)
        if n < 0:
            raise ValueError(f"oracle pretokenize failed ({n})")
        return starts[: n + 1].tolist()

    def bpe(self, piece: bytes) -> list[int]:
        out = np.zeros(max(1, len(piece)), dtype=np.uint32)
        n = self._lib.tko_bpe(C.byref(self._t), piece, len(piece), out.ctypes.data)
        return out[:n].tolist()

    def nfc_qc(self, data: bytes) -> bool:
        r = self._lib.tko_nfc_qc(C.byref(self._t), data, len(data))
        if r < 0:
            raise ValueError("invalid UTF-8")
        return bool(r)

    def encode_bytes(self, data: bytes, normalized: bool = False,
                     literals: bool = True) -> np.ndarray | int:
        """ids as uint32, or a negative status (E_NEEDS_NFC, E_UTF8).
        ``normalized``: the text already went through the family's NFC, so
        the quick check is skipped (the engine's TK_FLAG_NORMALIZED).
        ``literals``: split out the added-token literals set by
        ``set_added`` (off: the text is one segment between literals, the
        engine's TK_FLAG_NO_ADDED)."""
        out = np.zeros(max(1, len(data)), dtype=np.uint32)
        t = self._t
        if normalized and t.needs_nfc:
            t = _Tables.from_buffer_copy(self._t)
            t.needs_nfc = 0
        if self._added is not None and literals:
            n = self._lib.tko_encode_added(C.byref(t), C.byref(self._added),
                                           data, len(data), out.ctypes.data,
                                           out.size)
        else:
            n = self._lib.tko_encode(C.byref(t), data, len(data),
                                     out.ctypes.data, out.size)
        if n < 0:
            return int(n)
        return out[:n]


def span_checkpoints(data: bytes, ids, token_len, stride: int) -> np.ndarray:
    """The session store's sparse span checkpoints of an encoding, restated
    from ``crates/toktier-store-core/src/tail.rs:173-205``
    (``build_span_checkpoints``): walking the ids with a byte cursor (the
    sum of the token byte lengths so far), at every token index that is a
    multiple of ``stride`` record (byte, first byte of the character holding
    it, that character's index). Raises unless the tokens close exactly
    over ``data``. ``token_len[id]`` is the id's byte length."""
    out = []
    byte = 0
    # characters before each byte offset: the lead bytes before it
    lead = (np.frombuffer(data, dtype=np.uint8) & 0xC0) != 0x80
    before = np.concatenate([[0], np.cumsum(lead)])
    for k, t in enumerate(ids):
        if k % stride == 0:
            a = byte
            while a > 0 and (data[a] & 0xC0) == 0x80:
                a -= 1
            out.append((byte, a, int(before[a])))
        n = int(token_len[int(t)])
        if n <= 0:
            raise ValueError(f"id {int(t)} has no byte length")
        byte += n
    if byte != len(data):
        raise ValueError(f"tokens close at byte {byte}, text has {len(data)}")
    return np.asarray(out, dtype=np.uint64).reshape(-1, 3)


def token_byte_lengths(tokenizer_json: str) -> np.ndarray:
    """Byte length of every id of a byte-level BPE artifact: its vocabulary
    string mapped back through the ByteLevel alphabet (printable bytes are
    themselves, the others shifted to U+0100 onward); added tokens are their
    UTF-8 contents."""
    import json
    spec = json.loads(tokenizer_json)
    vocab = spec["model"]["vocab"]
    added = spec.get("added_tokens") or []
    n = max([*vocab.values(), *(a["id"] for a in added)], default=-1) + 1
    out = np.zeros(n, dtype=np.int64)
    for tok, i in vocab.items():
        out[i] = len(tok)  # one alphabet character per byte
    for a in added:
        out[a["id"]] = len(a["content"].encode("utf-8"))
    return out
