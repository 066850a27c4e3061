"""ctypes binding of ``libtoktier_hip.so`` (the C-ABI in
``include/toktier_hip.h``).

Loading fails loudly: there is no CPU fallback behind this module.
"""

from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

from ._build import LIB

TK_ABI_VERSION = 1
TK_OK = 0
TK_E_INVALID_ARG = -1
TK_E_SHAPE = -2
TK_E_DEVICE = -3
TK_E_ARCH = -4
TK_E_UTF8 = -5
TK_E_NEEDS_NFC = -6
TK_E_CAPACITY = -7
TK_E_INTERNAL = -8
TK_E_UNSUPPORTED = -9
TK_RULESET_CL100K = 0
TK_RULESET_R50K = 1
TK_RULESET_LAGUNA = 2
TK_RULESET_DEEPSEEK = 3
TK_RULESET_O200K = 4
TK_RULESET_KIMI = 5
TK_FLAG_NORMALIZED = 1
TK_FLAG_NO_ADDED = 2
TK_NOALLOC_MAX_BYTES = 1 << 20
TK_OPT_COMPACT_PAIRS = 1
TK_OPT_REPAIR_WIDEN = 2
TK_OPT_TIMED_KERNEL = 3
TK_OPT_HOT_PAIRS = 4
# TK_KERNEL_* in the header's order: the kernels the timing modes time
KERNELS = ("k_pretok", "k_bpe_pack", "k_compact", "k_bpe_rows",
           "k_long_windows", "k_added")
# added-token flags (tokenizer.json "added_tokens" fields)
TK_ADDED_SPECIAL = 1
TK_ADDED_SINGLE_WORD = 2
TK_ADDED_LSTRIP = 4
TK_ADDED_RSTRIP = 8
TK_ADDED_NORMALIZED = 16

STATUS_NAMES = {
    TK_OK: "TK_OK", TK_E_INVALID_ARG: "TK_E_INVALID_ARG",
    TK_E_SHAPE: "TK_E_SHAPE", TK_E_DEVICE: "TK_E_DEVICE",
    TK_E_ARCH: "TK_E_ARCH", TK_E_UTF8: "TK_E_UTF8",
    TK_E_NEEDS_NFC: "TK_E_NEEDS_NFC", TK_E_CAPACITY: "TK_E_CAPACITY",
    TK_E_INTERNAL: "TK_E_INTERNAL", TK_E_UNSUPPORTED: "TK_E_UNSUPPORTED",
}

#: every entry point include/toktier_hip.h declares
SYMBOLS = (
    "tk_engine_preflight", "tk_engine_open", "tk_engine_close",
    "tk_engine_encode", "tk_engine_encode_batch", "tk_engine_encode_batch_docs",
    "tk_engine_encode_device",
    "tk_engine_encode_device_noalloc", "tk_engine_encode_seed",
    "tk_engine_encode_seed_host",
    "tk_engine_delivery", "tk_engine_architecture", "tk_engine_set_timing",
    "tk_engine_last_timing", "tk_engine_set_added",
    "tk_engine_last_literals", "tk_engine_last_stats", "tk_engine_set_option",
    "tk_engine_set_fault_marker",
    "tk_engine_driver_version", "tk_last_error",
)


class TkConfig(C.Structure):
    _fields_ = [
        ("abi_version", C.c_uint32), ("device_ordinal", C.c_int32),
        ("ruleset", C.c_int32), ("digits_max", C.c_int32),
        ("contractions", C.c_int32), ("needs_nfc", C.c_int32),
        ("ignore_merges", C.c_int32), ("pair_count", C.c_uint64),
        ("vocab_count", C.c_uint64), ("family", C.c_char_p),
        ("artifact_sha256", C.c_char_p),
        ("expected_architecture", C.c_char_p),
    ]


class EngineError(RuntimeError):
    """A failed engine call: ``status`` is the TK_* code."""

    def __init__(self, status: int, call: str, detail: str):
        self.status = status
        self.call = call
        self.detail = detail
        super().__init__(f"{call}: {STATUS_NAMES.get(status, status)}: {detail}")


_lib: C.CDLL | None = None


def lib(path: Path | None = None) -> C.CDLL:
    """Load the engine library (``RuntimeError`` if it was never built)."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else LIB
    if not p.exists():
        raise RuntimeError(
            f"{p} is missing: build it with toktier_amd._build.build() "
            "(hipcc --offload-arch=gfx950); there is no CPU fallback")
    L = C.CDLL(str(p))
    vp, sz = C.c_void_p, C.c_size_t
    L.tk_last_error.restype = C.c_char_p
    L.tk_last_error.argtypes = []
    L.tk_engine_preflight.restype = C.c_int
    L.tk_engine_preflight.argtypes = [C.POINTER(TkConfig)] + [vp, sz] * 7
    L.tk_engine_open.restype = C.c_int
    L.tk_engine_open.argtypes = ([C.POINTER(TkConfig)] + [vp, sz] * 9
                                 + [C.POINTER(vp)])
    L.tk_engine_close.restype = None
    L.tk_engine_close.argtypes = [vp]
    L.tk_engine_encode.restype = C.c_int
    L.tk_engine_encode.argtypes = [vp, vp, sz, C.c_uint32, vp, sz,
                                   C.POINTER(sz)]
    L.tk_engine_encode_batch.restype = C.c_int
    L.tk_engine_encode_batch.argtypes = [vp, vp, vp, sz, C.c_uint32, vp, sz,
                                         vp, vp]
    L.tk_engine_encode_batch_docs.restype = C.c_int
    L.tk_engine_encode_batch_docs.argtypes = [vp, vp, vp, sz, C.c_uint32, vp,
                                              sz, vp, vp]
    L.tk_engine_encode_device.restype = C.c_int
    L.tk_engine_encode_device.argtypes = [vp, vp, sz, C.c_uint32, vp, sz,
                                          C.POINTER(sz), vp]
    L.tk_engine_encode_device_noalloc.restype = C.c_int
    L.tk_engine_encode_device_noalloc.argtypes = [vp, vp, sz, C.c_uint32, vp,
                                                  sz, C.POINTER(sz), vp]
    L.tk_engine_encode_seed.restype = C.c_int
    L.tk_engine_encode_seed.argtypes = [vp, vp, sz, C.c_uint32, vp, sz,
                                        C.c_uint32, vp, sz, C.POINTER(sz),
                                        C.POINTER(sz), vp]
    L.tk_engine_encode_seed_host.restype = C.c_int
    L.tk_engine_encode_seed_host.argtypes = [vp, vp, sz, C.c_uint32, vp, sz,
                                             C.c_uint32, vp, sz,
                                             C.POINTER(C.c_size_t),
                                             C.POINTER(C.c_size_t)]
    L.tk_engine_delivery.restype = C.c_char_p
    L.tk_engine_delivery.argtypes = [vp]
    L.tk_engine_architecture.restype = C.c_char_p
    L.tk_engine_architecture.argtypes = [vp]
    L.tk_engine_set_timing.restype = C.c_int
    L.tk_engine_set_timing.argtypes = [vp, C.c_int]
    L.tk_engine_last_timing.restype = C.c_int
    L.tk_engine_last_timing.argtypes = [vp, C.POINTER(C.c_double), C.c_int]
    L.tk_engine_set_added.restype = C.c_int
    L.tk_engine_set_added.argtypes = [vp, sz, vp, vp, vp, vp]
    L.tk_engine_driver_version.restype = C.c_int
    L.tk_engine_driver_version.argtypes = [vp, C.POINTER(C.c_int)]
    L.tk_engine_last_literals.restype = C.c_int
    L.tk_engine_last_literals.argtypes = [vp, C.POINTER(C.c_uint64)]
    L.tk_engine_set_option.restype = C.c_int
    L.tk_engine_set_option.argtypes = [vp, C.c_int, C.c_int64]
    L.tk_engine_set_fault_marker.restype = C.c_int
    L.tk_engine_set_fault_marker.argtypes = [vp, vp, sz]
    L.tk_engine_last_stats.restype = C.c_int
    L.tk_engine_last_stats.argtypes = [vp, C.POINTER(C.c_uint64), C.c_int]
    if path is None:
        _lib = L
    return L


def check(status: int, call: str) -> None:
    if status != TK_OK:
        detail = (lib().tk_last_error() or b"").decode("utf-8", "replace")
        raise EngineError(status, call, detail)


def _ptr(a: np.ndarray | None) -> tuple[int | None, int]:
    if a is None:
        return None, 0
    a = np.ascontiguousarray(a)
    return a.ctypes.data, a.nbytes


class Engine:
    """One opened engine (a family's tables resident on one GPU)."""

    def __init__(self, cfg: TkConfig, class_table, tables, nfc_qc):
        self._L = lib()
        self._keep = (cfg, class_table, tables, nfc_qc)
        args = []
        blob = tables.vocab_blob if tables.vocab_blob.size else np.zeros(1, np.uint8)
        unsafe = tables.unsafe_bits if tables.unsafe_bits.size else np.zeros(0, np.uint32)
        self._keep = self._keep + (blob, unsafe)
        for arr in (class_table, tables.pair_keys, tables.pair_vals,
                    tables.byte_id, tables.vocab_keys, tables.vocab_vals,
                    blob, unsafe, nfc_qc):
            args.extend(_ptr(arr))
        handle = C.c_void_p()
        check(self._L.tk_engine_open(C.byref(cfg), *args, C.byref(handle)),
              "tk_engine_open")
        self._h = handle
        self.device = int(cfg.device_ordinal)

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._L.tk_engine_close(self._h)
            self._h = None

    def __del__(self) -> None:  # pragma: no cover - interpreter teardown
        try:
            self.close()
        except Exception:
            pass

    @property
    def delivery(self) -> str:
        return self._L.tk_engine_delivery(self._h).decode()

    @property
    def architecture(self) -> str:
        return self._L.tk_engine_architecture(self._h).decode()

    def encode(self, data: bytes, flags: int = 0,
               out: np.ndarray | None = None) -> np.ndarray:
        """Host bytes in, host ids out. ``out``: a reusable uint32 buffer of
        at least ``len(data)`` entries (the result is a view of it)."""
        if (out is None or out.dtype != np.uint32 or out.ndim != 1
                or not out.flags.c_contiguous or out.size < max(1, len(data))):
            out = np.empty(max(1, len(data)), dtype=np.uint32)
        n = C.c_size_t()
        st = self._L.tk_engine_encode(self._h, data, len(data), flags,
                                      out.ctypes.data, out.size, C.byref(n))
        check(st, "tk_engine_encode")
        return out[: n.value]

    def encode_batch(self, docs: list[bytes], flags: int = 0,
                     out: np.ndarray | None = None
                     ) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
        """Documents in their own buffers (tk_engine_encode_batch_docs: the
        engine gathers them); returns (ids, row offsets, row status).
        ``out``: a reusable uint32 buffer of at least the documents' total
        bytes (``ids`` is then a view of it)."""
        lens = np.fromiter((len(d) for d in docs), dtype=np.uint64, count=len(docs))
        ptrs = (C.c_char_p * max(1, len(docs)))(*docs)
        nb = int(lens.sum())
        if (out is None or out.dtype != np.uint32 or out.ndim != 1
                or not out.flags.c_contiguous or out.size < max(1, nb)):
            out = np.empty(max(1, nb), dtype=np.uint32)
        rows = np.zeros(len(docs) + 1, dtype=np.uint64)
        status = np.zeros(max(1, len(docs)), dtype=np.int32)
        st = self._L.tk_engine_encode_batch_docs(
            self._h, ptrs, lens.ctypes.data, len(docs), flags,
            out.ctypes.data, out.size, rows.ctypes.data, status.ctypes.data)
        check(st, "tk_engine_encode_batch_docs")
        return out, rows, status[: len(docs)]

    def encode_batch_joined(self, joined: bytes, doc_offsets: np.ndarray,
                            flags: int = 0
                            ) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
        """The same batch as one buffer of concatenated documents and their
        offsets (tk_engine_encode_batch)."""
        offs = np.ascontiguousarray(doc_offsets, dtype=np.uint64)
        n = offs.size - 1
        ids = np.empty(max(1, len(joined)), dtype=np.uint32)
        rows = np.zeros(n + 1, dtype=np.uint64)
        status = np.zeros(max(1, n), dtype=np.int32)
        st = self._L.tk_engine_encode_batch(
            self._h, joined, offs.ctypes.data, n, flags,
            ids.ctypes.data, ids.size, rows.ctypes.data, status.ctypes.data)
        check(st, "tk_engine_encode_batch")
        return ids, rows, status[:n]

    def encode_device(self, d_text: int, nbytes: int, d_ids: int,
                      ids_cap: int, flags: int = 0, stream: int | None = None
                      ) -> int:
        n = C.c_size_t()
        st = self._L.tk_engine_encode_device(self._h, d_text, nbytes, flags,
                                             d_ids, ids_cap, C.byref(n),
                                             stream)
        check(st, "tk_engine_encode_device")
        return n.value

    def encode_device_noalloc(self, d_text: int, nbytes: int, d_ids: int,
                              ids_cap: int, flags: int = 0,
                              stream: int | None = None) -> int:
        """``encode_device`` with the workspace in the library's static
        scratch array (no device allocation); inputs of at most
        ``TK_NOALLOC_MAX_BYTES``."""
        n = C.c_size_t()
        st = self._L.tk_engine_encode_device_noalloc(
            self._h, d_text, nbytes, flags, d_ids, ids_cap, C.byref(n), stream)
        check(st, "tk_engine_encode_device_noalloc")
        return n.value

    def encode_seed(self, d_text: int, nbytes: int, d_ids: int, ids_cap: int,
                    stride: int, d_points: int, points_cap: int,
                    flags: int = 0, stream: int | None = None
                    ) -> tuple[int, int]:
        """Device-resident encode plus span checkpoints (three uint64 per
        checkpoint at d_points); returns (n_ids, n_points)."""
        n = C.c_size_t()
        m = C.c_size_t()
        st = self._L.tk_engine_encode_seed(self._h, d_text, nbytes, flags,
                                           d_ids, ids_cap, stride, d_points,
                                           points_cap, C.byref(n), C.byref(m),
                                           stream)
        check(st, "tk_engine_encode_seed")
        return n.value, m.value

    def encode_seed_host(self, data: bytes, stride: int, flags: int = 0
                         ) -> tuple[np.ndarray, np.ndarray]:
        """Host-buffer encode plus span checkpoints: (ids uint32, points
        uint64 of shape (n, 3))."""
        nb = len(data)
        ids = np.empty(max(1, nb), dtype=np.uint32)
        cap = max(1, nb // max(1, stride) + 1)
        pts = np.empty(3 * cap, dtype=np.uint64)
        n = C.c_size_t()
        m = C.c_size_t()
        st = self._L.tk_engine_encode_seed_host(self._h, data, nb, flags,
                                                ids.ctypes.data, ids.size, stride,
                                                pts.ctypes.data, cap,
                                                C.byref(n), C.byref(m))
        check(st, "tk_engine_encode_seed_host")
        return ids[:n.value].copy(), pts[:3 * m.value].reshape(m.value, 3).copy()

    def set_added(self, contents: list[bytes], ids: list[int],
                  flags: list[int]) -> None:
        """Install the artifact's added tokens (``TK_ADDED_*`` flags); an
        empty list removes them."""
        n = len(contents)
        blob = np.frombuffer(b"".join(contents) or b"\0", dtype=np.uint8).copy()
        offs = np.zeros(n + 1, dtype=np.uint64)
        if n:
            offs[1:] = np.cumsum([len(c) for c in contents], dtype=np.uint64)
        idv = np.asarray(ids if n else [0], dtype=np.uint32)
        fl = np.asarray(flags if n else [0], dtype=np.uint8)
        check(self._L.tk_engine_set_added(self._h, n, blob.ctypes.data,
                                          offs.ctypes.data, idv.ctypes.data,
                                          fl.ctypes.data),
              "tk_engine_set_added")

    @property
    def driver_version(self) -> int:
        v = C.c_int()
        check(self._L.tk_engine_driver_version(self._h, C.byref(v)),
              "tk_engine_driver_version")
        return int(v.value)

    def last_literals(self) -> int:
        n = C.c_uint64()
        check(self._L.tk_engine_last_literals(self._h, C.byref(n)),
              "tk_engine_last_literals")
        return int(n.value)

    def set_option(self, option: int, value: int) -> None:
        """``TK_OPT_COMPACT_PAIRS``: 1 probe the compact pair table (the
        default when the artifact fits it), 0 the boundary-format table.
        ``TK_OPT_REPAIR_WIDEN``: the first certification repair pass that
        also drops cuts around each failed one (default 4); 0 merges every
        piece over 512 bytes whole, with no cut. ``TK_OPT_TIMED_KERNEL``:
        the kernel timing mode 2 times (an index into ``KERNELS``)."""
        check(self._L.tk_engine_set_option(self._h, int(option), int(value)),
              "tk_engine_set_option")

    def set_fault_marker(self, marker: bytes) -> None:
        """Test-only: while set, a host-buffer call whose input holds
        ``marker`` fails as a whole (``TK_E_INTERNAL``) after its pipeline
        ran, writing no ids; ``b""`` clears it."""
        check(self._L.tk_engine_set_fault_marker(self._h, marker or None, len(marker)),
              "tk_engine_set_fault_marker")

    def last_stats(self) -> dict[str, int]:
        """Facts of the last encode: literals extracted, pieces over 64
        and over 512 bytes, certification repair passes."""
        buf = (C.c_uint64 * 4)()
        k = self._L.tk_engine_last_stats(self._h, buf, 4)
        if k < 0:
            check(k, "tk_engine_last_stats")
        names = ("literals", "long_pieces", "big_pieces", "repair_passes")
        return {n: int(buf[i]) for i, n in enumerate(names[:k])}

    def set_timing(self, mode: int) -> None:
        """0 off, 1 (or True) every stage and every kernel, 2 one kernel
        only (``TK_OPT_TIMED_KERNEL``; default the packed merge)."""
        check(self._L.tk_engine_set_timing(self._h, int(mode)),
              "tk_engine_set_timing")

    def last_timing(self) -> list[float]:
        """Device stage times [0..4] (timing modes 1 / 2), the host wall
        times [5..7] of the last host-to-host encode (bytes in, pipeline,
        ids out), and (mode 1) each kernel's own duration [8 + k] for k in
        ``KERNELS``, microseconds."""
        buf = (C.c_double * (8 + len(KERNELS)))()
        k = self._L.tk_engine_last_timing(self._h, buf, len(buf))
        return list(buf[:k])
