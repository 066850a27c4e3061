"""The host-buffer routes of the host-to-host entries, against the CPU
oracle bit for bit: pageable and page-locked request bytes; page-locked ids
buffers, which the compaction kernel writes straight into; pageable ones,
filled from the pinned staging by the copy threads; a misaligned
page-locked buffer, which takes the staged route; and a capacity failure
into a page-locked buffer, which must not write past ids_cap."""

from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from conftest import kit
from toktier_amd import _ffi

pytestmark = pytest.mark.gpu

SENTINEL = 0xA5A5A5A5


@pytest.fixture(scope="module")
def qwen():
    import toktier_amd
    return kit("qwen3_8b"), toktier_amd.load("qwen3_8b")


def _pinned(n: int, dtype):
    import torch
    t = torch.empty(n, dtype=dtype, pin_memory=True)
    assert t.is_pinned()
    return t


def _raw_encode(E, text_ptr: int, nbytes: int, ids_ptr: int, cap: int):
    n = C.c_size_t()
    st = E._L.tk_engine_encode(E._h, C.c_void_p(text_ptr), nbytes, 0,
                               C.c_void_p(ids_ptr), cap, C.byref(n))
    return st, n.value


def _texts(k):
    from toktier_amd import workloads
    # below and above the single-thread copy size (256 KiB), and one of a
    # few MiB (many chunks for the copy threads)
    return [workloads.config2(k.json, n_chars=n, sample=9 + i)
            for i, n in enumerate((3_000, 400_000, 2_500_000))]


def test_pageable_and_pinned_ids_buffers(qwen):
    import torch
    k, t = qwen
    E = t.engine
    texts = [s.encode() for s in _texts(k)]
    cap = max(len(b) for b in texts) + 1
    pinned = _pinned(cap, torch.int32).numpy().view(np.uint32)
    pageable = np.zeros(cap, dtype=np.uint32)
    # largest first, so the second and third calls reuse a dirtier buffer
    for b in sorted(texts, key=len, reverse=True):
        want = k.oracle.encode_bytes(b)
        for out in (pinned, pageable):
            got = E.encode(b, out=out)
            assert np.array_equal(got, want), (len(b), out is pinned)


def test_pinned_request_bytes(qwen):
    import torch
    k, t = qwen
    E = t.engine
    for s in _texts(k):
        b = s.encode()
        src = _pinned(len(b), torch.uint8)
        src.numpy()[:] = np.frombuffer(b, dtype=np.uint8)
        for out in (np.zeros(len(b), dtype=np.uint32),
                    _pinned(len(b), torch.int32).numpy().view(np.uint32)):
            st, n = _raw_encode(E, src.data_ptr(), len(b), out.ctypes.data, out.size)
            assert st == 0, E._L.tk_last_error()
            assert np.array_equal(out[:n], k.oracle.encode_bytes(b)), len(b)


def test_capacity_failure_keeps_past_cap_untouched(qwen):
    import torch
    k, t = qwen
    E = t.engine
    b = _texts(k)[2].encode()
    want = k.oracle.encode_bytes(b)
    guard = 1 << 16
    buf = _pinned(want.size + guard, torch.int32).numpy().view(np.uint32)
    for cap in (want.size // 2, want.size - 1):
        buf[:] = SENTINEL
        st, n = _raw_encode(E, C.cast(C.c_char_p(b), C.c_void_p).value, len(b),
                            buf.ctypes.data, cap)
        assert st == _ffi.TK_E_CAPACITY and n == 0
        assert np.all(buf[cap:] == SENTINEL), cap
    # the exact capacity is enough
    buf[:] = SENTINEL
    st, n = _raw_encode(E, C.cast(C.c_char_p(b), C.c_void_p).value, len(b),
                        buf.ctypes.data, want.size)
    assert st == 0 and n == want.size
    assert np.array_equal(buf[:n], want)
    assert np.all(buf[n:] == SENTINEL)


def test_misaligned_pinned_ids_buffer_is_staged(qwen):
    import torch
    k, t = qwen
    E = t.engine
    b = _texts(k)[1].encode()
    want = k.oracle.encode_bytes(b)
    raw = _pinned(4 * (len(b) + 2), torch.uint8)
    ptr = raw.data_ptr() + 2
    st, n = _raw_encode(E, C.cast(C.c_char_p(b), C.c_void_p).value, len(b), ptr,
                        len(b) + 1)
    assert st == 0, E._L.tk_last_error()
    got = np.frombuffer((C.c_uint8 * (4 * n)).from_address(ptr), dtype=np.uint32)
    assert np.array_equal(got, want)


def test_batch_into_pinned_ids_with_a_failed_row(qwen):
    import torch
    k, t = qwen
    E = t.engine
    base = _texts(k)[1]
    docs = [base[i * 9000:(i + 1) * 9000].encode() for i in range(30)]
    docs[7] = docs[7][:100] + b"\xff\xfe" + docs[7][100:]  # not UTF-8
    offs = np.zeros(len(docs) + 1, dtype=np.uint64)
    offs[1:] = np.cumsum([len(d) for d in docs])
    joined = b"".join(docs)
    ids = _pinned(len(joined) + 1, torch.int32).numpy().view(np.uint32)
    rows = np.zeros(len(docs) + 1, dtype=np.uint64)
    status = np.zeros(len(docs), dtype=np.int32)
    st = E._L.tk_engine_encode_batch(
        E._h, joined, offs.ctypes.data, len(docs), 0, ids.ctypes.data, ids.size,
        rows.ctypes.data, status.ctypes.data)
    assert st == 0, E._L.tk_last_error()
    for d, doc in enumerate(docs):
        if d == 7:
            assert status[d] == _ffi.TK_E_UTF8 and rows[d] == rows[d + 1]
            continue
        assert status[d] == 0
        assert np.array_equal(ids[rows[d]:rows[d + 1]], k.oracle.encode_bytes(doc)), d


def test_batch_of_separate_documents_equals_the_joined_batch(qwen):
    """tk_engine_encode_batch_docs (each document in its own buffer, gathered
    into the pinned staging by the engine) against tk_engine_encode_batch on
    the same documents joined: empty documents at the start, inside and at
    the end, a document that is not UTF-8, a batch the calling thread
    gathers alone (under 256 KiB) and one spread over the copy threads
    (ragged documents across many 64 KiB claims), ids into a fresh buffer
    and into a reused page-locked one; every good row against the oracle."""
    import torch
    k, t = qwen
    E = t.engine
    base = _texts(k)[2]
    small = [b"", base[:300].encode(), b"", base[300:2900].encode(), b""]
    big = [base[7000 * i:7000 * (i + 1) + 13 * (i % 5)].encode() for i in range(60)]
    big[3] = b""
    big[11] = big[11][:50] + b"\xff" + big[11][50:]  # not UTF-8
    big.append(b"")
    pinned = _pinned(sum(map(len, big)) + 1, torch.int32).numpy().view(np.uint32)
    for docs in (small, big):
        offs = np.zeros(len(docs) + 1, dtype=np.uint64)
        offs[1:] = np.cumsum([len(d) for d in docs])
        want_ids, want_rows, want_status = E.encode_batch_joined(b"".join(docs), offs)
        for out in (None, pinned):
            ids, rows, status = E.encode_batch(docs, out=out)
            assert np.array_equal(rows, want_rows)
            assert np.array_equal(status, want_status)
            assert np.array_equal(ids[:int(rows[-1])], want_ids[:int(want_rows[-1])])
        for d, doc in enumerate(docs):
            if docs is big and d == 11:
                assert status[d] == _ffi.TK_E_UTF8 and rows[d] == rows[d + 1]
                continue
            assert status[d] == 0
            assert np.array_equal(ids[int(rows[d]):int(rows[d + 1])],
                                  k.oracle.encode_bytes(doc)), d
