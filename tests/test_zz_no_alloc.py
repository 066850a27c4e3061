"""The allocation-free entry (``tk_engine_encode_device_noalloc``) against
``tk_engine_encode_device``, through the C-ABI: the same ids, bit for bit,
on consecutive calls (the second smaller, so stale scratch contents from
the first would show), interleaved with the engine's own workspace and
with a second engine on the same device sharing the scratch array; inputs
over the limit are refused before anything runs."""

from __future__ import annotations

import numpy as np
import pytest

from conftest import kit

pytestmark = pytest.mark.gpu


def _text(js: str, n_chars: int, sample: int, long_run: bool) -> bytes:
    from toktier_amd import workloads
    t = workloads.config2(js, n_chars=n_chars, sample=sample)
    if long_run:
        # a 3,000-byte letter run (the cut / segment / certify path) and
        # chat markers (added-token literals) inside the request
        mid = len(t) // 2
        t = (t[:mid] + " " + "abcdefgh" * 375 + " <|im_start|>user\n" +
             t[mid:] + "<|im_end|>")
    return t.encode("utf-8")


def _dev(data: bytes):
    import torch
    d = torch.frombuffer(bytearray(data), dtype=torch.uint8).to("cuda:0")
    ids = torch.empty(len(data) + 1, dtype=torch.int32, device="cuda:0")
    return d, ids


def _run(eng, data: bytes, noalloc: bool) -> np.ndarray:
    d, ids = _dev(data)
    f = eng.encode_device_noalloc if noalloc else eng.encode_device
    n = f(d.data_ptr(), len(data), ids.data_ptr(), ids.numel())
    return ids[:n].cpu().numpy().view(np.uint32).copy()


def test_noalloc_matches_encode_device_on_consecutive_calls():
    import toktier_amd
    from toktier_amd._ffi import TK_NOALLOC_MAX_BYTES
    k = kit("qwen3_8b")
    tok = toktier_amd.load("qwen3_8b")
    try:
        big = _text(k.json, 1_000_000, 7, True)
        while len(big) > TK_NOALLOC_MAX_BYTES:
            big = big[: len(big) - 4096]
            while big and (big[-1] & 0xC0) == 0x80:
                big = big[:-1]
            big = big[:-1]
        small = _text(k.json, 90_000, 8, False)
        for data in (big, small):
            print(f"noalloc qwen3_8b: {len(data)} bytes", flush=True)
            got = _run(tok.engine, data, True)
            want = _run(tok.engine, data, False)
            assert np.array_equal(got, want), len(data)
            orc = k.expected(data.decode("utf-8"))
            assert not isinstance(orc, int)
            assert np.array_equal(got, orc), len(data)
        # the engine's own workspace is untouched by the scratch calls
        again = _run(tok.engine, small, False)
        assert np.array_equal(again, _run(tok.engine, small, True))
    finally:
        tok.close()


def test_noalloc_shared_by_two_engines_and_limits():
    import toktier_amd
    from toktier_amd._ffi import EngineError, TK_E_CAPACITY, TK_NOALLOC_MAX_BYTES
    a = toktier_amd.load("llama_3_1_8b")
    b = toktier_amd.load("deepseek_v3")
    try:
        ka, kb = kit("llama_3_1_8b"), kit("deepseek_v3")
        ta = _text(ka.json, 200_000, 9, True)
        tb = _text(kb.json, 60_000, 10, False)
        for eng, kk, data in ((a, ka, ta), (b, kb, tb), (a, ka, tb), (b, kb, ta)):
            print(f"noalloc {kk.name}: {len(data)} bytes", flush=True)
            got = _run(eng.engine, data, True)
            assert np.array_equal(got, _run(eng.engine, data, False))
            orc = kk.expected(data.decode("utf-8"))
            assert np.array_equal(got, orc)
        # one byte over the limit: refused before anything runs
        over = b"a" * (TK_NOALLOC_MAX_BYTES + 1)
        d, ids = _dev(over)
        with pytest.raises(EngineError) as err:
            a.engine.encode_device_noalloc(d.data_ptr(), len(over),
                                           ids.data_ptr(), ids.numel())
        assert err.value.status == TK_E_CAPACITY
        assert "limit" in err.value.detail
        # empty input: no ids
        assert a.engine.encode_device_noalloc(d.data_ptr(), 0, ids.data_ptr(),
                                              ids.numel()) == 0
    finally:
        a.close()
        b.close()


def test_noalloc_refuses_a_capturing_stream():
    """The entry waits for the id count, which a stream under HIP graph
    capture cannot do: it returns TK_E_INVALID_ARG and records nothing (the
    capture ends with an empty graph), and the engine works after it."""
    import torch
    import toktier_amd
    from toktier_amd._ffi import EngineError, TK_E_INVALID_ARG
    k = kit("qwen3_8b")
    tok = toktier_amd.load("qwen3_8b")
    try:
        data = _text(k.json, 20_000, 11, False)
        d, ids = _dev(data)
        torch.cuda.synchronize()
        s = torch.cuda.Stream()
        g = torch.cuda.CUDAGraph()
        err = None
        with torch.cuda.graph(g, stream=s, capture_error_mode="relaxed"):
            try:
                tok.engine.encode_device_noalloc(d.data_ptr(), len(data),
                                                 ids.data_ptr(), ids.numel(),
                                                 stream=s.cuda_stream)
            except EngineError as x:
                err = x
        assert err is not None and err.status == TK_E_INVALID_ARG
        assert "captur" in err.detail
        got = _run(tok.engine, data, True)
        assert np.array_equal(got, k.expected(data.decode("utf-8")))
    finally:
        tok.close()
