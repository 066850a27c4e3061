"""GPU: the session seed (``tk_engine_encode_seed``) against the oracle:
ids bit-identical, checkpoints equal to the store's restated
construction over the oracle's ids (``tail.rs:173-205``)."""

from __future__ import annotations

import numpy as np
import pytest

from conftest import kit

pytestmark = pytest.mark.gpu

_TOKS: dict = {}


def tok(name: str):
    if name not in _TOKS:
        import toktier_amd
        _TOKS[name] = toktier_amd.load(name)
    return _TOKS[name]


def _lens(k):
    from oracle.oracle import token_byte_lengths
    lens = token_byte_lengths(k.json)
    for t in k.added:
        lens[t.id] = len(t.content.encode("utf-8"))
    return lens


def _check(name, text, stride):
    from oracle.oracle import span_checkpoints
    k, t = kit(name), tok(name)
    data = text.encode("utf-8")
    want = k.oracle.encode_bytes(data)
    assert not isinstance(want, int)
    s = t.seed(text, stride=stride)
    assert np.array_equal(s.ids, want), (name, stride)
    pts = span_checkpoints(data, want, _lens(k), stride)
    assert s.checkpoints.shape == pts.shape, (name, stride)
    assert np.array_equal(s.checkpoints, pts), (name, stride)


@pytest.mark.parametrize("stride", [4096, 64, 1])
def test_seed_of_mixed_text(stride):
    from toktier_amd import workloads
    k = kit("qwen3_8b")
    _check("qwen3_8b", workloads.config2(k.json, n_chars=200_000), stride)


@pytest.mark.family("deepseek_v3")
def test_seed_of_cjk_text_through_deepseek():
    from toktier_amd import workloads
    k = kit("deepseek_v3")
    text = workloads.config5(k.json, n_chars=300_000, n_runs=2, run_chars=20_000)
    _check("deepseek_v3", text, 1000)


@pytest.mark.parametrize("name", ["qwen3_8b", "llama_3_1_8b"])
def test_seed_of_chat_turns(name):
    from toktier_amd import workloads
    k = kit(name)
    _check(name, workloads.chat(k.json, name, n_chars=100_000), 7)


def test_seed_edges():
    t = tok("gpt2")
    s = t.seed("", stride=4096)
    assert s.ids.size == 0 and s.checkpoints.shape == (0, 3)
    _check("gpt2", "a", 4096)
    _check("gpt2", "héllo wörld 中文 " * 40, 4096)
    _check("gpt2", "x" * 9000, 3)


def test_seed_capacity_and_arguments():
    import torch
    from toktier_amd import _ffi
    t = tok("gpt2")
    data = ("word " * 2000).encode()
    d_text = torch.frombuffer(bytearray(data), dtype=torch.uint8).to("cuda:0")
    d_ids = torch.empty(len(data), dtype=torch.int32, device="cuda:0")
    d_pts = torch.empty(3, dtype=torch.int64, device="cuda:0")
    with pytest.raises(_ffi.EngineError) as err:   # ~2000 ids, 1 checkpoint slot
        t.engine.encode_seed(d_text.data_ptr(), len(data), d_ids.data_ptr(),
                             len(data), 100, d_pts.data_ptr(), 1)
    assert err.value.status == _ffi.TK_E_CAPACITY
    with pytest.raises(_ffi.EngineError) as err:
        t.engine.encode_seed(d_text.data_ptr(), len(data), d_ids.data_ptr(),
                             len(data), 0, d_pts.data_ptr(), 1)
    assert err.value.status == _ffi.TK_E_INVALID_ARG
    # the engine still encodes normally afterwards
    n, m = t.engine.encode_seed(d_text.data_ptr(), len(data), d_ids.data_ptr(),
                                len(data), 4096, d_pts.data_ptr(), 1)
    assert n > 1000 and m == 1
    assert d_pts.cpu().tolist() == [0, 0, 0]


def test_seed_past_one_launch_of_checkpoints():
    """More than 2^22 checkpoints (stride 1 over 5,000,000 tokens): the
    checkpoint workgroups go out in several launches."""
    _check("gpt2", "a " * 5_000_000, 1)
