"""GPU parity of the added-token split (k_added ahead
of k_pretok) through the C-ABI: the engine against HF tokenizers 0.22.2
and the oracle, bit for bit."""

from __future__ import annotations

import numpy as np
import pytest

from conftest import FAMILY_NAMES, kit
from test_added import PROBES, bare, with_added

pytestmark = pytest.mark.gpu

_TOKS: dict = {}


def tok(name: str):
    if name not in _TOKS:
        import toktier_amd
        _TOKS[name] = toktier_amd.load(name)
    return _TOKS[name]


def _probe_tok(contents: list[str]):
    """A GPT-2 engine opened on the stand-in with `contents` as its added
    tokens (HF assigns their ids)."""
    import toktier_amd
    key = ("probe",) + tuple(contents)
    if key not in _TOKS:
        js = with_added(kit("gpt2").json, contents)
        _TOKS[key] = (toktier_amd.Tokenizer("gpt2", js), js)
    return _TOKS[key]


@pytest.mark.parametrize("name", FAMILY_NAMES)
def test_chat_text_matches_hf_and_counts_literals(name):
    from toktier_amd import workloads
    k, t = kit(name), tok(name)
    text = workloads.chat(k.json, name, n_chars=40_000)
    got = t.encode(text).array
    assert list(got) == k.hf_ids(text)
    n_lit = sum(1 for _, lit in t.split_literals(text) if lit is not None)
    assert n_lit > 10
    assert t.explain()["last_execution"]["added_literals"] == n_lit


@pytest.mark.parametrize("probe", range(len(PROBES)))
def test_probe_tables(probe):
    from tokenizers import Tokenizer
    contents, docs = PROBES[probe]
    t, js = _probe_tok(contents)
    full = Tokenizer.from_str(js)
    for d in docs:
        assert list(t.encode(d).array) == \
            full.encode(d, add_special_tokens=False).ids, d
    # overlapping candidates in bulk: clusters walked by one thread each
    rng = np.random.default_rng(5)
    frags = contents + ["<", ">", "a", "b", "c", "t", " "]
    for _ in range(60):
        d = "".join(frags[int(i)] for i in rng.integers(0, len(frags), 400))
        assert list(t.encode(d).array) == \
            full.encode(d, add_special_tokens=False).ids, d


@pytest.mark.family("qwen3_8b")
def test_literals_across_tile_and_block_edges():
    """A literal starting at every offset around the pretokenizer's tiles
    (PT_TILE bytes) and the literal kernels' 4096-byte blocks."""
    from toktier_amd import workloads
    k, t = kit("qwen3_8b"), tok("qwen3_8b")
    base = workloads.config2(k.json, n_chars=20_000)
    base = "".join(ch for ch in base if ord(ch) < 128)[:13_000]
    lit = "<|im_end|>"
    from test_gpu_parity import TILE
    for edge in (TILE, 2 * TILE, 3072, 4096, 6144, 8192, 12288):
        for d in range(-12, 3):
            p = edge + d
            s = base[:p] + lit + base[p:]
            got = t.encode(s).array
            want = k.oracle.encode_bytes(s.encode())
            assert np.array_equal(got, want), (edge, d)


@pytest.mark.family("qwen3_8b")
def test_dense_literal_streams():
    k, t = kit("qwen3_8b"), tok("qwen3_8b")
    for s in ["<|im_end|>" * 50_000, ("<|im_start|>" + "x") * 30_000,
              "<|im_end|" * 20_000 + ">", "<think>" * 10_000 + " ok"]:
        got = t.encode(s).array
        want = k.oracle.encode_bytes(s.encode())
        assert np.array_equal(got, want), s[:40]
    assert list(t.encode("<|im_end|>" * 300).array) == [151645] * 300


@pytest.mark.family("qwen3_8b")
def test_full_size_chat_request_matches_oracle():
    from toktier_amd import workloads
    k, t = kit("qwen3_8b"), tok("qwen3_8b")
    data = workloads.chat(k.json, "qwen3_8b").encode()
    got = t.encode_bytes(data)
    want = k.oracle.encode_bytes(data)
    assert not isinstance(want, int)
    assert np.array_equal(got, want)


def test_batch_rows_with_literals():
    name = "llama_3_1_8b"
    k, t = kit(name), tok(name)
    from toktier_amd import workloads
    chat = workloads.chat(k.json, name, n_chars=30_000)
    rng = np.random.default_rng(8)
    docs = []
    for _ in range(30):
        a = int(rng.integers(0, len(chat) - 1))
        docs.append(chat[a:a + int(rng.integers(0, 2500))])
    # a literal cut in two by a document boundary is no literal
    docs += ["<|eot_", "id|>", "<|eot_id|>", "", "x<|eot_id|>"]
    rows = t.encode_batch(docs)
    for d, r in zip(docs, rows):
        assert list(r.array) == k.hf_ids(d), d[:60]


@pytest.mark.family("qwen3_8b")
def test_nfc_fallback_splits_literals_first():
    k, t = kit("qwen3_8b"), tok("qwen3_8b")
    texts = ["<|im_end|≯ x", "e<|im_start|>́",
             "café<|im_end|>\nnäive<think>x</think>"]
    for s in texts:
        assert list(t.encode(s).array) == k.hf_ids(s), s
    rows = t.encode_batch(texts + ["plain <|im_end|>"])
    for s, r in zip(texts + ["plain <|im_end|>"], rows):
        assert list(r.array) == k.hf_ids(s), s


@pytest.mark.family("qwen3_8b")
def test_no_added_flag_and_device_entry():
    import torch
    from tokenizers import Tokenizer
    from toktier_amd import _ffi, workloads
    k, t = kit("qwen3_8b"), tok("qwen3_8b")
    text = workloads.chat(k.json, "qwen3_8b", n_chars=50_000)
    data = text.encode()
    plain = Tokenizer.from_str(bare(k.json))
    got = t.engine.encode(data, _ffi.TK_FLAG_NO_ADDED)
    assert list(got) == plain.encode(text, add_special_tokens=False).ids
    d_text = torch.frombuffer(bytearray(data), dtype=torch.uint8).to("cuda:0")
    d_ids = torch.empty(len(data), dtype=torch.int32, device="cuda:0")
    n = t.engine.encode_device(d_text.data_ptr(), len(data),
                               d_ids.data_ptr(), len(data))
    assert np.array_equal(d_ids[:n].cpu().numpy().view(np.uint32),
                          k.oracle.encode_bytes(data))


def test_unsupported_tables_are_refused():
    import json
    from toktier_amd import _ffi
    t = tok("gpt2")
    for flags in (_ffi.TK_ADDED_LSTRIP, _ffi.TK_ADDED_RSTRIP,
                  _ffi.TK_ADDED_SINGLE_WORD):
        with pytest.raises(_ffi.EngineError) as err:
            t.engine.set_added([b"<m>"], [50257], [flags])
        assert err.value.status == _ffi.TK_E_UNSUPPORTED
    # raw and normalized literals that can overlap (two extraction passes)
    with pytest.raises(_ffi.EngineError) as err:
        t.engine.set_added([b"ab", b"bc"], [50257, 50258],
                           [0, _ffi.TK_ADDED_NORMALIZED])
    assert err.value.status == _ffi.TK_E_UNSUPPORTED
    # a normalized literal where the family normalizes
    with pytest.raises(_ffi.EngineError) as err:
        tok("qwen3_8b").engine.set_added([b"<n>"], [151700],
                                         [_ffi.TK_ADDED_NORMALIZED])
    assert err.value.status == _ffi.TK_E_UNSUPPORTED
    with pytest.raises(_ffi.EngineError):
        t.engine.set_added([b"<a>", b"<a>"], [1, 2], [0, 0])  # duplicate
    # the family table still stands after refusals: reinstall and check
    import toktier_amd
    added = toktier_amd.added_tokens(kit("gpt2").json)
    t.engine.set_added([a.content.encode() for a in added],
                       [a.id for a in added], [a.flags for a in added])
    s = "a<|endoftext|>b"
    assert list(t.encode(s).array) == kit("gpt2").hf_ids(s)
    # normalized and raw literals that cannot overlap: one pass is exact
    from tokenizers import Tokenizer
    spec = json.loads(kit("gpt2").json)
    spec["added_tokens"] = [
        {"id": 0, "content": "<r>", "single_word": False, "lstrip": False,
         "rstrip": False, "normalized": False, "special": True},
        {"id": 0, "content": "[N]", "single_word": False, "lstrip": False,
         "rstrip": False, "normalized": True, "special": False}]
    js = json.dumps(spec)
    t2 = toktier_amd.Tokenizer("gpt2", js)
    hf = Tokenizer.from_str(js)
    for s in ["x<r>[N]y", "[N]<r>", "<r[N]>", "[<r>N]"]:
        assert list(t2.encode(s).array) == \
            hf.encode(s, add_special_tokens=False).ids, s
    t2.close()


@pytest.mark.parametrize("name", ["llama_3_1_8b", "qwen3_8b"])
def test_document_starts_inside_runs(name):
    """Document starts (batch boundaries and literal edges) inside digit
    runs (Llama-3 groups digits by three) and CR/LF whitespace runs: the
    pretokenizer's word-mask shortcuts must end a run at each of them."""
    k, t = kit(name), tok(name)
    lit = k.added[-1].content
    rng = np.random.default_rng(21)
    pieces = ["1234567", "89", "0", " \r\n", "\r\n", "\r\n x", " \t\r\n\r\n ",
              "a", "'s", "  ", "\n\n", lit, "x" * 30, "12" * 20]
    docs = []
    for _ in range(80):
        docs.append("".join(pieces[int(i)] for i in
                            rng.integers(0, len(pieces), int(rng.integers(1, 9)))))
    rows = t.encode_batch(docs)
    for d, r in zip(docs, rows):
        assert list(r.array) == k.hf_ids(d), repr(d)
    joined = "".join(docs)
    assert list(t.encode(joined).array) == k.hf_ids(joined)


def test_laguna_newline_parts():
    """Laguna's stage 0 (a (?:\\r?\\n)+ split that keeps each run with the
    text after it) on the device: batch boundaries inside newline runs,
    literals next to runs, a full-size code request, and the refusal of
    literals that begin or end with CR / LF."""
    from toktier_amd import _ffi, workloads
    name = "laguna_s_2_1"
    k, t = kit(name), tok(name)
    rng = np.random.default_rng(31)
    pieces = ["\n", "\r\n", "\r", "\n\n", " ", "  \n", "x", "def", "1",
              "<|im_end|>", "\t", "!", "'s", "é"]
    docs = ["".join(pieces[int(i)] for i in rng.integers(0, len(pieces), int(n)))
            for n in rng.integers(1, 12, size=120)]
    rows = t.encode_batch(docs)
    for d, r in zip(docs, rows):
        assert list(r.array) == k.hf_ids(d), repr(d)
    joined = "".join(docs)
    assert list(t.encode(joined).array) == k.hf_ids(joined)
    data = workloads.config4(k.json).encode()
    got = t.encode_bytes(data)
    want = k.oracle.encode_bytes(data)
    assert not isinstance(want, int) and np.array_equal(got, want)
    for bad in (b"\n<x>", b"<x>\r"):
        with pytest.raises(_ffi.EngineError) as err:
            t.engine.set_added([bad], [100100], [0])
        assert err.value.status == _ffi.TK_E_UNSUPPORTED
