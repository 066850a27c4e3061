"""CPU: the benchmark generators are deterministic and have the shapes the
configurations state."""

from __future__ import annotations

import numpy as np

from conftest import kit
from toktier_amd import workloads


def test_c1_ascii_shape():
    js = kit("qwen3_8b").json
    t = workloads.config1(js)
    assert len(t) == 65_536 and t.isascii()
    assert t == workloads.config1(js)
    assert "\n" in t and any(ch.isdigit() for ch in t)
    assert "  " not in t  # single spaces between words


def test_c2_mixed_script_shape():
    js = kit("qwen3_8b").json
    t = workloads.config2(js, n_chars=300_000)
    assert len(t) == 300_000 and t == workloads.config2(js, n_chars=300_000)
    latin1 = sum(1 for ch in t if 0xC0 <= ord(ch) <= 0xFF)
    assert latin1 > 1000
    assert "\t" in t and "\r\n" in t
    assert max(ord(ch) for ch in t) <= 0xFF


def test_c3_documents():
    js = kit("gpt2").json
    docs = workloads.config3(js, n_docs=16)
    assert len(docs) == 16
    assert all(1024 <= len(d) <= 32768 and d.isascii() for d in docs)


def test_c4_code_shape():
    js = kit("llama_3_1_8b").json
    t = workloads.config4(js, n_chars=200_000)
    assert len(t) == 200_000
    assert "0x" in t and "\\n" in t and "_" in t and "\n    " in t


def test_c5_stress_shape():
    js = kit("qwen3_8b").json
    t = workloads.config5(js, n_chars=400_000, n_runs=4, run_chars=20_000)
    assert len(t) == 400_000
    cjk = sum(1 for ch in t if 0x4E00 <= ord(ch) <= 0x9FFF)
    assert 0.35 < cjk / len(t) < 0.75
    assert "\u200d" in t and any(ord(ch) >= 0x1F300 for ch in t)
    # the embedded runs: letter-only stretches of at least run_chars
    runs, cur = [], 0
    for ch in t:
        cur = cur + 1 if ch.isalpha() else 0
        if cur == 20_000:
            runs.append(1)
    assert len(runs) >= 4


def test_full_size_configs_are_exact():
    js = kit("qwen3_8b").json
    assert len(workloads.config2(js)) == workloads.CHARS_4M
    rng = np.random.default_rng(0)
    assert rng is not None
