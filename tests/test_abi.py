"""CPU: the C-ABI library loads, exports every entry point that
include/toktier_hip.h declares, and validates its inputs without a GPU
(preflight mirrors validate_tables, gpu.rs:1642-1679)."""

from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

from conftest import kit
from toktier_amd import _ffi, classes
from toktier_amd._build import LIB

HEADER = Path(__file__).resolve().parent.parent / "include" / "toktier_hip.h"


def declared_symbols() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"\b(tk_[a-z_]+)\s*\(", text))


def test_header_declares_the_binding_surface():
    assert declared_symbols() == set(_ffi.SYMBOLS)


def test_library_exports_every_declared_symbol():
    assert LIB.exists(), "run __graft_entry__.build() first"
    lib = C.CDLL(str(LIB))
    for name in declared_symbols():
        assert hasattr(lib, name), name


def _cfg(k, **over):
    t = k.tables
    f = k.family
    cfg = _ffi.TkConfig(
        abi_version=_ffi.TK_ABI_VERSION, device_ordinal=0, ruleset=f.ruleset,
        digits_max=f.digits_max, contractions=1, needs_nfc=int(f.needs_nfc),
        ignore_merges=int(t.ignore_merges), pair_count=t.pair_count,
        vocab_count=t.vocab_count, family=f.name.encode(),
        artifact_sha256=b"x", expected_architecture=b"gfx950")
    for key, val in over.items():
        setattr(cfg, key, val)
    return cfg


def _preflight(cfg, k, **arrays):
    t = k.tables
    a = dict(cls=classes.class_table(), pk=t.pair_keys, pv=t.pair_vals,
             bid=t.byte_id, vk=t.vocab_keys, vv=t.vocab_vals,
             ub=t.unsafe_bits if t.unsafe_bits.size else np.zeros(0, np.uint32))
    a.update(arrays)
    args = []
    for key in ("cls", "pk", "pv", "bid", "vk", "vv", "ub"):
        arr = np.ascontiguousarray(a[key])
        args += [arr.ctypes.data if arr.size else None, arr.nbytes]
    return _ffi.lib().tk_engine_preflight(C.byref(cfg), *args)


@pytest.mark.parametrize("name", ["qwen3_8b", "gpt2"])
def test_preflight_accepts_valid_tables(name):
    k = kit(name)
    assert _preflight(_cfg(k), k) == _ffi.TK_OK


def test_preflight_rejects_bad_shapes_and_config():
    k = kit("gpt2")
    L = _ffi.lib()
    assert _preflight(_cfg(k, abi_version=99), k) == _ffi.TK_E_INVALID_ARG
    assert b"abi_version" in L.tk_last_error()
    assert _preflight(_cfg(k, ruleset=7), k) == _ffi.TK_E_INVALID_ARG
    assert _preflight(_cfg(k, ruleset=0, digits_max=0), k) == _ffi.TK_E_INVALID_ARG
    assert _preflight(_cfg(k, contractions=0), k) == _ffi.TK_E_INVALID_ARG
    assert _preflight(_cfg(k), k, cls=classes.class_table()[:1000]) == _ffi.TK_E_SHAPE
    assert b"U+10FFFF" in L.tk_last_error()
    assert _preflight(_cfg(k, pair_count=k.tables.pair_count - 1), k) == _ffi.TK_E_SHAPE
    assert _preflight(_cfg(k), k, pv=k.tables.pair_vals[:-1]) == _ffi.TK_E_SHAPE
    assert _preflight(_cfg(k), k, bid=k.tables.byte_id[:255]) == _ffi.TK_E_SHAPE
    assert _preflight(_cfg(k), k, ub=np.zeros(3, np.uint8)) == _ffi.TK_E_SHAPE


def test_preflight_checks_the_ruleset_class_table():
    """deepseek reads a seven-class table and has no contractions; the
    other rulesets read four classes (values above a ruleset's top class
    are refused before anything reaches the device)."""
    k = kit("gpt2")
    L = _ffi.lib()
    ds = classes.deepseek_class_table()
    DS = _ffi.TK_RULESET_DEEPSEEK
    assert _preflight(_cfg(k, ruleset=DS, digits_max=3, contractions=0), k,
                      cls=ds) == _ffi.TK_OK
    assert _preflight(_cfg(k, ruleset=DS, digits_max=3, contractions=1), k,
                      cls=ds) == _ffi.TK_E_INVALID_ARG
    assert b"contractions" in L.tk_last_error()
    assert _preflight(_cfg(k, ruleset=0, digits_max=1), k, cls=ds) == _ffi.TK_E_SHAPE
    bad = ds.copy()
    bad[0x4E00] = 7
    assert _preflight(_cfg(k, ruleset=DS, digits_max=3, contractions=0), k,
                      cls=bad) == _ffi.TK_E_SHAPE
    assert b"class table value" in L.tk_last_error()


def test_open_without_a_device_fails_cleanly():
    try:
        import torch
        if torch.cuda.is_available():
            pytest.skip("a GPU is visible")
    except ImportError:
        pass
    k = kit("gpt2")
    with pytest.raises(_ffi.EngineError) as err:
        _ffi.Engine(_cfg(k), classes.class_table(), k.tables, None)
    assert err.value.status == _ffi.TK_E_DEVICE


def test_null_arguments_are_refused():
    L = _ffi.lib()
    n = C.c_size_t()
    assert L.tk_engine_encode(None, b"abc", 3, 0, None, 0, C.byref(n)) == _ffi.TK_E_INVALID_ARG
    assert L.tk_engine_set_timing(None, 1) == _ffi.TK_E_INVALID_ARG
    assert L.tk_engine_delivery(None) == b""


CRATE = HEADER.parent.parent / "crates" / "toktier-hip-driver" / "src" / "lib.rs"


def _header_defines() -> dict[str, int]:
    out = {}
    for name, val in re.findall(r"#define\s+(TK_[A-Z0-9_]+)\s+\(?(-?\d+)u?\)?",
                                HEADER.read_text()):
        out[name] = int(val)
    return out


def test_rust_crate_binds_every_symbol_with_the_headers_constants():
    """The source crate `toktier-hip-driver` (no Rust toolchain here, so it
    is checked as text): it loads every entry point the header declares,
    and each constant it repeats has the header's value, the ruleset codes
    included. Its ruleset strings are the reference's (gpu.rs:40-62)."""
    src = CRATE.read_text()
    loaded = set(re.findall(r'symbol\(handle, "(tk_[a-z_]+)"\)', src))
    assert loaded == declared_symbols()
    consts = {n: int(v.replace("_", "")) for n, v in re.findall(
        r"pub const (TK_[A-Z0-9_]+): \w+ = (-?[\d_]+);", src)}
    defines = _header_defines()
    assert consts, "no constants found"
    for name, val in consts.items():
        assert name in defines, name
        assert defines[name] == val, name
    for name in defines:
        if name.startswith(("TK_RULESET_", "TK_E_", "TK_OPT_", "TK_KERNEL")):
            assert name in consts, name
    arms = dict(re.findall(r'"([a-z0-9]+)" => Ok\(Self::(\w+)\)', src))
    assert set(arms) == {"cl100k", "r50k", "laguna", "deepseek", "o200k", "kimi"}
    codes = dict(re.findall(r"Self::(\w+) => (TK_RULESET_[A-Z0-9]+),", src))
    for s, variant in arms.items():
        assert codes[variant] == "TK_RULESET_" + s.upper()
