"""Per-codepoint tables shipped with the package.

Both tables are probed from the certified engine by
``toktier_amd.tables_gen`` and verified here against the sha256 of the
reference's own tables (``src/toktier/kernels/tables/kernel_families.v1.json:11``
for ``cl100k_v3``, ``:21`` for ``cl100k_m2l_v3``, ``:65`` for ``nfc_qc_v1``;
digest of the ``.npy``
serialisation of the 0x110000-entry ``uint8`` array). A table that does not
hash to its pin is refused.
"""

from __future__ import annotations

import hashlib
import io
from functools import lru_cache
from pathlib import Path

import numpy as np

TABLE_DIR = Path(__file__).resolve().parent / "data" / "tables"
PLANE = 0x110000

CLASS_TABLE_SHA256 = "aab53c6705260d07f65d9762aecba729b18e11cb9710a4aea54157475cbfdf97"
NFC_QC_SHA256 = "1a7d121e9092cdf577d992452393d25116b2577ab74dd5a067e6ca00a535d311"
#: kernel_families.v1.json class_tables.cl100k_m2l_v3 (marks as letters)
M2L_TABLE_SHA256 = "e75a70e3aeb90efe7ad16502d932845a56e22f903f43d6b5061767574bcf3d8f"
#: kernel_families.v1.json class_tables.deepseek_v1
DEEPSEEK_TABLE_SHA256 = "b4242c04ffc981d9f457981546c43b2a82b53e3d18bf6f7d1ee1e7625c423bf7"
#: kernel_families.v1.json class_tables.o200k_v4
O200K_TABLE_SHA256 = "28e6d9e468b2c83db4188787515fa0e89d49750c20c966a9a89481aaf3b9e8ea"
#: kernel_families.v1.json class_tables.kimi_v1
KIMI_TABLE_SHA256 = "9b752f3757bdec444ed745f27bac35fdb2aca8893521ef3d40cff7b17f681383"

__all__ = ["class_table", "m2l_class_table", "deepseek_class_table",
           "o200k_class_table", "kimi_class_table", "table_named",
           "nfc_qc_table",
           "npy_sha256", "PLANE", "table_for"]


def npy_sha256(arr: np.ndarray) -> str:
    buf = io.BytesIO()
    np.save(buf, arr)
    return hashlib.sha256(buf.getvalue()).hexdigest()


def _load(name: str, key: str, sha: str) -> np.ndarray:
    with np.load(TABLE_DIR / name, allow_pickle=False) as z:
        arr = np.ascontiguousarray(z[key], dtype=np.uint8)
    if arr.shape != (PLANE,):
        raise ValueError(f"{name}: bad shape {arr.shape}")
    got = npy_sha256(arr)
    if got != sha:
        raise ValueError(f"{name}: sha256 {got} != pinned {sha}")
    arr.setflags(write=False)
    return arr


@lru_cache(maxsize=None)
def class_table() -> np.ndarray:
    """Classes P=0, L=1, N=2, S=3 for every codepoint."""
    return _load("classes.npz", "cl100k", CLASS_TABLE_SHA256)


@lru_cache(maxsize=None)
def m2l_class_table() -> np.ndarray:
    """The four classes with Mark code points in L (Qwen3.5's split)."""
    return _load("classes_m2l.npz", "cl100k_m2l", M2L_TABLE_SHA256)


@lru_cache(maxsize=None)
def nfc_qc_table() -> np.ndarray:
    """NFC quick-check values: 0 safe starter, 1..K class rank, 255 unsafe."""
    return _load("nfc_qc.npz", "nfc_qc", NFC_QC_SHA256)


@lru_cache(maxsize=None)
def deepseek_class_table() -> np.ndarray:
    """DeepSeek classes O=0 L=1 M=2 N=3 PS=4 WS=5 CRLF=6 for every codepoint."""
    return _load("classes_deepseek.npz", "deepseek", DEEPSEEK_TABLE_SHA256)


@lru_cache(maxsize=None)
def o200k_class_table() -> np.ndarray:
    """o200k classes P=0 U=1 L=2 C=3 N=4 S=5 M=6 for every codepoint."""
    return _load("classes_o200k.npz", "o200k", O200K_TABLE_SHA256)


@lru_cache(maxsize=None)
def kimi_class_table() -> np.ndarray:
    """kimi classes: the o200k seven (letters without Han) plus HL=7 HN=8
    HP=9 (Han letters, Han numbers, other Han)."""
    return _load("classes_kimi.npz", "kimi", KIMI_TABLE_SHA256)


def table_named(name: str) -> np.ndarray:
    """A class table by its reference name (``kernel_families.v1.json``
    ``class_tables``)."""
    return {"cl100k_v3": class_table, "cl100k_m2l_v3": m2l_class_table,
            "deepseek_v1": deepseek_class_table, "o200k_v4": o200k_class_table,
            "kimi_v1": kimi_class_table}[name]()


def table_for(ruleset_name: str) -> np.ndarray:
    """The class table a ruleset reads by default (a family may name
    another: ``Family.class_table``)."""
    if ruleset_name == "deepseek":
        return deepseek_class_table()
    if ruleset_name == "o200k":
        return o200k_class_table()
    if ruleset_name == "kimi":
        return kimi_class_table()
    return class_table()
