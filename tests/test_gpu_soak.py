"""Seeded parity soak through ``encode_batch``: batches of documents drawn
from a seed (fuzz over each family's branch atoms, slices of the C2 / C4 /
C5 / chat workloads, long runs; ``soak_docs.py``), every row checked against
the oracle, bit for bit. Worker processes (spawned, no GPU) draw the
documents and compute the expected ids while the engine encodes the batch
before. The volume per family is ``TK_SOAK_CHARS`` characters (default
2,000,000: one batch per family, so the suite stays short); the soak stops
at its first mismatch and writes what it covered, batch by batch, to
``gpurun_out/soak/<family>.json``."""

from __future__ import annotations

import json
import math
import multiprocessing as mp
import os
import time
from pathlib import Path

import numpy as np
import pytest

import soak_docs
from conftest import FAMILY_NAMES

pytestmark = pytest.mark.gpu

SOAK_CHARS = int(os.environ.get("TK_SOAK_CHARS", "2000000"))
WORKERS = int(os.environ.get("TK_SOAK_WORKERS", "15"))
OUT = Path(__file__).resolve().parent.parent / "gpurun_out" / "soak"


@pytest.fixture(scope="module")
def pool():
    ctx = mp.get_context("spawn")
    with ctx.Pool(WORKERS) as p:
        yield p


@pytest.mark.timeout(max(300, SOAK_CHARS // 100_000))
@pytest.mark.parametrize("name", FAMILY_NAMES)
def test_soak_rows_match_oracle(name, pool):
    import toktier_amd
    n_batches = max(1, math.ceil(SOAK_CHARS / soak_docs.BATCH_CHARS))
    OUT.mkdir(parents=True, exist_ok=True)
    rec = {"family": name, "seed": soak_docs.SOAK_SEED, "target_chars": SOAK_CHARS,
           "batches": 0, "documents": 0, "chars": 0, "bytes": 0, "ids": 0,
           "long_documents": 0, "gpu_seconds": 0.0,
           "mismatch": None}
    t = toktier_amd.load(name)
    t0 = time.perf_counter()
    try:
        jobs = [(name, i) for i in range(n_batches)]
        for index, docs, want in pool.imap(soak_docs.work, jobs):
            g0 = time.perf_counter()
            rows = t.encode_batch(docs, errors="return")
            rec["gpu_seconds"] += time.perf_counter() - g0
            for d, (doc, row, w) in enumerate(zip(docs, rows, want)):
                ok = (not isinstance(w, int) and not isinstance(row, Exception)
                      and np.array_equal(row.array, w))
                if not ok:
                    rec["mismatch"] = {"batch": index, "document": d,
                                       "chars": len(doc), "head": doc[:80],
                                       "engine": repr(row)[:200] if isinstance(row, Exception) else None}
                    break
                rec["ids"] += len(w)
                rec["long_documents"] += len(doc) > 512
            rec["batches"] += 1
            rec["documents"] += len(docs)
            rec["chars"] += sum(map(len, docs))
            rec["bytes"] += sum(len(d.encode("utf-8")) for d in docs)
            rec["seconds"] = round(time.perf_counter() - t0, 2)
            (OUT / f"{name}.json").write_text(json.dumps(rec, indent=1, ensure_ascii=False))
            print(f"soak {name}: batch {index} {rec['chars']:,} chars", flush=True)
            assert rec["mismatch"] is None, rec["mismatch"]
    finally:
        t.close()
    assert rec["chars"] >= min(SOAK_CHARS, soak_docs.BATCH_CHARS)
