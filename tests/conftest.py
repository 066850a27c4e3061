"""Shared fixtures. GPU tests carry ``@pytest.mark.gpu``; everything else
runs on the CPU (the oracle, the table export, the host logic and the
C-ABI symbol surface)."""

from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

FAMILY_NAMES = ("qwen3_8b", "llama_3_1_8b", "gpt2", "laguna_s_2_1",
                "deepseek_v3", "gpt_oss_120b", "kimi_k3", "qwen3_5_08b",
                "nemotron_3_nano_4b")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long-running CPU test")
    config.addinivalue_line("markers", "family(name): the one family a test "
                            "covers (counted under it in the route evidence)")


def _gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


_GPU_OUTCOMES = {"passed": 0, "failed": 0, "skipped": 0}
# per family (a test whose parameters name a family), and "shared" for the
# GPU tests that cover no single family
_FAMILY_OUTCOMES: dict[str, dict[str, int]] = {}
_SELECTION = {"deselected_gpu": 0}
# GPU tests parked in the source with an explicit skip mark and its reason
# (listed in the evidence by node id; any other skip blocks certification)
_PARKED: set[str] = set()
_PARKED_SEEN: list[str] = []
# the family a test covers when no parameter names it: its
# ``@pytest.mark.family(name)`` mark
_NODE_FAMILY: dict[str, str] = {}


def _family_of(nodeid: str) -> str:
    if nodeid in _NODE_FAMILY:
        return _NODE_FAMILY[nodeid]
    params = nodeid.split("[", 1)[1] if "[" in nodeid else ""
    for name in FAMILY_NAMES:
        if name in params:
            return name
    return "shared"


def pytest_runtest_logreport(report):
    """Count the outcomes of GPU parity tests (the route's evidence)."""
    if "gpu" not in report.keywords:
        return
    if report.when == "call" or (report.when == "setup" and not report.passed):
        fam = _FAMILY_OUTCOMES.setdefault(
            _family_of(report.nodeid),
            {"passed": 0, "failed": 0, "skipped": 0, "parked": 0})
        if report.skipped and report.nodeid in _PARKED:
            # counted against the family it covers (a shared one, against
            # every family): a parked test blocks certification
            _PARKED_SEEN.append(report.nodeid)
            fam["parked"] += 1
            return
        key = ("passed" if report.passed else
               "skipped" if report.skipped else "failed")
        _GPU_OUTCOMES[key] += 1
        fam[key] += 1


def pytest_deselected(items):
    _SELECTION["deselected_gpu"] += sum(1 for i in items if "gpu" in i.keywords)


def _complete_selection(config) -> bool:
    """The whole GPU suite was selected: no -k, every gpu-marked test of
    the tests directory collected and none deselected."""
    if getattr(config.option, "keyword", ""):
        return False
    if _SELECTION["deselected_gpu"]:
        return False
    tests_dir = Path(__file__).resolve().parent
    args = [Path(str(a).split("::", 1)[0]).resolve() for a in config.args]
    return any(a in (tests_dir, ROOT) for a in args)


def pytest_sessionfinish(session, exitstatus):
    """After a run that executed GPU parity tests on a device, write the
    evidence the gfx950 route rows are generated from
    (``python -m toktier_amd.registry <evidence file>``): the library's build
    key, the device architecture and driver, the outcome counts overall and
    per family, and whether the whole GPU suite was selected. It goes to the
    output folder that GPU runs hand back."""
    if _GPU_OUTCOMES["passed"] + _GPU_OUTCOMES["failed"] == 0:
        return
    try:
        import json
        import torch
        from toktier_amd._build import MANIFEST, verify
        if not torch.cuda.is_available():
            return
        arch = torch.cuda.get_device_properties(0).gcnArchName.split(":")[0]
        man = json.loads(MANIFEST.read_text())
        import toktier_amd
        t = toktier_amd.load("gpt2")
        driver = t.engine.driver_version
        t.close()
        ev = {"evidence_id": f"ev-gfx950-parity-{man['build_key'][:12]}",
              "suite": "tests -m gpu", "build_key": man["build_key"],
              "build_mismatch": verify(man),
              "architecture": arch, "driver_version": driver,
              "hip_version": torch.version.hip, **_GPU_OUTCOMES,
              "parked": sorted(_PARKED_SEEN),
              "families": _FAMILY_OUTCOMES,
              "selection": {
                  "complete": _complete_selection(session.config),
                  "collected_gpu": session.testscollected and sum(
                      1 for i in session.items if "gpu" in i.keywords),
                  "deselected_gpu": _SELECTION["deselected_gpu"],
                  "markexpr": getattr(session.config.option, "markexpr", ""),
                  "keyword": getattr(session.config.option, "keyword", ""),
                  "exitstatus": int(exitstatus)}}
        out = ROOT / "gpurun_out"
        out.mkdir(exist_ok=True)
        (out / "gfx950_evidence.v1.json").write_text(
            json.dumps(ev, indent=1, sort_keys=True) + "\n")
    except Exception as err:  # evidence is a by-product; never fail the run
        print(f"gfx950 evidence not written: {err}")


def pytest_collection_modifyitems(config, items):
    for item in items:
        mark = item.get_closest_marker("family")
        if mark is not None:
            _NODE_FAMILY[item.nodeid] = mark.args[0]
        if "gpu" in item.keywords and any(
                m.name == "skip" and m.kwargs.get("reason")
                for m in item.iter_markers("skip")):
            _PARKED.add(item.nodeid)
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


class FamilyKit:
    """Everything a parity test needs for one family."""

    def __init__(self, name: str):
        from toktier_amd import bpe_tables, classes, families, standin
        from oracle.oracle import Oracle

        self.name = name
        self.family = families.family(name)
        self.json = standin.load_artifact_json(name)
        self.tables = bpe_tables.load_tables(self.json)
        self.oracle = Oracle(self.tables,
                             classes.table_named(families.class_table_name(self.family)),
                             classes.nfc_qc_table(), self.family.ruleset,
                             self.family.digits_max, self.family.needs_nfc,
                             contractions=self.family.contractions)
        # the artifact's added-token literals, split out as HF does
        import toktier_amd
        self.added = toktier_amd.added_tokens(self.json)
        self.oracle.set_added([t.content.encode() for t in self.added],
                              [t.id for t in self.added])
        self._hf = None

    @property
    def hf(self):
        if self._hf is None:
            from tokenizers import Tokenizer
            self._hf = Tokenizer.from_str(self.json)
        return self._hf

    def hf_ids(self, text: str) -> list[int]:
        return self.hf.encode(text, add_special_tokens=False).ids

    def expected(self, text: str):
        """The oracle's ids for ``text``; when a segment fails the NFC
        quick check, the text is split at its literals, each segment is
        normalized by the certified engine's NFC and encoded alone, and the
        literal ids are spliced back in (what the facade does)."""
        got = self.oracle.encode_bytes(text.encode("utf-8"))
        if not (isinstance(got, int) and self.family.needs_nfc):
            return got
        import numpy as np
        from tokenizers import normalizers
        from toktier_amd import LiteralSplitter
        nfc = normalizers.NFC()
        parts = []
        for seg, lit in LiteralSplitter(self.added).split(text):
            if lit is not None:
                parts.append(np.asarray([lit], dtype=np.uint32))
                continue
            ids = self.oracle.encode_bytes(
                nfc.normalize_str(seg).encode("utf-8"), normalized=True,
                literals=False)
            if isinstance(ids, int):
                return ids
            parts.append(ids)
        return np.concatenate(parts) if parts else np.zeros(0, np.uint32)


_KITS: dict[str, FamilyKit] = {}


def kit(name: str) -> FamilyKit:
    if name not in _KITS:
        _KITS[name] = FamilyKit(name)
    return _KITS[name]


@pytest.fixture(params=FAMILY_NAMES)
def family_kit(request) -> FamilyKit:
    return kit(request.param)


@pytest.fixture(scope="session", autouse=True)
def _oracle_built():
    from oracle import oracle
    if not oracle.LIB.exists():
        oracle.build()


def drop_byte_tokens(tokenizer_json: str, drop: bytes) -> str:
    """A variant of a byte-level artifact without the single-byte tokens of
    `drop` (and the merges that use a token holding one): those bytes have
    no id, so the engine and HF drop them before merging."""
    import json
    from toktier_amd import bpe_tables
    spec = json.loads(tokenizer_json)
    b2u = bpe_tables.bytes_to_unicode()
    gone = {b2u[b] for b in drop}
    model = spec["model"]
    model["vocab"] = {t: i for t, i in model["vocab"].items() if t not in gone}
    model["merges"] = [[a, b] for a, b in bpe_tables._merge_pairs(model["merges"])
                       if not any(ch in gone for ch in a + b)]
    return json.dumps(spec)
