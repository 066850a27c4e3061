"""The gfx950 route in routing data: registry rows and planner admission
(reference: src/toktier/routing/plan.py:1-39, :211-324, :470-580;
registry_view.py:192-206). CPU only: admission is a pure function of the
facts and the rows."""

from __future__ import annotations

import json

import pytest

from toktier_amd import registry as R

KEY = "k" * 64
SHA = "a" * 64


def _row(status=R.STATUS_CERTIFIED, devices=("gfx950",), driver_min=60000000,
         digest=KEY, oracle="0.22.2"):
    rec = {"artifact_sha256": SHA, "family": "qwen3_8b",
           "oracle_version": oracle, "evidence_id": "ev",
           "backends": {"gpu": {"status": status, "deliveries": {"prebuilt": {
               "status": status, "binary_digest": digest,
               "devices": list(devices), "devices_experimental": [],
               "driver_min": driver_min}}}}}
    reg = {"schema_version": 1, "artifacts": [rec]}
    reg["root_digest"] = R.root_digest(reg)
    return reg


def _facts(**kw):
    base = dict(library_loaded=True, build_key=KEY, build_failed=False,
                architectures=("gfx950",), driver_version=70226015,
                oracle_version="0.22.2")
    base.update(kw)
    return R.Facts(**base)


def _codes(adm):
    return [r.code for r in adm.refusals]


def test_certified_row_is_admitted_under_both_policies():
    for pol in (R.POLICY_CERTIFIED, R.POLICY_EXPERIMENTAL):
        adm = R.admit(_row(), SHA, _facts(), pol)
        assert adm.admitted and not adm.refusals and not adm.waivers


@pytest.mark.parametrize("case,facts,reg,code,waivable", [
    ("no library", dict(library_loaded=False), None, R.R_BACKEND_UNAVAILABLE, False),
    ("no device", dict(architectures=()), None, R.R_NO_GPU_DETECTED, False),
    ("unknown artifact", {}, {"schema_version": 1, "artifacts": []},
     R.R_UNCERTIFIED_ARTIFACT, True),
    ("experimental row", {}, dict(status=R.STATUS_EXPERIMENTAL),
     R.R_UNCERTIFIED_ARTIFACT, True),
    ("unsupported row", {}, dict(status=R.STATUS_UNSUPPORTED),
     R.R_UNCERTIFIED_ARTIFACT, False),
    ("oracle drift", dict(oracle_version="0.21.0"), {}, R.R_ORACLE_MISMATCH, True),
    ("other architecture", dict(architectures=("gfx942",)), {},
     R.R_SM_UNCERTIFIED, True),
    ("old driver", dict(driver_version=50000000), {}, R.R_DRIVER_TOO_OLD, True),
    ("unknown driver", dict(driver_version=None), {}, R.R_DRIVER_TOO_OLD, True),
    ("build failed", dict(build_failed=True), {}, R.R_KERNEL_BUILD_FAILED, False),
    ("other build", dict(build_key="b" * 64), {}, R.R_KERNEL_DIGEST_MISMATCH, True),
    ("no build key", dict(build_key=None), {}, R.R_KERNEL_DIGEST_MISMATCH, True),
])
def test_each_check_refuses_with_the_reference_code(case, facts, reg, code,
                                                    waivable):
    reg = reg if isinstance(reg, dict) and "schema_version" in reg else \
        _row(**(reg or {}))
    strict = R.admit(reg, SHA, _facts(**facts), R.POLICY_CERTIFIED)
    assert not strict.admitted, case
    assert _codes(strict)[-1] == code, case
    assert strict.refusals[-1].waivable == waivable, case
    loose = R.admit(reg, SHA, _facts(**facts), R.POLICY_EXPERIMENTAL)
    assert loose.admitted == waivable, case
    if waivable:
        assert [w.code for w in loose.waivers] == [code], case


def test_checks_run_in_the_reference_order():
    # several problems at once: the certified policy stops at the first,
    # the experimental one waives each waivable one in order
    facts = _facts(architectures=("gfx942",), driver_version=1,
                   build_key="b" * 64)
    strict = R.admit(_row(), SHA, facts, R.POLICY_CERTIFIED)
    assert _codes(strict) == [R.R_SM_UNCERTIFIED]
    loose = R.admit(_row(), SHA, facts, R.POLICY_EXPERIMENTAL)
    assert [w.code for w in loose.waivers] == [
        R.R_SM_UNCERTIFIED, R.R_DRIVER_TOO_OLD, R.R_KERNEL_DIGEST_MISMATCH]
    # a non-waivable refusal ends the route even after waivers
    dead = R.admit(_row(), SHA, _facts(architectures=("gfx942",),
                                        build_failed=True), R.POLICY_EXPERIMENTAL)
    assert not dead.admitted
    assert _codes(dead) == [R.R_SM_UNCERTIFIED, R.R_KERNEL_BUILD_FAILED]


def _evidence(**kw):
    ev = {"evidence_id": "ev1", "build_key": KEY, "build_mismatch": None,
          "architecture": "gfx950", "passed": 40, "failed": 0, "skipped": 0,
          "driver_version": 70226015,
          "families": {"qwen3_8b": {"passed": 30, "failed": 0, "skipped": 0},
                       "gpt2": {"passed": 0, "failed": 0, "skipped": 0},
                       "shared": {"passed": 10, "failed": 0, "skipped": 0}},
          "selection": {"complete": True, "collected_gpu": 40,
                        "deselected_gpu": 0, "markexpr": "gpu", "keyword": ""}}
    ev.update(kw)
    return ev


def _status(reg, i=0):
    return reg["artifacts"][i]["backends"]["gpu"]["deliveries"]["prebuilt"]


def test_generate_certifies_only_a_judged_build():
    man = {"build_key": KEY, "hipcc": ["HIP version: 7.2"], "flags": ["-O3"]}
    reg = R.generate(_evidence(), man, {"qwen3_8b": SHA})
    row = _status(reg)
    assert row["status"] == R.STATUS_CERTIFIED and row["devices"] == ["gfx950"]
    assert row["readings"] == {"passed": 30, "failed": 0, "skipped": 0}
    assert R.architecture_statuses(row) == {"gfx950": R.STATUS_CERTIFIED}
    assert R.admit(reg, SHA, _facts(), R.POLICY_CERTIFIED).admitted
    sel = _evidence()["selection"]
    for bad in (dict(failed=1), dict(build_key="b" * 64),
                dict(architecture="gfx942"), dict(passed=0),
                dict(skipped=1),
                dict(build_mismatch="library bytes differ from the manifest"),
                # a subset of the suite (-k, deselected tests, a single file)
                dict(selection={**sel, "complete": False}),
                dict(selection={**sel, "deselected_gpu": 3}),
                dict(selection={**sel, "collected_gpu": 41}),
                # the family's own tests failed, were skipped or never ran
                dict(families={"qwen3_8b": {"passed": 29, "failed": 1, "skipped": 0}}),
                dict(families={"qwen3_8b": {"passed": 29, "failed": 0, "skipped": 1}}),
                dict(families={"shared": {"passed": 40, "failed": 0, "skipped": 0}}),
                dict(families=None),
                # a test of the family, or one shared by every family, is
                # parked by an explicit skip mark (listed, not run)
                dict(families={"qwen3_8b": {"passed": 30, "failed": 0, "skipped": 0,
                                            "parked": 1}},
                     parked=["tests/x.py::test_p"],
                     selection={**sel, "collected_gpu": 41}),
                dict(families={"qwen3_8b": {"passed": 30, "failed": 0, "skipped": 0},
                               "shared": {"passed": 10, "failed": 0, "skipped": 0,
                                          "parked": 1}},
                     parked=["tests/x.py::test_p"],
                     selection={**sel, "collected_gpu": 41})):
        reg = R.generate(_evidence(**bad), man, {"qwen3_8b": SHA})
        row = _status(reg)
        assert row["status"] == R.STATUS_EXPERIMENTAL, bad
        assert R.architecture_statuses(row) == {"gfx950": R.STATUS_EXPERIMENTAL}
        assert not R.admit(reg, SHA, _facts(), R.POLICY_CERTIFIED).admitted


def test_a_parked_test_blocks_only_its_own_family():
    man = {"build_key": KEY, "hipcc": [], "flags": []}
    sel = _evidence()["selection"]
    ev = _evidence(families={
        "qwen3_8b": {"passed": 30, "failed": 0, "skipped": 0},
        "deepseek_v3": {"passed": 9, "failed": 0, "skipped": 0, "parked": 1},
        "shared": {"passed": 10, "failed": 0, "skipped": 0}},
        passed=49, parked=["tests/x.py::test_p"],
        selection={**sel, "collected_gpu": 50})
    reg = R.generate(ev, man, {"qwen3_8b": SHA, "deepseek_v3": "c" * 64})
    by_family = {a["family"]: a["backends"]["gpu"]["status"]
                 for a in reg["artifacts"]}
    assert by_family == {"qwen3_8b": R.STATUS_CERTIFIED,
                         "deepseek_v3": R.STATUS_EXPERIMENTAL}


def test_generate_judges_each_family_on_its_own_tests():
    # gpt2's parity tests did not run in this evidence: its row stays
    # experimental while qwen3's is certified
    man = {"build_key": KEY, "hipcc": [], "flags": []}
    reg = R.generate(_evidence(), man, {"qwen3_8b": SHA, "gpt2": "b" * 64})
    by_family = {a["family"]: a["backends"]["gpu"]["status"]
                 for a in reg["artifacts"]}
    assert by_family == {"qwen3_8b": R.STATUS_CERTIFIED,
                         "gpt2": R.STATUS_EXPERIMENTAL}


def test_a_library_that_is_not_the_manifest_build_is_refused():
    facts = _facts(build_mismatch="sources changed since the build: csrc/tk_device.h")
    strict = R.admit(_row(), SHA, facts, R.POLICY_CERTIFIED)
    assert not strict.admitted
    assert _codes(strict) == [R.R_KERNEL_DIGEST_MISMATCH]
    assert strict.refusals[0].detail["cause"].startswith("sources changed")
    loose = R.admit(_row(), SHA, facts, R.POLICY_EXPERIMENTAL)
    assert loose.admitted and [w.code for w in loose.waivers] == [
        R.R_KERNEL_DIGEST_MISMATCH]


def test_build_key_covers_every_source_and_the_abi_header(tmp_path, monkeypatch):
    from toktier_amd import _build
    names = set(_build.hashed_files())
    assert "include/toktier_hip.h" in names
    assert {"csrc/tk_device.h", "csrc/tk_device.hip", "csrc/tk_added.hip",
            "csrc/tk_engine.cpp"} <= names
    # an edit to a header alone changes the key and is caught by verify()
    base = _build.source_digests()
    k0 = _build.build_key(base, ["-O3"], ["v"])
    edited = dict(base, **{"csrc/tk_device.h": "0" * 64})
    assert _build.build_key(edited, ["-O3"], ["v"]) != k0
    man = {"sha256": "x", "sources": base}
    lib = tmp_path / "lib.so"
    lib.write_bytes(b"abc")
    monkeypatch.setattr(_build, "LIB", lib)
    man["sha256"] = _build.library_digest(lib)
    assert _build.verify(man) is None
    assert "sources changed" in _build.verify(dict(man, sources=edited))
    assert "library bytes" in _build.verify(dict(man, sha256="0" * 64))


def test_root_digest_binds_the_rows(tmp_path):
    reg = _row()
    p = tmp_path / "r.json"
    p.write_text(json.dumps(reg))
    assert R.load_registry(p)["artifacts"]
    reg["artifacts"][0]["family"] = "gpt2"
    p.write_text(json.dumps(reg))
    with pytest.raises(ValueError):
        R.load_registry(p)


def test_committed_rows_cover_the_stand_ins():
    from toktier_amd import standin
    if not R.REGISTRY_PATH.exists():
        pytest.skip("no registry rows committed yet")
    reg = R.load_registry()
    shas = {a["family"]: a["artifact_sha256"] for a in reg["artifacts"]}
    assert shas == dict(standin.ARTIFACT_SHA256)
    for a in reg["artifacts"]:
        row = a["backends"]["gpu"]["deliveries"]["prebuilt"]
        assert row["status"] in (R.STATUS_CERTIFIED, R.STATUS_EXPERIMENTAL)
        assert "gfx950" in R.architecture_statuses(row)
        assert len(row["binary_digest"]) == 64


def test_committed_soak_covers_every_family():
    """The committed soak reading (tests/test_gpu_soak.py at
    TK_SOAK_CHARS=100000000 on gfx950): at least 100 M characters per
    family, every row equal to the oracle's."""
    from conftest import FAMILY_NAMES
    path = R.REGISTRY_PATH.with_name("gfx950_soak.v1.json")
    soak = json.loads(path.read_text(encoding="utf-8"))
    assert soak["mismatches"] == 0
    for name in FAMILY_NAMES:
        rec = soak["families"][name]
        assert rec["chars"] >= 100_000_000, name
        assert rec["mismatch"] is None, name
        assert rec["documents"] > 10_000 and rec["long_documents"] > 1_000, name
