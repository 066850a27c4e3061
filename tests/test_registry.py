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


def test_generate_certifies_only_a_judged_build():
    man = {"build_key": KEY, "hipcc": ["HIP version: 7.2"], "flags": ["-O3"]}
    ok = {"evidence_id": "ev1", "build_key": KEY, "architecture": "gfx950",
          "passed": 40, "failed": 0, "skipped": 0, "driver_version": 70226015}
    reg = R.generate(ok, man, {"qwen3_8b": SHA})
    row = reg["artifacts"][0]["backends"]["gpu"]["deliveries"]["prebuilt"]
    assert row["status"] == R.STATUS_CERTIFIED and row["devices"] == ["gfx950"]
    assert R.architecture_statuses(row) == {"gfx950": R.STATUS_CERTIFIED}
    assert R.admit(reg, SHA, _facts(), R.POLICY_CERTIFIED).admitted
    for bad in (dict(failed=1), dict(build_key="b" * 64),
                dict(architecture="gfx942"), dict(passed=0)):
        reg = R.generate({**ok, **bad}, man, {"qwen3_8b": SHA})
        row = reg["artifacts"][0]["backends"]["gpu"]["deliveries"]["prebuilt"]
        assert row["status"] == R.STATUS_EXPERIMENTAL, bad
        assert R.architecture_statuses(row) == {"gfx950": R.STATUS_EXPERIMENTAL}
        assert not R.admit(reg, SHA, _facts(), R.POLICY_CERTIFIED).admitted


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
